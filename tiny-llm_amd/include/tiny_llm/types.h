// Configuration structs of the KV-cache path.
#pragma once

namespace tiny_llm {

// KV cache geometry; field order, names and defaults as in the reference
// (include/tiny_llm/types.h:122-128).  num_heads is the number of KV heads
// (InferenceEngine sets it from num_kv_heads, src/inference_engine.cpp:59).
struct KVCacheConfig {
    int num_layers = 32;
    int num_heads = 32;
    int head_dim = 128;
    int max_seq_len = 2048;
    int max_batch_size = 1;
};

} // namespace tiny_llm
