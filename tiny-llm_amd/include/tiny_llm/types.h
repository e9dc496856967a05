// Configuration and weight-descriptor types of tiny-llm, for the HIP build.
//
// This header stands in for the reference's include/tiny_llm/types.h when
// this library's include directory comes first on the include path: it
// declares every type that header declares, with the same names, members and
// defaults, so the reference's other headers (transformer.h, validator.h,
// inference_engine.h, model_loader.h) keep compiling against it.  The one
// difference is the fp16 type: `half` from <hip/hip_fp16.h> instead of
// <cuda_fp16.h>.  GenerationConfig::validate() stays defined by the
// reference's src/types.cpp; this library neither defines nor calls it.
#pragma once

#include "tiny_llm/result.h"

#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace tiny_llm {

// Model hyper-parameters (types.h:12-26); num_kv_heads < num_heads is GQA.
struct ModelConfig {
    int   vocab_size = 32000;
    int   hidden_dim = 4096;
    int   num_layers = 32;
    int   num_heads = 32;
    int   num_kv_heads = 32;
    int   head_dim = 128;
    int   intermediate_dim = 11008;
    int   max_seq_len = 2048;
    float rope_theta = 10000.0f;
    float rms_norm_eps = 1e-5f;
    int   eos_token_id = 2;
    int   bos_token_id = 1;
};

// W8A16 quantisation parameters (types.h:29-32).
struct QuantizationParams {
    int  group_size = 128;
    bool symmetric = true;
};

// One int8 weight matrix [rows][cols] with fp16 group scales
// [ceil(rows / group_size)][cols] (types.h:35-58).
struct QuantizedWeight {
    int8_t *data = nullptr;
    half   *scales = nullptr;
    int     rows = 0;
    int     cols = 0;
    int     group_size = 128;

    int    scaleRows() const { return (rows + group_size - 1) / group_size; }
    int    scaleCols() const { return cols; }
    size_t weightElements() const { return static_cast<size_t>(rows) * cols; }
    size_t scaleElements() const { return static_cast<size_t>(scaleRows()) * scaleCols(); }
    size_t weightBytes() const { return weightElements() * sizeof(int8_t); }
    size_t scaleBytes() const { return scaleElements() * sizeof(half); }
    size_t totalBytes() const { return weightBytes() + scaleBytes(); }
    bool   isValid() const {
        return data != nullptr && scales != nullptr && rows > 0 && cols > 0 && group_size > 0;
    }
};

// Weights of one decoder layer (types.h:61-76): attention projections, the
// SwiGLU FFN and the two RMSNorm weight vectors.
struct TransformerWeights {
    QuantizedWeight wq;
    QuantizedWeight wk;
    QuantizedWeight wv;
    QuantizedWeight wo;
    QuantizedWeight w1;
    QuantizedWeight w2;
    QuantizedWeight w3;
    half           *rms_att_weight = nullptr;
    half           *rms_ffn_weight = nullptr;
};

// Whole-model weights (types.h:79-89).
struct ModelWeights {
    half                           *token_embedding = nullptr;
    std::vector<TransformerWeights> layers;
    half                           *final_norm_weight = nullptr;
    QuantizedWeight                 lm_head;
};

class Validator;

// Sampling and length limits of generate() (types.h:95-109).
struct GenerationConfig {
    int   max_new_tokens = 256;
    float temperature = 1.0f;
    int   top_k = 50;
    float top_p = 0.9f;
    bool  do_sample = false;
    float repetition_penalty = 1.0f;

    Result<void> validate() const;
};

// Timings and counts of one generate() call (types.h:112-119).
struct GenerationStats {
    float  prefill_time_ms = 0.0f;
    float  decode_time_ms = 0.0f;
    int    prompt_tokens = 0;
    int    tokens_generated = 0;
    float  tokens_per_second = 0.0f;
    size_t peak_memory_bytes = 0;
};

// KV cache geometry (types.h:122-128).  num_heads is the number of KV heads
// (InferenceEngine sets it from num_kv_heads, src/inference_engine.cpp:59).
struct KVCacheConfig {
    int num_layers = 32;
    int num_heads = 32;
    int head_dim = 128;
    int max_seq_len = 2048;
    int max_batch_size = 1;
};

} // namespace tiny_llm
