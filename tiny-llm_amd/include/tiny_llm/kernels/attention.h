// Decode attention entry points (replaces kernels/attention.cuh:15-18).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

namespace tiny_llm {
namespace kernels {

// Q: [batch, num_heads, 1, head_dim], K/V: [batch, num_heads, seq_len,
// head_dim], O: [batch, num_heads, 1, head_dim]; fp16, fp32 accumulate.
// Same contract as the reference: silently returns when a dimension is not
// positive (attention.cu:117-119).  Unlike the reference, seq_len is not
// limited by shared memory (split-K over chunks of the sequence) and launch errors
// are reported through the logger instead of being dropped.
void attention_decode(const half *__restrict__ query, const half *__restrict__ k_cache,
                      const half *__restrict__ v_cache, half *__restrict__ output, float scale,
                      int batch_size, int num_heads, int seq_len, int head_dim,
                      hipStream_t stream = 0);

} // namespace kernels
} // namespace tiny_llm
