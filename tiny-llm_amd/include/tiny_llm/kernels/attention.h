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

// Prefill attention (kernels/attention.cuh:20-26): Q, K, V, O [batch,
// num_heads, seq_len, head_dim], causal (query i attends to keys 0..i), the
// reference's softmax with 1/(sum+1e-6), fp32 accumulation on MFMA.  Silent
// return on non-positive dimensions (attention.cu:228-230); no shared-memory
// limit on seq_len.  head_dim in {32, 64, 128, 256}, else a logged error.
void attention_prefill(const half *__restrict__ query, const half *__restrict__ key,
                       const half *__restrict__ value, half *__restrict__ output, float scale,
                       int batch_size, int num_heads, int seq_len, int head_dim,
                       hipStream_t stream = 0);

// Row softmax (kernels/attention.cuh:28-30, attention.cu:288-354):
// [batch_size][seq_len] fp16 in and out.
void softmax(const half *__restrict__ input, half *__restrict__ output, int batch_size, int seq_len,
             hipStream_t stream = 0);

// Scaled scores fp16(scale * q.k) [batch, num_heads, query_len, key_len],
// zero above the diagonal when apply_causal_mask (kernels/attention.cuh:
// 32-36, attention.cu:240-286); no softmax is applied.
void get_attention_weights(const half *__restrict__ query, const half *__restrict__ key,
                           half *__restrict__ weights, float scale, int batch_size, int num_heads,
                           int query_len, int key_len, int head_dim, bool apply_causal_mask,
                           hipStream_t stream = 0);

} // namespace kernels
} // namespace tiny_llm
