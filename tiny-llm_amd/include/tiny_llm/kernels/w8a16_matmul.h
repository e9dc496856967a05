// W8A16 matrix multiplication (replaces kernels/w8a16_matmul.cuh:22-26).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace tiny_llm {
namespace kernels {

// output[M][N] = input[M][K] @ dequant(weight[K][N] int8, scales[ceil(K/gs)][N])
// with fp32 accumulation and fp16 output, like the reference; silently
// returns when a dimension or group_size is not positive.  MFMA path when
// K % 32 == 0, group_size in {32, 64, 128, 256, 512}, N % 16 == 0 and the pointers are 16-byte
// aligned, else a kernel that follows the reference's per-element formula.
void w8a16_matmul(const half *input, const int8_t *weight, const half *scales, half *output, int M,
                  int N, int K, int group_size, hipStream_t stream = 0);

// The o_proj + residual step of TransformerLayer::forward
// (src/transformer.cpp:149-151, 246-247): hidden[M][N] = fp16(f(hidden) +
// f(fp16(input @ dequant(weight, scales)))), i.e. w8a16_matmul into a
// temporary followed by add_inplace (kernels/elementwise.cu:7-14), in one
// launch.
// packed: weight is in the layout of w8a16_pack (faster: no transpose in
// the kernel; needs K % 32 == 0, N % 16 == 0, group_size in {32..512}).
void w8a16_matmul_residual(const half *input, const int8_t *weight, const half *scales, half *hidden,
                           int M, int N, int K, int group_size, hipStream_t stream = 0,
                           bool packed = false);

// One-time repack of weight [K][N] int8 (K % 32 == 0, N % 16 == 0) into the
// MFMA-fragment layout the packed entry points read (K*N bytes, device to
// device): the B fragments of 16 columns x 32 rows, 8 bytes per lane, two k
// steps' fragments interleaved in 1024 contiguous bytes (16 per lane), as
// offset-binary bytes (w ^ 0x80).
void w8a16_pack(const int8_t *weight, int K, int N, int8_t *packed, hipStream_t stream = 0);

} // namespace kernels
} // namespace tiny_llm
