// W8A16 GEMM with fused epilogues (kernels/w8a16_gemm.hip).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace tiny_llm {
namespace detail {

constexpr int kMaxSegs = 3;
enum : int { kEpiDense = 0, kEpiResidual = 1, kEpiCache = 2 };

// One weight matrix of a launch and where its output columns go.
struct W8A16Seg {
    const int8_t *w = nullptr;   // [K][n] int8, row-major
    const __half *s = nullptr;   // [ceil(K/gs)][n] fp16 scales
    int           n = 0;         // columns
    int           kind = kEpiDense;
    __half       *out = nullptr; // dense/residual: [M][ld]; cache: layer K or V base
    int64_t       ld = 0;        // dense/residual row pitch (elements)
    const __half *res = nullptr; // residual: same layout as out (may alias out)
};

// Destination rows of the cache epilogue: entry m's token row at write
// position wpos[m] of cache row seq_row[m] (block-table addressing when
// block_table is set; see KvView).
struct CacheRows {
    const int32_t *seq_row = nullptr;
    const int32_t *wpos = nullptr;
    const int32_t *block_table = nullptr;
    int            bt_stride = 0;
    int            log2_blk = 30;
    int64_t        blk_stride = 0;
    int64_t        tok_stride = 0;
};

// True when the MFMA path covers the shape (K % 32 == 0, gs a power of two in
// [32, 512], every
// segment's n % 16 == 0); other shapes take the reference-order kernel.
bool w8a16_mfma_ok(int K, int gs, const W8A16Seg *segs, int nseg);

// fp32 workspace (elements) that launch_w8a16 needs for split-K partials,
// the only source of that size.  It is 0 where w8a16_dec_kernel takes the
// shape -- M <= 64, K a multiple of 128 and at most 4096, every segment's
// n * K below 2^31 -- because that kernel runs over the whole of K; other
// MFMA shapes (e.g. M <= 64 with K = 14336) take the split-K pair and need it.
size_t w8a16_workspace_floats(int M, int K, int gs, const W8A16Seg *segs, int nseg);

// out = x @ dequant(W_i, s_i) for each segment i, with its epilogue.  x [M][K]
// fp16 at row pitch ldx; all pointers device; 16-byte alignment of x, W and
// the row pitches (x: ldx % 8 == 0) is the caller's check.
// packed: every segment's w is in the layout of launch_w8a16_pack (MFMA
// path only; shapes it does not cover are rejected).
void launch_w8a16(const __half *x, int64_t ldx, int M, int K, int gs, const W8A16Seg *segs, int nseg,
                  const CacheRows *cache, float *workspace, hipStream_t stream, bool packed = false);

// W [K][N] int8 -> the MFMA-fragment layout (K % 32 == 0, N % 16 == 0; K*N
// bytes): fragment (column block nb, k step ks) holds, for lane l, rows
// 32ks + 8(l/16) .. +7 of column 16nb + l%16 as 8 contiguous bytes.
void launch_w8a16_pack(const int8_t *w, int K, int N, int8_t *out, hipStream_t stream);

// 1: every launch takes the reference-order kernel; 0 / -1: normal selection.
void w8a16_force_generic(int on);

} // namespace detail
} // namespace tiny_llm
