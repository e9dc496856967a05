// W8A16 GEMM for gfx950 with fused epilogues: out = x @ dequant(W, scales),
// the arithmetic of kernels/w8a16_matmul.cu (reference kernel :71-98, tiled
// kernel :119-217): out[m][n] = fp16(sum_k f(x[m][k]) * (w[k][n] * s[k/gs][n]))
// with an fp32 accumulator, W [K][N] int8 row-major, scales
// [ceil(K/gs)][N] fp16.
//
// MFMA path (K % 32 == 0, gs in {32, 64, 128, 256, 512}, every segment's
// N % 16 == 0).  It splits K across workgroups for decode-sized M (the split
// count depends on (M, K) only, so an output element's value does not depend
// on which other weight matrices share the launch) and sums the splits in a
// fixed order, so results are deterministic.
//
// One kernel, w8a16_sk_kernel, for both weight layouts: one workgroup = 4
// waves = a 64x64 output tile over one split; wave w takes every fourth group
// of 4 k steps for the whole tile (16 MFMAs per step: 4 row blocks x 4
// column blocks of v_mfma_f32_16x16x32_f16 on the integer weights, converted
// to fp16 exactly; each scale group's product folded into the fp32
// accumulator with its scale).  x is staged two k steps at a time in the
// wave's own LDS by the LDS DMA load (coalesced rows).  W:
//   packed (layout of launch_w8a16_pack): B fragments, 8 bytes per lane,
//     loaded straight into registers;
//   reference ([K][N] row-major): two k steps of the tile's 64 columns staged
//     in LDS by the DMA load and read as B fragments by the transposing
//     ds_read_b64_tr_b8.
// Both layouts give the same fragments and the same summation order, hence
// the same bits.  No barrier until the waves' tiles are summed through LDS.
//
// With one split the GEMM kernel applies the epilogue directly; otherwise it
// writes fp32 partials and w8a16_reduce_kernel sums the splits in split order
// and applies the epilogue.
//
// Generic path (any shape): one thread per output, the reference formula
// sum = fma(x, w * s, sum) over k in order.
//
// Epilogues (per segment of output columns):
//   dense     out[m*ld + n] = fp16(acc)
//   residual  out[m*ld + n] = fp16(f(res[m*ld + n]) + f(fp16(acc)))   (the
//             o_proj output rounded to fp16, then add_inplace of
//             kernels/elementwise.cu:7-14 into the residual stream)
//   cache     the K or V row of entry m at its write position in the KV
//             cache (what appendKV(seq, layer, row, 1) copies there).
#include "kv_kernels.h"
#include "w8a16.h"

#include "tiny_llm/hip_utils.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

namespace tiny_llm {
namespace detail {

namespace {

constexpr int kBM = 64;       // rows per workgroup
constexpr int kBN = 64;       // columns per workgroup
constexpr int kBK = 64;       // k rows per chunk (split sizes count chunks)
constexpr int kRing = 8;      // chunks per 512-row batch
constexpr int kMaxSplits = 8; // K splits of the split-K plan, at most
constexpr int kWaitVm0 = 0x0F70;   // s_waitcnt vmcnt(0)
constexpr int kWaitLgkm0 = 0xC07F; // s_waitcnt lgkmcnt(0)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef int      v2i32 __attribute__((ext_vector_type(2)));

struct GemmArgs {
    const __half *x; // [M][K]
    int64_t       ldx;
    int           M, K, gs;
    int           nseg;
    int           splits;
    int           chunks_per_split; // 64-row chunks of K per split
    int           tiles;            // column tiles over all segments
    int           mtiles;           // row tiles
    float        *partial;          // [splits][M][ntot] when splits > 1
    int           ntot;
    W8A16Seg      seg[kMaxSegs];
    int           col0[kMaxSegs + 1]; // first global column of each segment
    CacheRows     cache;
};

__device__ __forceinline__ float h2f(__half h) { return __half2float(h); }

// Epilogue for output (m, global column c) with value v (fp32 accumulator).
__device__ __forceinline__ void epilogue(const GemmArgs &a, int si, int m, int n, float v) {
    const W8A16Seg &sg = a.seg[si];
    const __half    o = __float2half(v);
    if (sg.kind == kEpiDense) {
        sg.out[(int64_t)m * sg.ld + n] = o;
    } else if (sg.kind == kEpiResidual) {
        const int64_t i = (int64_t)m * sg.ld + n;
        sg.out[i] = __float2half(h2f(sg.res[i]) + h2f(o));
    } else { // cache row of entry m
        const CacheRows &c = a.cache;
        const int        row = c.seq_row[m];
        const int        t = c.wpos[m];
        int64_t          off;
        if (c.block_table) {
            const int blk = c.block_table[(int64_t)row * c.bt_stride + (t >> c.log2_blk)];
            off = (int64_t)blk * c.blk_stride + (int64_t)(t & ((1 << c.log2_blk) - 1)) * c.tok_stride;
        } else {
            off = (int64_t)row * c.blk_stride + (int64_t)t * c.tok_stride;
        }
        sg.out[off + n] = o;
    }
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Four signed bytes -> four fp16 (exact), as two dwords of an MFMA operand.
// u = b + 128 (b ^ 0x80) placed in the mantissa of 0x6400 (1024.0) is the
// fp16 value 1024 + u; subtracting 1152 leaves b exactly.
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t v) {
    const uint32_t u = v ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u); // [u0 64 u1 64]
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x05030402u); // [u2 64 u3 64]
    const f16x2    bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    return make_uint2(__builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, lo) + bias),
                      __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, hi) + bias));
}

// Split-K inside the workgroup: one workgroup (4 waves) per unit (64-row
// tile, 64-column tile, K split); wave w takes k steps 4w..4w+3 of every
// 16-step (512-row) batch of the split for the whole 64x64 tile, x through
// the wave's LDS stage, W straight from global memory (PACKED: 8 bytes per
// lane per fragment) or through a second LDS stage (reference layout), 16
// MFMAs per step.  Scale groups are folded in step order.  The four
// waves' tiles are summed through LDS in wave order, wave w finishing row
// block w (each wave passes on the three row blocks it does not finish: 48
// KB of LDS, three workgroups per CU).  ACC: a second accumulator for
// several scale groups per wave (group size < 128, or more than one batch);
// without it the wave's result is P * s.
template <int GS, bool ACC, bool PACKED>
__global__ __launch_bounds__(256, ACC ? 2 : 3) void w8a16_sk_kernel(GemmArgs a) {
    static_assert(GS % 32 == 0 && 512 % GS == 0, "group size");
    constexpr int SPG = GS / 32;
    constexpr int BS = 16;
    constexpr int NS = SPG >= 4 ? 1 : 4 / SPG; // scale groups per wave and batch
    static_assert(ACC || NS == 1, "several groups per wave need the accumulator");
    __shared__ __align__(16) float red[4 * 3 * 4 * 64 * 4]; // [src wave][rb != src][cb][lane][4]
    const int     lane = threadIdx.x & 63;
    const int     wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int     unit = blockIdx.x;
    const int     split = unit % a.splits;
    const int     rest = unit / a.splits;
    int           tile = rest % a.tiles;
    const int     mt = rest / a.tiles;
    if (mt >= a.mtiles) return;
    int si = 0;
    while (si + 1 < a.nseg && tile >= (a.seg[si].n + kBN - 1) / kBN) {
        tile -= (a.seg[si].n + kBN - 1) / kBN;
        ++si;
    }
    const W8A16Seg &sg = a.seg[si];
    const int       c0 = tile * kBN;
    const int       nblk = sg.n >> 4;
    const int       ksteps = a.K >> 5;
    const int       s_begin = split * 2 * a.chunks_per_split;
    const int       s_end = min(ksteps, s_begin + 2 * a.chunks_per_split);
    const int       ngroups = (a.K + GS - 1) / GS;
    const int       m0 = mt * kBM;

    const int8_t *wp[4]; // packed: uniform column-block bases; lanes add 8 * lane (+ 512 per step)
    const __half *sp[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int nb = min((c0 >> 4) + cb, nblk - 1);
        wp[cb] = sg.w + (int64_t)nb * ksteps * 512;
        sp[cb] = sg.s + 16 * nb;
    }
    // Reference layout (W [K][N] row-major): the wave stages the 64 rows x
    // 64 columns of two k steps (4 KB, rows of 64 bytes) with the LDS DMA
    // load, 16-byte piece p of row r in slot p ^ ((r >> 1) & 3), and reads each
    // B fragment with ds_read_b64_tr_b8: lane c of a 16-lane group names 8
    // bytes of row 8q + c/2 (q the group), columns 16cb + 8(c % 2); lane i then
    // holds column 16cb + i of rows 8q .. 8q+7 -- the packed fragment's bytes.
    uint8_t *const ws = reinterpret_cast<uint8_t *>(red) + 32768 + wave * 4096;
    auto issue_w = [&](int st0) __attribute__((always_inline)) { // steps st0, st0 + 1
        if constexpr (!PACKED) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int      r = 16 * u + (lane >> 2);                 // row of the stage
                const int      pc = (lane & 3) ^ ((r >> 1) & 3);         // piece the slot holds
                const int      k = min(32 * st0 + r, a.K - 1);
                const int      col = min(c0 + 16 * pc, sg.n - 16);
                const int8_t  *src = sg.w + (int64_t)k * sg.n + col;
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                                 (__attribute__((address_space(3))) void *)(ws + u * 1024), 16, 0,
                                                 0);
            }
        }
    };
    auto read_w = [&](int s, uint2(&dst)[4]) __attribute__((always_inline)) { // step s of the stage
        const int i = lane & 15, r = 32 * s + 8 * (lane >> 4) + (i >> 1);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const v2i32 t = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (__attribute__((address_space(3))) v2i32 *)(ws + r * 64 + 16 * (cb ^ ((r >> 1) & 3)) + 8 * (i & 1)));
            dst[cb] = make_uint2((uint32_t)t[0], (uint32_t)t[1]);
        }
    };
    // x reaches the MFMA through LDS: a wave stages two k steps of its 64 rows
    // (128 bytes per row, 8 KB) with the LDS DMA load, whole 128-byte row
    // pieces per 8 lanes, so that a load instruction touches 8 cache lines
    // (the A-layout load straight from global memory touches 64: 16 rows per
    // 16 lanes).  Row r's 16-byte chunk c sits in slot c ^ f(r) of the row,
    // f(r) = (r & 7) ^ ((r >> 3) & 1), so that the fragment reads (16 rows,
    // one chunk) fall on distinct banks.  The stage lives in `red`, which the
    // waves use for the cross-wave sum only after the main loop.
    uint16_t *const xs = reinterpret_cast<uint16_t *>(red) + wave * 4096;
    const __half   *xt = a.x + (int64_t)m0 * a.ldx; // the row tile (32-bit offsets below)
    auto issue_x = [&](int st0) __attribute__((always_inline)) { // steps st0, st0 + 1
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int      c = (lane & 7) ^ (lane >> 3) ^ (u & 1);
            const int      st = min(st0 + (c >> 2), ksteps - 1);
            const int      row = min(8 * u + (lane >> 3), a.M - 1 - m0);
            const uint32_t off = (uint32_t)row * (uint32_t)a.ldx + (uint32_t)(32 * st + 8 * (c & 3));
            const __half  *src = xt + off;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                             (__attribute__((address_space(3))) void *)(xs + u * 512), 16, 0, 0);
        }
    };
    auto read_x = [&](int s, f16x8(&dst)[4]) __attribute__((always_inline)) { // step s of the stage
        const int c = 4 * s + (lane >> 4);
        const int p = c ^ (lane & 7) ^ ((lane >> 3) & 1);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
            dst[rb] = *reinterpret_cast<const f16x8 *>(xs + (2 * rb + ((lane & 15) >> 3)) * 512 + (lane & 7) * 64 + 8 * p);
    };

    f32x4 P[4][4], acc[4][4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            P[rb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            acc[rb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    float s_last[4] = {0.0f, 0.0f, 0.0f, 0.0f}; // scale of the wave's last group (no ACC)

    for (int sb = s_begin; sb < s_end; sb += BS) {
        const int first = sb + 4 * wave; // this wave's 4 steps
        const int nsteps = max(0, min(4, s_end - first));
        if (nsteps == 0) continue;
        issue_x(first); // x first (L2 hits), then W (HBM)
        uint2 wv[4][4];
        if constexpr (PACKED) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int st = min(first + j, ksteps - 1);
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
                    wv[j][cb] = *reinterpret_cast<const uint2 *>(wp[cb] + (uint32_t)(st * 512 + 8 * lane));
            }
        } else {
            issue_w(first);
        }
        uint16_t sraw[NS][4];
#pragma unroll
        for (int g = 0; g < NS; ++g)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
                sraw[g][cb] = *reinterpret_cast<const uint16_t *>(
                    sp[cb] + (uint32_t)(min((first + g * SPG) * 32 / GS, ngroups - 1) * sg.n + (lane & 15)));
        f16x8 xv[2][4];
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        read_x(0, xv[0]);
        read_x(1, xv[1]);
        if constexpr (!PACKED) {
            read_w(0, wv[0]);
            read_w(1, wv[1]);
        }
        if (nsteps > 2) { // the stages' reads complete before the DMA refills them
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            issue_x(first + 2);
            issue_w(first + 2);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j >= nsteps) continue; // uniform
            if (j == 2) {
                __builtin_amdgcn_s_waitcnt(kWaitVm0);
                read_x(0, xv[0]);
                read_x(1, xv[1]);
                if constexpr (!PACKED) {
                    read_w(0, wv[2]);
                    read_w(1, wv[3]);
                }
            }
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const uint2 lo = i8x4_to_f16x4(wv[j][cb].x), hi = i8x4_to_f16x4(wv[j][cb].y);
                const f16x8 bop = __builtin_bit_cast(f16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
                    P[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[j & 1][rb], bop, P[rb][cb], 0, 0, 0);
            }
            if constexpr (ACC) {
                if ((j + 1) % SPG == 0 || j + 1 == nsteps) { // end of a group or of the wave's steps
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        const float s_ = h2f(__builtin_bit_cast(__half, sraw[j / SPG % NS][cb]));
#pragma unroll
                        for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
                            for (int i = 0; i < 4; ++i) acc[rb][cb][i] = fmaf(P[rb][cb][i], s_, acc[rb][cb][i]);
                            P[rb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                        }
                    }
                }
            }
        }
        if constexpr (!ACC) {
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) s_last[cb] = h2f(__builtin_bit_cast(__half, sraw[0][cb]));
        }
        // the next batch's DMA refills the stage: its reads are complete
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    }
    // The wave's result r = acc, or P * s.
    if constexpr (!ACC) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[rb][cb][i] = P[rb][cb][i] * s_last[cb];
    }

    __builtin_amdgcn_s_waitcnt(kWaitVm0); // no DMA into the stage is still in flight
    __syncthreads();                      // every wave is done with its x stage in `red`
    // Pass on the three row blocks this wave does not finish.
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        if (rb == wave) continue;
        const int k = rb - (rb > wave);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
            *reinterpret_cast<f32x4 *>(&red[(((wave * 3 + k) * 4 + cb) * 64 + lane) * 4]) = acc[rb][cb];
    }
    __syncthreads();
    // Sum row block w over the waves in wave order.
    const int rb = wave;
    f32x4     v[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        v[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int src = 0; src < 4; ++src) {
            f32x4 u;
            if (src == wave) {
#pragma unroll
                for (int q = 0; q < 4; ++q) u = q == wave ? acc[q][cb] : u; // static indices
            } else {
                const int k = rb - (rb > src);
                u = *reinterpret_cast<const f32x4 *>(&red[(((src * 3 + k) * 4 + cb) * 64 + lane) * 4]);
            }
            if (src == 0) {
                v[cb] = u;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[cb][i] += u[i];
            }
        }
    }
    if (a.splits == 1) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            if (c0 + 16 * cb >= sg.n) continue; // uniform
            const int n = c0 + 16 * cb + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + 16 * rb + 4 * (lane >> 4) + i;
                if (m < a.M) epilogue(a, si, m, n, v[cb][i]);
            }
        }
        return;
    }
    // Partials: the row block is transposed through LDS (rows of 64 floats,
    // pitch 68) so that every lane stores 16 contiguous bytes and each group
    // of 16 lanes one row's 256 bytes.
    __syncthreads(); // every wave has read the passed-on blocks
    constexpr int TP = 68;
    float        *t = &red[wave * 16 * TP];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int i = 0; i < 4; ++i) t[(4 * (lane >> 4) + i) * TP + 16 * cb + (lane & 15)] = v[cb][i];
    const int cw = min(kBN, sg.n - c0); // live columns of the tile (a multiple of 16)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int   r = 4 * q + (lane >> 4);
        const int   c = 4 * (lane & 15);
        const int   m = m0 + 16 * rb + r;
        const f32x4 u = *reinterpret_cast<const f32x4 *>(&t[r * TP + c]);
        if (m < a.M && c < cw)
            *reinterpret_cast<f32x4 *>(&a.partial[((int64_t)split * a.M + m) * a.ntot + a.col0[si] + c0 + c]) = u;
    }
}

// Repacks W [K][N] int8 (K % 32 == 0, N % 16 == 0) so that the B fragment of
// v_mfma_f32_16x16x32_f16 for column block nb and k step ks is 512
// contiguous bytes: packed[((nb * K/32 + ks) * 64 + l) * 8 + j] =
// W[32 ks + 8 (l / 16) + j][16 nb + l % 16].  One thread per (nb, ks, l).
__global__ __launch_bounds__(256) void w8a16_pack_kernel(const int8_t *w, int K, int N, int8_t *out) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)(N / 16) * (K / 32) * 64;
    if (idx >= total) return;
    const int     l = (int)(idx & 63);
    const int64_t frag = idx >> 6;
    const int     ks = (int)(frag % (K / 32));
    const int     nb = (int)(frag / (K / 32));
    const int     col = 16 * nb + (l & 15);
    const int     k0 = 32 * ks + 8 * (l >> 4);
    uint32_t      lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        lo |= (uint32_t)(uint8_t)w[(int64_t)(k0 + j) * N + col] << (8 * j);
        hi |= (uint32_t)(uint8_t)w[(int64_t)(k0 + 4 + j) * N + col] << (8 * j);
    }
    *reinterpret_cast<uint2 *>(out + idx * 8) = make_uint2(lo, hi);
}

// The epilogue of four consecutive columns n..n+3 of one segment (n % 4 ==
// 0; every segment of the MFMA path has n % 16 == 0): one 8-byte store, and
// one cache-row lookup, per thread.
__device__ __forceinline__ void epilogue4(const GemmArgs &a, int si, int m, int n, const float4 &v) {
    const W8A16Seg &sg = a.seg[si];
    const __half2   lo = __floats2half2_rn(v.x, v.y), hi = __floats2half2_rn(v.z, v.w);
    __half         *dst;
    if (sg.kind == kEpiCache) {
        const CacheRows &c = a.cache;
        const int        row = c.seq_row[m];
        const int        t = c.wpos[m];
        int64_t          off;
        if (c.block_table) {
            const int blk = c.block_table[(int64_t)row * c.bt_stride + (t >> c.log2_blk)];
            off = (int64_t)blk * c.blk_stride + (int64_t)(t & ((1 << c.log2_blk) - 1)) * c.tok_stride;
        } else {
            off = (int64_t)row * c.blk_stride + (int64_t)t * c.tok_stride;
        }
        dst = sg.out + off + n;
    } else {
        dst = sg.out + (int64_t)m * sg.ld + n;
    }
    uint2 w = make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
    if (sg.kind == kEpiResidual) { // fp16(f(res) + f(fp16(acc))), element by element
        const uint2   r = *reinterpret_cast<const uint2 *>(sg.res + (int64_t)m * sg.ld + n);
        const __half2 rl = __builtin_bit_cast(__half2, r.x), rh = __builtin_bit_cast(__half2, r.y);
        const __half2 sl = __floats2half2_rn(__low2float(rl) + __low2float(lo), __high2float(rl) + __high2float(lo));
        const __half2 sh = __floats2half2_rn(__low2float(rh) + __low2float(hi), __high2float(rh) + __high2float(hi));
        w = make_uint2(__builtin_bit_cast(uint32_t, sl), __builtin_bit_cast(uint32_t, sh));
    }
    *reinterpret_cast<uint2 *>(dst) = w;
}

// Sums the split-K partials in split order and applies the epilogue, four
// consecutive columns per thread (16-byte partial loads).
__global__ __launch_bounds__(256) void w8a16_reduce_kernel(GemmArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int     q = a.ntot >> 2;
    if (idx >= (int64_t)a.M * q) return;
    const int m = (int)(idx / q);
    const int c = 4 * (int)(idx - (int64_t)m * q);
    int       si = 0;
    while (si + 1 < a.nseg && c >= a.col0[si + 1]) ++si;
    // Every split's load in flight at once (at most kMaxSplits; an index past
    // the last split re-reads it), then the sum in split order.
    float4 p[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s)
        p[s] = *reinterpret_cast<const float4 *>(a.partial + ((int64_t)min(s, a.splits - 1) * a.M + m) * a.ntot + c);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) { // a select, not a branch: the loads stay up front
        const bool live = s < a.splits;
        v.x = live ? v.x + p[s].x : v.x;
        v.y = live ? v.y + p[s].y : v.y;
        v.z = live ? v.z + p[s].z : v.z;
        v.w = live ? v.w + p[s].w : v.w;
    }
    epilogue4(a, si, m, c - a.col0[si], v);
}

// Reference-order fallback: one thread per (m, column), sequential k.
__global__ __launch_bounds__(256) void w8a16_generic_kernel(GemmArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)a.M * a.ntot) return;
    const int m = (int)(idx / a.ntot);
    const int c = (int)(idx - (int64_t)m * a.ntot);
    int       si = 0;
    while (si + 1 < a.nseg && c >= a.col0[si + 1]) ++si;
    const W8A16Seg &sg = a.seg[si];
    const int       n = c - a.col0[si];
    const __half   *xr = a.x + (int64_t)m * a.ldx;
    float           sum = 0.0f;
    for (int k = 0; k < a.K; ++k) {
        const float w = (float)sg.w[(int64_t)k * sg.n + n] * h2f(sg.s[(int64_t)(k / a.gs) * sg.n + n]);
        sum = fmaf(h2f(xr[k]), w, sum);
    }
    epilogue(a, si, m, n, sum);
}

int g_force_generic = -1;

} // namespace

bool w8a16_mfma_ok(int K, int gs, const W8A16Seg *segs, int nseg) {
    if (K % 32 != 0 || (gs != 32 && gs != 64 && gs != 128 && gs != 256 && gs != 512)) return false;
    for (int i = 0; i < nseg; ++i)
        if (segs[i].n % 16 != 0) return false;
    return true;
}

namespace {
// Split-K plan, a function of (M, K) only -- never of the columns sharing the
// launch -- so that every output element is summed in the same order whether
// its weight matrix is multiplied alone or fused with others (the fused
// projection's cache bytes equal the unfused path's).  Decode-sized M splits K
// into up to 8 ranges of >= 512 rows (at most kRing chunks each for K <= 4096,
// so a split's loads are all in flight together); larger M has enough row
// tiles.  Sets the 64-row chunks per split.
int split_plan(int M, int K, int *chunks_per_split) {
    const int kchunks = (K + kBK - 1) / kBK;
    int       splits = M <= 256 ? std::min(kMaxSplits, std::max(1, K / 512)) : 1;
    // chunks per split: a multiple of kRing, so that every batch starts on a
    // 512-row (scale-group) boundary
    const int cps = ((kchunks + splits - 1) / splits + kRing - 1) / kRing * kRing;
    if (chunks_per_split) *chunks_per_split = cps;
    return (kchunks + cps - 1) / cps;
}
} // namespace

size_t w8a16_workspace_floats(int M, int K, int gs, const W8A16Seg *segs, int nseg) {
    if (!w8a16_mfma_ok(K, gs, segs, nseg)) return 0;
    int ntot = 0;
    for (int i = 0; i < nseg; ++i) ntot += segs[i].n;
    const int splits = split_plan(M, K, nullptr);
    return splits > 1 ? (size_t)splits * M * ntot : 0;
}

void launch_w8a16(const __half *x, int64_t ldx, int M, int K, int gs, const W8A16Seg *segs, int nseg,
                  const CacheRows *cache, float *workspace, hipStream_t stream, bool packed) {
    if (nseg < 1 || nseg > kMaxSegs) throw std::invalid_argument("w8a16: 1..3 weight segments");
    GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = x;
    a.ldx = ldx;
    a.M = M;
    a.K = K;
    a.gs = gs;
    a.nseg = nseg;
    int tiles = 0;
    a.col0[0] = 0;
    for (int i = 0; i < nseg; ++i) {
        a.seg[i] = segs[i];
        a.col0[i + 1] = a.col0[i] + segs[i].n;
        tiles += (segs[i].n + kBN - 1) / kBN;
        if (segs[i].kind == kEpiCache && !cache)
            throw std::invalid_argument("w8a16: cache epilogue without cache rows");
    }
    a.ntot = a.col0[nseg];
    if (cache) a.cache = *cache;
    bool aligned = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && ldx % 8 == 0;
    for (int i = 0; i < nseg; ++i) aligned &= (reinterpret_cast<uintptr_t>(segs[i].w) & 15u) == 0;
    const bool mfma = packed || (g_force_generic != 1 && aligned && w8a16_mfma_ok(K, gs, segs, nseg));
    if (packed && !w8a16_mfma_ok(K, gs, segs, nseg))
        throw std::invalid_argument("w8a16: packed weights need K % 32 == 0, N % 16 == 0 and a "
                                    "group size in {32, 64, 128, 256, 512}");
    if (packed && !aligned) throw std::invalid_argument("w8a16: x and weights must be 16-byte aligned");
    if (!mfma) {
        a.splits = 1;
        const int64_t total = (int64_t)M * a.ntot;
        profile_begin(KernelId::W8A16, stream);
        hipLaunchKernelGGL(w8a16_generic_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           stream, a);
        HIP_CHECK(hipGetLastError());
        profile_end(KernelId::W8A16, stream);
        return;
    }
    const int mt = (M + kBM - 1) / kBM;
    const int splits = split_plan(M, K, &a.chunks_per_split);
    a.splits = splits;
    a.tiles = tiles;
    a.mtiles = mt;
    a.partial = splits > 1 ? workspace : nullptr;
    if (splits > 1 && !workspace) throw std::invalid_argument("w8a16: split-K needs a workspace");
    profile_begin(KernelId::W8A16, stream);
    {
        // Several scale groups per wave (gs < 128) or more than one 512-row
        // batch per split need the second accumulator.
        const bool     acc = gs < 128 || a.chunks_per_split > 8;
        const unsigned units = (unsigned)(splits * tiles * mt);
#define TL_W8_SK_LAUNCH(G, P)                                                                          \
    do {                                                                                               \
        if (acc)                                                                                       \
            hipLaunchKernelGGL((w8a16_sk_kernel<G, true, P>), dim3(units), dim3(256), 0, stream, a);   \
        else                                                                                           \
            hipLaunchKernelGGL((w8a16_sk_kernel<(G < 128 ? 128 : G), false, P>), dim3(units), dim3(256), 0, \
                               stream, a);                                                             \
    } while (0)
#define TL_W8_SK_GS(P)                          \
    switch (gs) {                               \
    case 32: TL_W8_SK_LAUNCH(32, P); break;     \
    case 64: TL_W8_SK_LAUNCH(64, P); break;     \
    case 128: TL_W8_SK_LAUNCH(128, P); break;   \
    case 256: TL_W8_SK_LAUNCH(256, P); break;   \
    default: TL_W8_SK_LAUNCH(512, P); break;    \
    }
        if (packed) {
            TL_W8_SK_GS(true)
        } else {
            TL_W8_SK_GS(false)
        }
#undef TL_W8_SK_GS
#undef TL_W8_SK_LAUNCH
    }
    HIP_CHECK(hipGetLastError());
    profile_end(KernelId::W8A16, stream);
    if (splits > 1) {
        const int64_t total = (int64_t)M * (a.ntot / 4);
        profile_begin(KernelId::W8A16Reduce, stream);
        hipLaunchKernelGGL(w8a16_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           stream, a);
        HIP_CHECK(hipGetLastError());
        profile_end(KernelId::W8A16Reduce, stream);
    }
}

void w8a16_force_generic(int on) { g_force_generic = on; }

void launch_w8a16_pack(const int8_t *w, int K, int N, int8_t *out, hipStream_t stream) {
    if (K % 32 != 0 || N % 16 != 0 || K <= 0 || N <= 0)
        throw std::invalid_argument("w8a16_pack: K must be a positive multiple of 32 and N of 16");
    const int64_t total = (int64_t)(N / 16) * (K / 32) * 64;
    hipLaunchKernelGGL(w8a16_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, w,
                       K, N, out);
    HIP_CHECK(hipGetLastError());
}

} // namespace detail
} // namespace tiny_llm
