// W8A16 GEMM for gfx950 with fused epilogues: out = x @ dequant(W, scales),
// the arithmetic of kernels/w8a16_matmul.cu (reference kernel :71-98, tiled
// kernel :119-217): out[m][n] = fp16(sum_k f(x[m][k]) * (w[k][n] * s[k/gs][n]))
// with an fp32 accumulator, W [K][N] int8 row-major, scales
// [ceil(K/gs)][N] fp16.
//
// MFMA path (K % 32 == 0, gs in {32, 64, 128, 256, 512}, every segment's
// N % 16 == 0), two kernels, each for both weight layouts (packed: the
// launch_w8a16_pack layout, B fragments of 8 bytes per lane, two k steps per
// 16-byte lane load; reference:
// [K][N] row-major, staged in LDS and read as B fragments by the transposing
// ds_read_b64_tr_b8).  Both layouts give the same fragments and the same
// summation order, hence the same bits.  The int8 weights become fp16
// exactly and multiply on v_mfma_f32_16x16x32_f16; each scale group's
// product is folded into the fp32 accumulator with its scale.
//
//   w8a16_dec_kernel (M <= 64, K a multiple of 128 up to 4096: the decode
//     projections): one launch over the whole of K, no partials (described
//     at the kernel).
//   w8a16_sk_kernel (every other MFMA shape): one workgroup = 4 waves = a
//     64x64 output tile over one K split; wave w takes every fourth group of
//     4 k steps for the whole tile; x staged two k steps at a time in the
//     wave's own LDS by the LDS DMA load.  The split count depends on (M, K)
//     only.  With one split the kernel applies the epilogue; otherwise it
//     writes fp32 partials and w8a16_reduce_kernel sums the splits in split
//     order and applies it.
//
// The summation order of an output element depends on (M, K) only -- never
// on which other weight matrices share the launch -- so results are
// deterministic and the fused projection equals the unfused products.
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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

// Four offset-binary bytes u = b + 128 -> four fp16 b (exact), as two dwords
// of an MFMA operand: u placed in the mantissa of 0x6400 (1024.0) is the fp16
// value 1024 + u; subtracting 1152 leaves b exactly.
__device__ __forceinline__ uint2 u8x4_to_f16x4(uint32_t u) {
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u); // [u0 64 u1 64]
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x05030402u); // [u2 64 u3 64]
    const f16x2    bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    return make_uint2(__builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, lo) + bias),
                      __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, hi) + bias));
}

// Four bytes of W -> four fp16.  The packed layout holds offset-binary bytes
// (b ^ 0x80, written by w8a16_pack_kernel); the reference layout holds b.
template <bool PACKED> __device__ __forceinline__ uint2 w8x4_to_f16x4(uint32_t v) {
    return u8x4_to_f16x4(PACKED ? v : v ^ 0x80808080u);
}

// Byte offset, within its column block, of lane `lane`'s 8 bytes of k step st
// in the packed layout (see w8a16_pack_kernel): steps are stored in pairs,
// 16 bytes per lane (step 2p in the low 8), a last unpaired step (K % 64 ==
// 32) at 8 bytes per lane.
__device__ __forceinline__ uint32_t packed_step_offset(int st, int ksteps, int lane) {
    const uint32_t base = (uint32_t)(st >> 1) * 1024u;
    return st < (ksteps & ~1) ? base + 16u * lane + 8u * (st & 1) : base + 8u * lane;
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

    const int8_t *wp[4]; // packed: uniform column-block bases (+ packed_step_offset)
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
                    wv[j][cb] = *reinterpret_cast<const uint2 *>(wp[cb] + packed_step_offset(st, ksteps, lane));
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
                const uint2 lo = w8x4_to_f16x4<PACKED>(wv[j][cb].x), hi = w8x4_to_f16x4<PACKED>(wv[j][cb].y);
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

// ---------------------------------------------------------------------------
// Decode-sized M (<= 64 rows; K a multiple of 128 up to 4096):
// w8a16_dec_kernel, one launch over the whole of K (no split-K partials, no
// second kernel).
//
// A workgroup of 8 waves owns a tile of CB 16-column blocks (numbered over all
// segments, so a tile may span two segments) for one half of the rows (32
// rows, two MFMA row blocks).  K is cut into 128-row chunks (4 k steps); wave
// w takes chunks w, w + 8, w + 16, w + 24 through a two-deep register ring:
// x in whole 128-byte lines (4 rows x 256 bytes per load) and packed W
// fragments (16 bytes per lane: two k steps) load into registers, so the compiler's own
// load counters order each use after exactly the data it needs, and the next
// chunks' loads are in flight while one is multiplied.  (The LDS DMA load
// would not do: this compiler waits for every outstanding load before the
// first LDS read that follows one.)  x reaches the MFMA A layout through the
// wave's own LDS stage.  Reference-layout W ([K][N] row-major) is loaded as
// 16-byte row pieces, written to the wave's W stage and read back as B
// fragments with the transposing ds_read_b64_tr_b8 -- the same fragments as
// the packed layout.
// Each fold group's product (a chunk for gs >= 128, else gs / 32 steps) is
// folded into the fp32 accumulator with its scale; the 8 waves' tiles are
// summed through LDS in wave order and the epilogue is applied.
//
// The two row halves of a tile run on the same XCD (workgroups b and b + 8 of
// the round-robin dispatch) at the same time, so the second reads the tile's
// weights from that XCD's L2; each XCD takes a contiguous range of tiles.
// The summation order of an output depends on K alone (chunks, waves), never
// on the column tiling or the segments sharing the launch, so the fused
// projection's cache bytes equal the unfused product's, and both weight
// layouts give the same bits.
constexpr int kDecRows = 64;   // the kernel's M limit
constexpr int kDecMaxK = 4096; // and K limit (a multiple of 128): 4 chunks per wave
constexpr int kDecHalf = 32;   // rows per workgroup
constexpr int kDecWaves = 8;

struct DecArgs {
    const __half *x; // [M][K]
    int64_t       ldx;
    int           M, K, gs;
    int           log2_gs; // gs is a power of two
    int           nseg;
    int           tiles;  // column tiles of CB blocks
    int           tpx;    // tiles per XCD: ceil(tiles / 8)
    int           halves; // row halves (1 when M <= 32)
    int           blocks; // 16-column blocks over all segments
    W8A16Seg      seg[kMaxSegs];
    int           col0[kMaxSegs + 1];
    CacheRows     cache;
};

// Field f of segment si (uniform), with static indices only.
#define TL_DEC_SEG(a, si, f) ((si) == 0 ? (a).seg[0].f : (si) == 1 ? (a).seg[1].f : (a).seg[2].f)

// Segment of global 16-column block gb.
__device__ __forceinline__ int dec_seg_of(const DecArgs &a, int gb) {
    const int c = 16 * gb;
    return (a.nseg > 1 && c >= a.col0[1]) ? ((a.nseg > 2 && c >= a.col0[2]) ? 2 : 1) : 0;
}

// Rotation of the reference-layout LDS stage: piece p of stage row r sits in
// slot (p + dec_rot(r)) % CB of the row, so that the 8 rows a
// ds_read_b64_tr_b8 group reads fall on distinct 16-byte bank slots (odd
// widths need none: rows 16 * CB bytes apart already do).
template <int CB> __device__ __forceinline__ int dec_rot(int r) {
    return CB == 2 ? (r >> 2) : CB == 4 ? (r >> 1) : 0;
}

// Buffer resource of a raw byte range (stride 0, the gfx9 data format word).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dec_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// FS: k steps per scale fold (gs / 32, at most 4 = one chunk).  CB: column
// blocks per tile.  PACKED: W in the launch_w8a16_pack layout.
template <int FS, int CB, bool PACKED>
__global__ __launch_bounds__(512, 1) void w8a16_dec_kernel(DecArgs a) {
    static_assert(FS == 1 || FS == 2 || FS == 4, "fold");
    static_assert(CB >= 1 && CB <= 4, "column blocks");
    constexpr int NF = 4 / FS;                                  // folds per chunk
    constexpr int RED = kDecWaves * 2 * CB * 64 * 4;            // floats: every wave's tile
    constexpr int XPITCH = 256 + 32;                            // bytes: an x stage row (padded)
    constexpr int XST = kDecHalf * XPITCH;                      // bytes: a wave's x stage (one chunk)
    constexpr int WST = PACKED ? 0 : 128 * CB * 16;             // bytes: its W stage (reference layout)
    constexpr int STAGE = kDecWaves * (XST + WST) / 4;          // floats
    __shared__ __align__(16) float lds[RED > STAGE ? RED : STAGE];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Workgroup b runs on XCD b % 8 (round-robin dispatch).  XCD x takes the
    // contiguous tiles [x * tpx, (x + 1) * tpx), both row halves of a tile
    // (workgroups b and b + 8): the halves share the tile's weights, and
    // column-adjacent tiles the 128-byte lines of row-major weights, in that
    // XCD's L2.  (Another placement costs speed, never correctness.)
    const int slot = blockIdx.x >> 3;
    const int half = a.halves == 2 ? (slot & 1) : 0;
    const int tile = (int)(blockIdx.x & 7) * a.tpx + (a.halves == 2 ? slot >> 1 : slot);
    if (tile >= a.tiles) return; // uniform for the workgroup
    const int ksteps = a.K >> 5;
    const int nchunks = (ksteps + 3) >> 2;
    const int ngroups = (a.K + a.gs - 1) >> a.log2_gs;
    const int mine = wave < nchunks ? (nchunks - wave + kDecWaves - 1) / kDecWaves : 0; // this wave's chunks

    // The tile's column blocks: segment, local block, and the buffer
    // resources of their weights and scales (uniform: the loads take the
    // chunk and group offsets in scalar registers and a lane offset fixed for
    // the whole kernel, so they cost no vector address arithmetic).
    int                    si[CB], nb[CB], sn[CB];
    const int8_t          *wb[CB]; // reference layout: column base
    __amdgpu_buffer_rsrc_t rw[CB], rs[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int gb = min(tile * CB + cb, a.blocks - 1);
        si[cb] = dec_seg_of(a, gb);
        nb[cb] = gb - ((si[cb] == 0 ? 0 : si[cb] == 1 ? a.col0[1] : a.col0[2]) >> 4);
        sn[cb] = TL_DEC_SEG(a, si[cb], n);
        wb[cb] = TL_DEC_SEG(a, si[cb], w) + (int64_t)16 * nb[cb];
        rw[cb] = dec_rsrc(TL_DEC_SEG(a, si[cb], w), (uint32_t)sn[cb] * (uint32_t)a.K);
        rs[cb] = dec_rsrc(TL_DEC_SEG(a, si[cb], s), (uint32_t)ngroups * (uint32_t)sn[cb] * 2u);
    }
    const uint32_t sv = 2u * (lane & 15); // scale lane offset (+ 32 nb)
    // This wave's output block (waves < 2 CB): row block wave & 1, column
    // block wave >> 1.  Its epilogue operands -- the cache rows and write
    // positions, or the residual -- are loaded now, so that the stores at the
    // end do not wait a round trip for them.
    const int erb = wave & 1, ecb = wave >> 1;
    int       esi = 0, en = 0;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) // static indices
        if (cb == ecb) {
            esi = si[cb];
            en = 16 * nb[cb] + (lane & 15);
        }
    const bool eact = wave < 2 * CB && tile * CB + ecb < a.blocks; // (a block past the last segment: none)
    const int  ekind = TL_DEC_SEG(a, esi, kind);
    // These loads go out before the weight stream, so nothing may wait for
    // them here.  Rows and write positions are never negative: held
    // unsigned, their widening to 64 bits is a zero high word (a
    // sign-extending load is lowered to the load and a shift right after
    // it, a wait per row).  The kind test is outside the row loop, so each
    // path is a straight run of loads (a test per row let one path's zero
    // overwrite a register another path still had a load in flight for,
    // which needs a wait).
    uint32_t erow[4] = {0, 0, 0, 0}, epos[4] = {0, 0, 0, 0};
    __half   eres[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) eres[i] = __float2half(0.0f);
    int em[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) em[i] = min(kDecHalf * half + 16 * erb + 4 * (lane >> 4) + i, a.M - 1);
    if (eact && ekind == kEpiCache) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            erow[i] = (uint32_t)a.cache.seq_row[em[i]];
            epos[i] = (uint32_t)a.cache.wpos[em[i]];
        }
    } else if (eact && ekind == kEpiResidual) {
        const __half *res = TL_DEC_SEG(a, esi, res);
        const int64_t ld = TL_DEC_SEG(a, esi, ld);
#pragma unroll
        for (int i = 0; i < 4; ++i) eres[i] = res[(int64_t)em[i] * ld + en];
    }
    // x is loaded in whole 128-byte lines -- 4 rows x 256 bytes (one chunk)
    // per load -- and rearranged into MFMA A fragments through the wave's LDS
    // stage: the A layout itself (16 rows x 64 bytes per load) touches every
    // line twice and ran at less than half the rate.  Load i: row 4i + lane
    // / 16 of the half (clamped to M - 1; rows >= M are never stored).
    const __amdgpu_buffer_rsrc_t rx = dec_rsrc(a.x, (uint32_t)a.M * (uint32_t)a.ldx * 2u);
    uint32_t                     xv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        xv[i] = (uint32_t)min(kDecHalf * half + 4 * i + (lane >> 4), a.M - 1) * (uint32_t)a.ldx * 2u + 16u * (lane & 15);

    // A chunk's x (XSlot) and its weights and scales (WSlot), in registers.
    struct XSlot {
        u32x4 x[8]; // 4 rows x 256 bytes of x per load
    };
    struct WSlot {
        u32x4  w[PACKED ? 2 * CB : 1]; // [k step pair][cb]: steps 2p (.xy) and 2p + 1 (.zw)
        u32x4  r[PACKED ? 1 : 2 * CB]; // row pieces (reference layout)
        __half s[NF][CB];              // converted at the fold: a conversion here would wait for the load
    };
    auto load_x = [&](XSlot &sl, int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            sl.x[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xv[i], 256 * c, 0));
    };
    auto load_w = [&](WSlot &sl, int c) __attribute__((always_inline)) {
        if constexpr (PACKED) {
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    sl.w[p * CB + cb] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw[cb], 16 * lane + 1024 * p, (nb[cb] * ksteps + 4 * c) * 512, 0));
        } else {
            // stage slot q = t * 64 + lane (16 bytes): row q / CB, slot q % CB
            // of the row, which holds piece (q % CB - dec_rot(row)) mod CB
#pragma unroll
            for (int t = 0; t < 2 * CB; ++t) {
                const int q = t * 64 + lane;
                const int r = q / CB;
                const int p = (q % CB + CB * 64 - dec_rot<CB>(r)) % CB;
                const int k = 128 * c + r;
                const int8_t *src = wb[0];
                int64_t       pitch = sn[0];
#pragma unroll
                for (int cb = 1; cb < CB; ++cb) {
                    src = p == cb ? wb[cb] : src;
                    pitch = p == cb ? (int64_t)sn[cb] : pitch;
                }
                sl.r[t] = *reinterpret_cast<const u32x4 *>(src + k * pitch);
            }
        }
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const int g = (128 * c + 32 * FS * f) >> a.log2_gs;
                sl.s[f][cb] = __builtin_bit_cast(
                    __half, __builtin_amdgcn_raw_buffer_load_b16(rs[cb], sv + 32u * nb[cb], 2 * g * sn[cb], 0));
            }
    };

    f32x4 acc[2][CB], P[2][CB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            acc[rb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            P[rb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    // The wave's stages (one chunk each; LDS operations of a wave run in
    // order, so the next chunk's writes follow this chunk's reads).  x stage:
    // 32 rows of 256 bytes, 32 bytes of padding after each, so that every
    // address is a lane base plus an immediate and neither the stores (16
    // lanes = a row's 16 pieces) nor the A-fragment reads (16 lanes = 16 rows,
    // one piece, 288 bytes apart) conflict in the banks.  (With 16 bytes of
    // padding the reads conflicted: an LDS probe counted one conflict cycle
    // per active cycle; the XOR swizzle this replaces needed ~130 more VALU
    // per wave for its addresses.)
    uint8_t *const xst = reinterpret_cast<uint8_t *>(lds) + (size_t)wave * (XST + WST);
    uint8_t *const wst = xst + XST;
    auto compute = [&](const XSlot &xs, const WSlot &sl, int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 4 * i + (lane >> 4);
            *reinterpret_cast<u32x4 *>(xst + r * XPITCH + 16 * (lane & 15)) = xs.x[i];
        }
        if constexpr (!PACKED) {
#pragma unroll
            for (int t = 0; t < 2 * CB; ++t) *reinterpret_cast<u32x4 *>(wst + (t * 64 + lane) * 16) = sl.r[t];
        }
        // (K is a multiple of 128: every chunk has 4 k steps.)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            f16x8 xa[2]; // A fragments: row 16 rb + lane % 16, piece 4 s + lane / 16
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                const int r = 16 * rb + (lane & 15);
                xa[rb] = *reinterpret_cast<const f16x8 *>(xst + r * XPITCH + 16 * (4 * s + (lane >> 4)));
            }
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                uint2 raw;
                if constexpr (PACKED) {
                    const u32x4 &q = sl.w[(s >> 1) * CB + cb];
                    raw = (s & 1) ? make_uint2(q[2], q[3]) : make_uint2(q[0], q[1]);
                } else {
                    const int   i = lane & 15;
                    const int   r = 32 * s + 8 * (lane >> 4) + (i >> 1);
                    const int   pos = (cb + dec_rot<CB>(r)) % CB;
                    const v2i32 t = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                        (__attribute__((address_space(3))) v2i32 *)(wst + (r * CB + pos) * 16 + 8 * (i & 1)));
                    raw = make_uint2((uint32_t)t[0], (uint32_t)t[1]);
                }
                const uint2 lo = w8x4_to_f16x4<PACKED>(raw.x), hi = w8x4_to_f16x4<PACKED>(raw.y);
                const f16x8 bop = __builtin_bit_cast(f16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
// A fold group's first step starts from a zero accumulator (an
                // inline constant of the MFMA, no register clearing).
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
                    P[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        xa[rb], bop, s % FS == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : P[rb][cb], 0, 0, 0);
            }
            if ((s + 1) % FS == 0) { // end of a fold group
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[rb][cb][i] = fmaf(P[rb][cb][i], h2f(sl.s[s / FS][cb]), acc[rb][cb][i]);
            }
        }
    };

    // This wave's chunks wave, wave + 8, wave + 16, wave + 24 (K <= 4096),
    // fully unrolled.  The weights of all four are requested first (the HBM
    // stream never waits for arithmetic: issuing a chunk's weights only after
    // multiplying an earlier one left the stream at half rate), x through a
    // two-deep ring behind them.  Every load is issued on every path, so the
    // compiler's load counters see the same loads in flight at each wait
    // whichever way a branch went (after a conditional load it would wait
    // for all of them); a chunk past the wave's last one re-reads that last
    // one (cache hits, never multiplied).
    // (A wave without chunks -- K of fewer than 8 chunks -- loads the last
    // chunk of K: every offset below stays inside its operand only for
    // chunks < nchunks.)
    auto chunk_of = [&](int j) __attribute__((always_inline)) {
        return mine > 0 ? wave + kDecWaves * min(j, mine - 1) : nchunks - 1;
    };
    // The loads are issued in the order the multiplies consume them:
    // vector loads complete in issue order, so a chunk's multiply can start
    // once that chunk and the loads issued before it have landed.  The
    // scheduling barriers keep the compiler from hoisting later chunks'
    // weights above an earlier chunk's x, which made the first multiply wait
    // for three chunks of weights; the last chunk's weights follow the third
    // chunk's x, so only the last multiply waits for the end of the stream.
    if constexpr (CB <= 3) {
        WSlot ws[4];
        XSlot xs[2];
        load_w(ws[0], chunk_of(0));
        load_x(xs[0], chunk_of(0));
        __builtin_amdgcn_sched_barrier(0);
        load_w(ws[1], chunk_of(1));
        load_x(xs[1], chunk_of(1));
        __builtin_amdgcn_sched_barrier(0);
        load_w(ws[2], chunk_of(2));
        __builtin_amdgcn_sched_barrier(0);
        if (mine > 0) compute(xs[0], ws[0], chunk_of(0));
        load_x(xs[0], chunk_of(2));
        __builtin_amdgcn_sched_barrier(0);
        load_w(ws[3], chunk_of(3));
        __builtin_amdgcn_sched_barrier(0);
        if (mine > 1) compute(xs[1], ws[1], chunk_of(1));
        load_x(xs[1], chunk_of(3));
        if (mine > 2) compute(xs[0], ws[2], chunk_of(2));
        if (mine > 3) compute(xs[1], ws[3], chunk_of(3));
    } else { // four blocks: registers hold two chunks' weights
        WSlot ws[2];
        XSlot xs[2];
        load_w(ws[0], chunk_of(0));
        load_x(xs[0], chunk_of(0));
        __builtin_amdgcn_sched_barrier(0);
        load_w(ws[1], chunk_of(1));
        load_x(xs[1], chunk_of(1));
        __builtin_amdgcn_sched_barrier(0);
        if (mine > 0) compute(xs[0], ws[0], chunk_of(0));
        load_w(ws[0], chunk_of(2));
        load_x(xs[0], chunk_of(2));
        if (mine > 1) compute(xs[1], ws[1], chunk_of(1));
        load_w(ws[1], chunk_of(3));
        load_x(xs[1], chunk_of(3));
        if (mine > 2) compute(xs[0], ws[0], chunk_of(2));
        if (mine > 3) compute(xs[1], ws[1], chunk_of(3));
    }

    // The 8 waves' tiles, summed in wave order: block (rb, cb) by wave 2cb + rb.
    __syncthreads(); // the sums overwrite the other waves' stages
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
            *reinterpret_cast<f32x4 *>(&lds[(((wave * 2 + rb) * CB + cb) * 64 + lane) * 4]) = acc[rb][cb];
    __syncthreads();
    if (!eact) return;
    f32x4 v = *reinterpret_cast<const f32x4 *>(&lds[(((0 * 2 + erb) * CB + ecb) * 64 + lane) * 4]);
#pragma unroll
    for (int src = 1; src < kDecWaves; ++src) {
        const f32x4 u = *reinterpret_cast<const f32x4 *>(&lds[(((src * 2 + erb) * CB + ecb) * 64 + lane) * 4]);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += u[i];
    }
    // Epilogue: dense out[m][n] = fp16(v); residual fp16(res + fp16(v));
    // cache: the K or V row of entry m at its write position.
    __half *const out = TL_DEC_SEG(a, esi, out);
    const int64_t ld = TL_DEC_SEG(a, esi, ld);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = kDecHalf * half + 16 * erb + 4 * (lane >> 4) + i;
        if (m >= a.M) continue;
        const __half o = __float2half(v[i]);
        if (ekind == kEpiCache) {
            const CacheRows &c = a.cache;
            int64_t          off;
            if (c.block_table) {
                const int blk = c.block_table[(int64_t)erow[i] * c.bt_stride + (int64_t)(epos[i] >> c.log2_blk)];
                off = (int64_t)blk * c.blk_stride + (int64_t)(epos[i] & ((1u << c.log2_blk) - 1)) * c.tok_stride;
            } else {
                off = (int64_t)erow[i] * c.blk_stride + (int64_t)epos[i] * c.tok_stride;
            }
            out[off + en] = o;
        } else if (ekind == kEpiResidual) {
            out[(int64_t)m * ld + en] = __float2half(h2f(eres[i]) + h2f(o));
        } else {
            out[(int64_t)m * ld + en] = o;
        }
    }
}

// Repacks W [K][N] int8 (K % 32 == 0, N % 16 == 0) into the B fragments of
// v_mfma_f32_16x16x32_f16: lane l of the fragment of column block nb and k
// step ks holds W[32 ks + 8 (l / 16) + j][16 nb + l % 16] ^ 0x80, j = 0..7 --
// offset binary (W + 128 as an unsigned byte), which the kernels turn into
// fp16 without the XOR a signed byte needs.  Column block nb takes the K * 16
// bytes from nb * K * 16; within it the steps come in pairs, 1024 bytes per
// pair p with lane l's 16 bytes at 16 l (step 2p, then step 2p + 1), so that
// one 16-byte load per lane brings two steps; a last unpaired step (K % 64 ==
// 32) takes 8 bytes per lane.  One thread per (nb, ks, l).
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
    int8_t *const dst = out + (int64_t)nb * K * 16 + packed_step_offset(ks, K / 32, l);
    *reinterpret_cast<uint2 *>(dst) = make_uint2(lo ^ 0x80808080u, hi ^ 0x80808080u);
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

namespace {
// Shapes w8a16_dec_kernel takes: M <= 64, K a multiple of 128 up to 4096
// (whole chunks, four per wave), byte ranges within its 32-bit buffer offsets.
bool dec_ok(int M, int K, const W8A16Seg *segs, int nseg) {
    if (M > kDecRows || K > kDecMaxK || K % 128 != 0) return false;
    for (int i = 0; i < nseg; ++i)
        if ((int64_t)segs[i].n * K >= ((int64_t)1 << 31)) return false;
    return true;
}

// Plan of w8a16_dec_kernel (M <= kDecRows): row halves, and the smallest
// column-tile width (1..4 blocks; 1..2 for gs < 128) whose tiles x halves fit
// one workgroup per CU.
struct DecPlan {
    int halves = 1, cb = 1, tiles = 0, blocks = 0;
};
DecPlan dec_plan(int M, int gs, const W8A16Seg *segs, int nseg) {
    DecPlan p;
    for (int i = 0; i < nseg; ++i) p.blocks += segs[i].n / 16;
    p.halves = M > kDecHalf ? 2 : 1;
    const int cus = device_cus();
    const int cbmax = gs >= 128 ? 4 : 2; // (several folds per chunk hold more registers)
    p.cb = 1;
    while (p.cb < cbmax && (int64_t)((p.blocks + p.cb - 1) / p.cb) * p.halves > cus) ++p.cb;
    p.tiles = (p.blocks + p.cb - 1) / p.cb;
    return p;
}
} // namespace

size_t w8a16_workspace_floats(int M, int K, int gs, const W8A16Seg *segs, int nseg) {
    if (!w8a16_mfma_ok(K, gs, segs, nseg) || dec_ok(M, K, segs, nseg)) return 0;
    int ntot = 0;
    for (int i = 0; i < nseg; ++i) ntot += segs[i].n;
    const int splits = split_plan(M, K, nullptr);
    return splits > 1 ? (size_t)splits * M * ntot : 0;
}

namespace {
// The decode-sized launch: g's x, shape, segments and cache rows are set.
void launch_dec(const GemmArgs &g, int gs, hipStream_t stream, bool packed) {
    DecArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = g.x;
    a.ldx = g.ldx;
    a.M = g.M;
    a.K = g.K;
    a.gs = gs;
    a.log2_gs = __builtin_ctz((unsigned)gs); // a power of two (w8a16_mfma_ok)
    a.nseg = g.nseg;
    for (int i = 0; i < g.nseg; ++i) a.seg[i] = g.seg[i];
    for (int i = 0; i <= g.nseg; ++i) a.col0[i] = g.col0[i];
    a.cache = g.cache;
    const DecPlan p = dec_plan(g.M, gs, g.seg, g.nseg);
    a.tiles = p.tiles;
    a.tpx = (p.tiles + 7) / 8;
    a.halves = p.halves;
    a.blocks = p.blocks;
    const unsigned grid = (unsigned)(8 * a.tpx * p.halves);
    const int      fs = gs >= 128 ? 4 : gs / 32;
    profile_begin(KernelId::W8A16, stream);
#define TL_W8_DEC(FS, CB)                                                                                  \
    do {                                                                                                   \
        if (packed)                                                                                        \
            hipLaunchKernelGGL((w8a16_dec_kernel<FS, CB, true>), dim3(grid), dim3(512), 0, stream, a);     \
        else                                                                                               \
            hipLaunchKernelGGL((w8a16_dec_kernel<FS, CB, false>), dim3(grid), dim3(512), 0, stream, a);    \
    } while (0)
    if (fs == 4) {
        switch (p.cb) {
        case 1: TL_W8_DEC(4, 1); break;
        case 2: TL_W8_DEC(4, 2); break;
        case 3: TL_W8_DEC(4, 3); break;
        default: TL_W8_DEC(4, 4); break;
        }
    } else if (fs == 2) {
        if (p.cb == 1) TL_W8_DEC(2, 1);
        else TL_W8_DEC(2, 2);
    } else {
        if (p.cb == 1) TL_W8_DEC(1, 1);
        else TL_W8_DEC(1, 2);
    }
#undef TL_W8_DEC
    HIP_CHECK(hipGetLastError());
    profile_end(KernelId::W8A16, stream);
}
} // namespace

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
    if (dec_ok(M, K, segs, nseg)) {
        launch_dec(a, gs, stream, packed);
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
