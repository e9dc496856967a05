// W8A16 GEMM for gfx950 with fused epilogues: out = x @ dequant(W, scales),
// the arithmetic of kernels/w8a16_matmul.cu (reference kernel :71-98, tiled
// kernel :119-217): out[m][n] = fp16(sum_k f(x[m][k]) * (w[k][n] * s[k/gs][n]))
// with an fp32 accumulator, W [K][N] int8 row-major, scales
// [ceil(K/gs)][N] fp16.
//
// MFMA paths (K % 32 == 0, gs in {32, 64, 128, 256, 512}, every segment's
// N % 16 == 0).  Both split K across workgroups for decode-sized M (the split
// count depends on (M, K) only, so an output element's value does not depend
// on which other weight matrices share the launch) and sum the splits in a
// fixed order, so results are deterministic.
//
// Packed weights (w8a16_sk_kernel, the fast path; layout of
// launch_w8a16_pack): one workgroup = 4 waves = a 64x64 output tile over one
// split; wave w takes every fourth group of 4 k steps for the whole tile,
// with W fragments (8 bytes per lane) loaded straight into MFMA operands and
// x staged two k steps at a time in the wave's own LDS by the LDS DMA load
// (coalesced rows) -- no barrier until the waves' tiles are summed through
// LDS.
//
// Reference layout (w8a16_mfma_kernel):
//   One workgroup = 4 waves = a 64-row x 64-column output tile over one split
//   of K (split-K across workgroups when the tiles alone would leave CUs
//   idle).  Per 64-row K chunk:
//     - the x chunk [64 rows][64 k] fp16 is loaded cooperatively and staged in
//       LDS (row-major, padded), read back in the A layout of
//       v_mfma_f32_16x16x32_f16 (lane l: row l%16, k 8*(l/16)..+7);
//     - the W chunk [64 k][64 columns] int8 is loaded cooperatively as
//       dwords (4 rows x 4 columns per thread), transposed in registers,
//       converted to fp16 (exact) and stored [column][k] in LDS, read back in
//       the B layout (lane l: column l%16, k 8*(l/16)..+7); wave w owns
//       columns 16w..16w+15;
//     - two 32-deep k steps of MFMA on the integer weights; at the end of each
//       scale group the group's partial product is folded into the fp32
//       accumulator with its scale: acc += P_g * s[g][n] (a k step never
//       straddles groups, and the fold points are compile-time constants).
//   The loads of up to 8 chunks are issued before the first is consumed.
// With one split the GEMM kernel applies the epilogue directly; otherwise it
// writes fp32 partials and w8a16_reduce_kernel sums the splits in split order
// and applies the epilogue.  The two MFMA kernels sum in different orders, so
// their results agree to within rounding, not bit for bit.
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
constexpr int kBN = 64;       // columns per workgroup (16 per wave)
constexpr int kBK = 64;       // k rows per chunk
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kRing = 8;      // chunks whose loads are issued together
constexpr int kXPitch = kBK + 8; // halves per staged x row (16-byte pad)
constexpr int kWPitch = kBK + 8; // halves per staged transposed W column (16-byte rows)
constexpr int kWaitVm0 = 0x0F70;   // s_waitcnt vmcnt(0)
constexpr int kWaitLgkm0 = 0xC07F; // s_waitcnt lgkmcnt(0)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const __half *x; // [M][K]
    int64_t       ldx;
    int           M, K, gs;
    int           nseg;
    int           splits;
    int           chunks_per_split; // 64-row chunks of K per split
    int           tiles;            // column tiles over all segments
    int           mtiles;           // row tiles
    int           units;            // column-tile pairs x splits x row tiles
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

// Byte transpose of a 4x4 block: d[r] holds columns 0..3 of row r; returns
// c[j] = (row 0..3 of column j).
__device__ __forceinline__ void transpose4x4(const uint32_t (&d)[4], uint32_t (&c)[4]) {
    const uint32_t lo01 = __builtin_amdgcn_perm(d[1], d[0], 0x05010400u); // r0c0 r1c0 r0c1 r1c1
    const uint32_t hi01 = __builtin_amdgcn_perm(d[1], d[0], 0x07030602u); // r0c2 r1c2 r0c3 r1c3
    const uint32_t lo23 = __builtin_amdgcn_perm(d[3], d[2], 0x05010400u);
    const uint32_t hi23 = __builtin_amdgcn_perm(d[3], d[2], 0x07030602u);
    c[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
    c[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
    c[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
    c[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Four signed bytes -> four fp16 (exact), packed for one 8-byte LDS store.
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

// Workgroup (4 waves, 256 threads) -> (64-row tile, 64-column tile, K split).
// Grid layout: the two column tiles of a pair (which share the 128-byte
// lines of every weight row) get block indices 8 apart, i.e. the same XCD
// under the round-robin dispatch of workgroups to XCDs, so each line is read
// from HBM into one L2 once.  K is processed in batches of kRing 64-row
// chunks; a batch starts on a multiple of 512 rows, so with GS | 512 its scale
// groups are fixed at compile time: the batch's scales (one per lane and
// group), W (four dwords per thread per chunk: rows 4*(t/16)..+3, columns
// 4*(t%16)..+3) and x (two 16-byte pieces per thread per chunk) are all
// issued before the first chunk is consumed, and the partial product of each
// group is folded into the accumulator at a static point.  Per chunk: W is
// transposed in registers (v_perm), converted to fp16 and stored [column][k]
// with 8-byte LDS writes, x is staged with 16-byte writes, then two 32-deep
// MFMA k-steps per 16-row block.
template <int GS>
__global__ __launch_bounds__(kThreads) void w8a16_mfma_kernel(GemmArgs a) {
    static_assert(GS % 32 == 0 && (kRing * kBK) % GS == 0, "group size");
    constexpr int SPG = GS / 32;                 // k steps per scale group
    constexpr int NG = kRing * kBK / GS;         // scale groups per batch
    // Double-buffered staging: chunk j uses buffer j & 1, so one barrier per
    // chunk suffices (a buffer is rewritten two chunks later, after every
    // wave has passed the intervening barrier, i.e. finished reading it).
    __shared__ __align__(16) _Float16 xs[2][kBM * kXPitch];
    __shared__ __align__(16) _Float16 wt[2][kBN * kWPitch];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = threadIdx.x;
    // block -> (unit, half); unit -> (pair, split, m tile)
    const int b = blockIdx.x;
    const int unit = (b >> 4) * 8 + (b & 7);
    const int half = (b >> 3) & 1;
    if (unit >= a.units) return;
    const int mt = unit % a.mtiles;
    const int rest = unit / a.mtiles;
    const int split = rest % a.splits;
    const int pair = rest / a.splits;
    int       tile = 2 * pair + half;
    if (tile >= a.tiles) return;
    int si = 0;
    while (si + 1 < a.nseg && tile >= (a.seg[si].n + kBN - 1) / kBN) {
        tile -= (a.seg[si].n + kBN - 1) / kBN;
        ++si;
    }
    const W8A16Seg &sg = a.seg[si];
    const int       c0 = tile * kBN;     // first column of the workgroup in the segment
    const int       n0 = c0 + 16 * wave; // this wave's first column
    const bool      wave_live = n0 < sg.n;
    const int       m0 = mt * kBM;
    const int       kchunks = (a.K + kBK - 1) / kBK;
    const int       c_begin = split * a.chunks_per_split; // a multiple of kRing
    const int       c_end = min(kchunks, c_begin + a.chunks_per_split);
    const int       ngroups = (a.K + GS - 1) / GS;

    // Loads are never masked: every address is clamped into the operand, and
    // what a clamped element feeds is either discarded (output columns >= n,
    // rows >= M) or skipped (k steps >= K, a uniform branch), so no load
    // ends up in a divergent branch with a wait right behind it.
    const int     wq = 4 * (t & 15); // W column quad (within the tile)
    const int     wr = 4 * (t >> 4); // W row quad (within the chunk)
    const int     wcol = min(c0 + wq, sg.n - 4);
    const int8_t *wbase = sg.w + (int64_t)wr * sg.n + wcol;
    const int64_t wchunk = (int64_t)kBK * sg.n;
    const int     ksteps = a.K >> 5;
    const __half *xrow[2];
    int           xk[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int q = t + kThreads * u;
        const int r = q >> 3, kp = q & 7;
        xrow[u] = a.x + (int64_t)min(m0 + r, a.M - 1) * a.ldx;
        xk[u] = 8 * kp;
    }
    const int     ncol = n0 + (lane & 15); // this lane's output column (D layout)
    const __half *sbase = sg.s + min(ncol, sg.n - 1);

    f32x4 acc[4], P[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        acc[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        P[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    for (int cb = c_begin; cb < c_end; cb += kRing) {
        // Every load below is unconditional, from an address that is valid
        // whether or not the element is (masked elements read element 0 and
        // are zeroed afterwards), so no load sits in a divergent branch and
        // the waits are deferred to the first use.
        const int g0 = cb * kBK / GS; // first scale group of the batch
        uint16_t  sraw[NG];
#pragma unroll
        for (int i = 0; i < NG; ++i)
            sraw[i] = *reinterpret_cast<const uint16_t *>(sbase + (int64_t)min(g0 + i, ngroups - 1) * sg.n);
        // W of all kRing chunks in flight at once (HBM); x (L2-resident) one
        // chunk ahead.
        uint32_t wbuf[kRing][4]; // reference layout: rows wr..wr+3 x columns wq..wq+3
        uint4    xbuf[2][2];
        auto     load_x = [&](int j, uint4(&xv)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
                xv[u] = *reinterpret_cast<const uint4 *>(xrow[u] + min((cb + j) * kBK + xk[u], a.K - 8));
        };
#pragma unroll
        for (int j = 0; j < kRing; ++j) {
            const int c = min(cb + j, kchunks - 1);
            const int8_t *wp = wbase + (int64_t)c * wchunk;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wbuf[j][i] = *reinterpret_cast<const uint32_t *>(
                    wp + (int64_t)min(i, a.K - 1 - c * kBK - wr) * sg.n); // row <= K - 1
        }
        load_x(0, xbuf[0]);
#pragma unroll
        for (int j = 0; j < kRing; ++j) {
            const int c = cb + j;
            if (c >= c_end) break; // uniform; zero steps add nothing, groups folded below
            if (j + 1 < kRing) load_x(j + 1, xbuf[(j + 1) & 1]);
            _Float16 *xsb = xs[j & 1];
            _Float16 *wtb = wt[j & 1];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int q = t + kThreads * u;
                const int r = q >> 3, kp = q & 7;
                *reinterpret_cast<uint4 *>(&xsb[r * kXPitch + 8 * kp]) = xbuf[j & 1][u];
            }
            {
                uint32_t col[4];
                transpose4x4(wbuf[j], col);
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    *reinterpret_cast<uint2 *>(&wtb[(wq + jj) * kWPitch + wr]) = i8x4_to_f16x4(col[jj]);
            }
            __syncthreads();
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                if (32 * (2 * c + ks) >= a.K) break; // uniform: the half chunk beyond K (K % 64 == 32)
                const f16x8 bop = *reinterpret_cast<const f16x8 *>(
                    &wtb[(16 * wave + (lane & 15)) * kWPitch + 32 * ks + 8 * (lane >> 4)]);
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    const f16x8 aop = *reinterpret_cast<const f16x8 *>(
                        &xsb[(16 * rb + (lane & 15)) * kXPitch + 32 * ks + 8 * (lane >> 4)]);
                    P[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, P[rb], 0, 0, 0);
                }
                const int step = 2 * j + ks; // static
                if ((step + 1) % SPG == 0) { // end of scale group step / SPG
                    const float s_ = h2f(__builtin_bit_cast(__half, sraw[step / SPG])) *
                                     (g0 + step / SPG < ngroups ? 1.0f : 0.0f);
#pragma unroll
                    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[rb][i] = fmaf(P[rb][i], s_, acc[rb][i]);
                        P[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    }
                }
            }
        }
        __syncthreads(); // the next batch restages both buffers
        // A batch cut short inside a group (K % GS != 0): fold the rest with
        // that group's scale.  Steps executed: those of the batch's chunks
        // that lie below K.
        const int done_steps = min(2 * min(kRing, c_end - cb), ksteps - 2 * cb);
        if (done_steps % SPG) {
            float s_ = 0.0f;
#pragma unroll
            for (int i = 0; i < NG; ++i)
                s_ = (i == done_steps / SPG && g0 + i < ngroups) ? h2f(__builtin_bit_cast(__half, sraw[i])) : s_;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[rb][i] = fmaf(P[rb][i], s_, acc[rb][i]);
                P[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    }
    if (!wave_live) return;

    // D layout: lane holds rows 16*rb + 4*(lane/16) + i, column lane%16.
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + 16 * rb + 4 * (lane >> 4) + i;
            if (m >= a.M) continue;
            if (a.splits > 1) {
                a.partial[((int64_t)split * a.M + m) * a.ntot + a.col0[si] + ncol] = acc[rb][i];
            } else {
                epilogue(a, si, m, ncol, acc[rb][i]);
            }
        }
    }
}

// Packed-weight kernel, split-K inside the workgroup: one workgroup (4 waves)
// per unit (64-row tile, 64-column tile, K split); wave w takes k steps
// 4w..4w+3 of every 16-step (512-row) batch of the split for the whole 64x64
// tile, W straight from global memory (8 bytes per lane per fragment,
// packed), x through the wave's LDS stage (below), 16 MFMAs per step.  Scale groups are folded in step order.  The four
// waves' tiles are summed through LDS in wave order, wave w finishing row
// block w (each wave passes on the three row blocks it does not finish: 48
// KB of LDS, three workgroups per CU).  ACC: a second accumulator for
// several scale groups per wave (group size < 128, or more than one batch);
// without it the wave's result is P * s.
template <int GS, bool ACC>
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

    const int8_t *wp[4]; // uniform column-block bases; lanes add 8 * lane (+ 512 per step)
    const __half *sp[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int nb = min((c0 >> 4) + cb, nblk - 1);
        wp[cb] = sg.w + (int64_t)nb * ksteps * 512;
        sp[cb] = sg.s + 16 * nb;
    }
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
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int st = min(first + j, ksteps - 1);
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
                wv[j][cb] = *reinterpret_cast<const uint2 *>(wp[cb] + (uint32_t)(st * 512 + 8 * lane));
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
        if (nsteps > 2) { // the stage's reads complete before the DMA refills it
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            issue_x(first + 2);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j >= nsteps) continue; // uniform
            if (j == 2) {
                __builtin_amdgcn_s_waitcnt(kWaitVm0);
                read_x(0, xv[0]);
                read_x(1, xv[1]);
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
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s = 0; s < a.splits; ++s) {
        const float4 p = *reinterpret_cast<const float4 *>(a.partial + ((int64_t)s * a.M + m) * a.ntot + c);
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
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
    int       splits = M <= 256 ? std::min(8, std::max(1, K / 512)) : 1;
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
    a.units = (tiles + 1) / 2 * splits * mt;
    a.partial = splits > 1 ? workspace : nullptr;
    if (splits > 1 && !workspace) throw std::invalid_argument("w8a16: split-K needs a workspace");
    const unsigned blocks = (unsigned)((a.units + 7) / 8 * 16); // pairs of 8-block groups
    profile_begin(KernelId::W8A16, stream);
    if (packed) {
        // Several scale groups per wave (gs < 128) or more than one 512-row
        // batch per split need the second accumulator.
        const bool     acc = gs < 128 || a.chunks_per_split > 8;
        const unsigned units = (unsigned)(splits * tiles * mt);
#define TL_W8_SK_LAUNCH(G)                                                                          \
    do {                                                                                            \
        if (acc)                                                                                    \
            hipLaunchKernelGGL((w8a16_sk_kernel<G, true>), dim3(units), dim3(256), 0, stream, a);   \
        else                                                                                        \
            hipLaunchKernelGGL((w8a16_sk_kernel<(G < 128 ? 128 : G), false>), dim3(units), dim3(256), 0, \
                               stream, a);                                                          \
    } while (0)
        switch (gs) {
        case 32: TL_W8_SK_LAUNCH(32); break;
        case 64: TL_W8_SK_LAUNCH(64); break;
        case 128: TL_W8_SK_LAUNCH(128); break;
        case 256: TL_W8_SK_LAUNCH(256); break;
        default: TL_W8_SK_LAUNCH(512); break;
        }
#undef TL_W8_SK_LAUNCH
    } else {
#define TL_W8_LAUNCH(G) \
    hipLaunchKernelGGL((w8a16_mfma_kernel<G>), dim3(blocks), dim3(kThreads), 0, stream, a)
        switch (gs) {
        case 32: TL_W8_LAUNCH(32); break;
        case 64: TL_W8_LAUNCH(64); break;
        case 128: TL_W8_LAUNCH(128); break;
        case 256: TL_W8_LAUNCH(256); break;
        default: TL_W8_LAUNCH(512); break;
        }
#undef TL_W8_LAUNCH
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
