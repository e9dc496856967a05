// W8A16 GEMM for gfx950 with fused epilogues: out = x @ dequant(W, scales),
// the arithmetic of kernels/w8a16_matmul.cu (reference kernel :71-98, tiled
// kernel :119-217): out[m][n] = fp16(sum_k f(x[m][k]) * (w[k][n] * s[k/gs][n]))
// with an fp32 accumulator, W [K][N] int8 row-major, scales
// [ceil(K/gs)][N] fp16.
//
// MFMA path (K % 32 == 0, gs % 32 == 0, every segment's N % 16 == 0):
//   One workgroup = 2 waves = a 64-row x 32-column output tile over one split
//   of K (split-K across workgroups when the tiles alone would leave CUs
//   idle).  Per 64-row K chunk:
//     - the x chunk [64 rows][64 k] fp16 is loaded cooperatively and staged in
//       LDS (row-major, padded), read back in the A layout of
//       v_mfma_f32_16x16x32_f16 (lane l: row l%16, k 8*(l/16)..+7);
//     - each wave loads its 16 columns of the W chunk (lane l: row l, 16
//       bytes), converts the int8 values to fp16 (exact) and stores them
//       transposed ([column][k]) in LDS, read back in the B layout (lane l:
//       column l%16, k 8*(l/16)..+7);
//     - two 32-deep k steps of MFMA on the integer weights; at the end of each
//       scale group the group's partial product is folded into the fp32
//       accumulator with its scale: acc += P_g * s[g][n] (gs % 32 == 0 keeps a
//       k step inside one group).
//   The next chunk's global loads are issued before the current chunk's MFMA.
//   With one split the workgroup applies the epilogue directly; otherwise it
//   writes fp32 partials and w8a16_reduce_kernel sums the splits in a fixed
//   order (deterministic) and applies the epilogue.  The split count depends
//   on (M, K) only, so an output element's value does not depend on which
//   other weight matrices share the launch.
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
constexpr int kBN = 32;       // columns per workgroup (16 per wave)
constexpr int kBK = 64;       // k rows per chunk
constexpr int kWaves = 2;
constexpr int kThreads = 64 * kWaves;
constexpr int kXPitch = kBK + 8; // halves per staged x row (16-byte pad)
constexpr int kWPitch = kBK + 8; // halves per staged transposed W column

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const __half *x; // [M][K]
    int64_t       ldx;
    int           M, K, gs;
    int           nseg;
    int           splits;
    int           chunks_per_split; // 64-row chunks of K per split
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

__global__ __launch_bounds__(kThreads) void w8a16_mfma_kernel(GemmArgs a) {
    __shared__ __align__(16) _Float16 xs[kBM * kXPitch];
    __shared__ __align__(16) _Float16 wt[kWaves][16 * kWPitch];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // tile -> segment, columns
    int tile = blockIdx.x;
    int si = 0;
    while (si + 1 < a.nseg && tile >= (a.seg[si].n + kBN - 1) / kBN) {
        tile -= (a.seg[si].n + kBN - 1) / kBN;
        ++si;
    }
    const W8A16Seg &sg = a.seg[si];
    const int       n0 = tile * kBN + 16 * wave; // this wave's first column in the segment
    const bool      wave_live = n0 < sg.n;
    const int       m0 = blockIdx.y * kBM;
    const int       split = blockIdx.z;
    const int       kchunks = a.K / kBK + (a.K % kBK ? 1 : 0);
    const int       c_begin = split * a.chunks_per_split;
    const int       c_end = min(kchunks, c_begin + a.chunks_per_split);

    // Global loads of one chunk: x (kXPer x 16 B per thread: 64 rows x 128 B),
    // W (16 B per lane: row k0 + lane, the wave's 16 columns).
    constexpr int kXPer = kBM * kBK / 8 / kThreads;
    auto load_chunk = [&](int c, uint4(&xv)[kXPer], uint4 &wv) __attribute__((always_inline)) {
        const int k0 = c * kBK;
#pragma unroll
        for (int u = 0; u < kXPer; ++u) {
            const int q = threadIdx.x + kThreads * u;
            const int r = q >> 3, kp = q & 7;
            const int m = m0 + r, k = k0 + 8 * kp;
            xv[u] = (m < a.M && k < a.K)
                        ? *reinterpret_cast<const uint4 *>(a.x + (int64_t)m * a.ldx + k)
                        : make_uint4(0u, 0u, 0u, 0u);
        }
        const int k = k0 + lane;
        wv = (wave_live && k < a.K)
                 ? *reinterpret_cast<const uint4 *>(sg.w + (int64_t)k * sg.n + n0)
                 : make_uint4(0u, 0u, 0u, 0u);
    };

    f32x4 acc[4], P[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        acc[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        P[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    int   gcur = -1;
    float scur = 0.0f;
    const int ncol = n0 + (lane & 15); // this lane's output column (D layout)
    auto fold = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[rb][i] = fmaf(P[rb][i], scur, acc[rb][i]);
            P[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    // Stage chunk c from (xv, wv), prefetch chunk c + 1 into (xn, wn), multiply.
    auto body = [&](int c, const uint4(&xv)[kXPer], const uint4 &wv, uint4(&xn)[kXPer],
                    uint4 &wn) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < kXPer; ++u) {
            const int q = threadIdx.x + kThreads * u;
            const int r = q >> 3, kp = q & 7;
            *reinterpret_cast<uint4 *>(&xs[r * kXPitch + 8 * kp]) = xv[u];
        }
        {
            const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
            _Float16      *dst = &wt[wave][lane];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int8_t v = (int8_t)((wd[j >> 2] >> (8 * (j & 3))) & 0xffu);
                dst[j * kWPitch] = (_Float16)v;
            }
        }
        __syncthreads();
        if (c + 1 < c_end) load_chunk(c + 1, xn, wn); // in flight during the MFMAs
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int k0 = c * kBK + 32 * ks;
            if (k0 >= a.K) break;
            const int g = k0 / a.gs;
            if (g != gcur) {
                if (gcur >= 0) fold();
                gcur = g;
                scur = wave_live ? h2f(sg.s[(int64_t)g * sg.n + ncol]) : 0.0f;
            }
            const f16x8 bop = *reinterpret_cast<const f16x8 *>(
                &wt[wave][(lane & 15) * kWPitch + 32 * ks + 8 * (lane >> 4)]);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const f16x8 aop = *reinterpret_cast<const f16x8 *>(
                    &xs[(16 * rb + (lane & 15)) * kXPitch + 32 * ks + 8 * (lane >> 4)]);
                P[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, P[rb], 0, 0, 0);
            }
        }
        __syncthreads(); // xs / wt are restaged by the next chunk
    };

    uint4 xa[kXPer], xb[kXPer], wa, wb;
    if (c_begin < c_end) load_chunk(c_begin, xa, wa);
    for (int c = c_begin; c < c_end; c += 2) {
        body(c, xa, wa, xb, wb);
        if (c + 1 < c_end) body(c + 1, xb, wb, xa, wa);
    }
    if (gcur >= 0) fold();
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

// Sums the split-K partials in split order and applies the epilogue.
__global__ __launch_bounds__(256) void w8a16_reduce_kernel(GemmArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)a.M * a.ntot) return;
    const int m = (int)(idx / a.ntot);
    const int c = (int)(idx - (int64_t)m * a.ntot);
    int       si = 0;
    while (si + 1 < a.nseg && c >= a.col0[si + 1]) ++si;
    float v = 0.0f;
    for (int s = 0; s < a.splits; ++s) v += a.partial[((int64_t)s * a.M + m) * a.ntot + c];
    epilogue(a, si, m, c - a.col0[si], v);
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
    if (K % 32 != 0 || gs % 32 != 0) return false;
    for (int i = 0; i < nseg; ++i)
        if (segs[i].n % 16 != 0) return false;
    return true;
}

namespace {
// Split-K plan, a function of (M, K) only -- never of the columns sharing the
// launch -- so that every output element is summed in the same order whether
// its weight matrix is multiplied alone or fused with others (the fused
// projection's cache bytes equal the unfused path's).  Decode-sized M splits K
// into up to 8 ranges of >= 1024 rows for parallelism; larger M has enough
// row tiles.  Sets the 64-row chunks per split.
int split_plan(int M, int K, int *chunks_per_split) {
    const int kchunks = (K + kBK - 1) / kBK;
    int       splits = M <= 256 ? std::min(8, std::max(1, K / 1024)) : 1;
    const int cps = (kchunks + splits - 1) / splits;
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
                  const CacheRows *cache, float *workspace, hipStream_t stream) {
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
    const bool mfma = g_force_generic != 1 && aligned && w8a16_mfma_ok(K, gs, segs, nseg);
    if (!mfma) {
        a.splits = 1;
        const int64_t total = (int64_t)M * a.ntot;
        hipLaunchKernelGGL(w8a16_generic_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           stream, a);
        HIP_CHECK(hipGetLastError());
        return;
    }
    const int mt = (M + kBM - 1) / kBM;
    const int splits = split_plan(M, K, &a.chunks_per_split);
    a.splits = splits;
    a.partial = splits > 1 ? workspace : nullptr;
    if (splits > 1 && !workspace) throw std::invalid_argument("w8a16: split-K needs a workspace");
    hipLaunchKernelGGL(w8a16_mfma_kernel, dim3((unsigned)tiles, (unsigned)mt, (unsigned)splits),
                       dim3(kThreads), 0, stream, a);
    HIP_CHECK(hipGetLastError());
    if (splits > 1) {
        const int64_t total = (int64_t)M * a.ntot;
        hipLaunchKernelGGL(w8a16_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           stream, a);
        HIP_CHECK(hipGetLastError());
    }
}

void w8a16_force_generic(int on) { g_force_generic = on; }

} // namespace detail
} // namespace tiny_llm
