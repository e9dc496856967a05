// Split-K flash-decoding GQA attention over the KV cache, for gfx950.
//
// Computes, for every batch entry b and query head h (kv head g = h / G):
//   s_t = (q_h . k_{g,t}) * scale,  p_t = exp(s_t - max s),
//   o_h = (sum_t p_t v_{g,t}) / (sum_t p_t + 1e-6)           t in [0, S_b)
// which is the arithmetic of attention_decode_kernel (kernels/attention.cu:
// 11-112: scores, max, expf, 1/(sum+1e-6f), P.V, RNE fp16 output), extended to
// GQA over the token-major cache of kv_cache.cpp:226-233.
//
// Work decomposition.  One workgroup (4 wave64) per (entry b, kv head g,
// chunk of <= 512 tokens).  The G query heads of the group share every K/V
// byte the workgroup reads: K and V are loaded once from HBM into VGPRs and
// used for all G heads.
//   phase 1  QK^T: 8 lanes per token, each lane holds D/8 contiguous-in-pieces
//            dims of q for the G heads in registers; v_dot2_f32_f16 partial
//            dots, summed over the 8 lanes with DPP (quad_perm x2,
//            row_half_mirror).  Scores are scaled by scale*log2(e) so that
//            exp(s - m) = exp2(s' - m'), evaluated with v_exp_f32 (the
//            standard change of base; no CUDA math routine is reproduced).
//   softmax  chunk max / sum per head: lane registers -> shfl-xor over the
//            lanes that own the head -> LDS across the 4 waves.  p_t goes to
//            LDS ([t][G] fp32) once.
//   phase 2  P.V: D/8 lanes per token, 8 dims per lane, fp32 FMAs with p
//            broadcast from LDS; partial sums reduced over the token lanes
//            (shfl-xor) and the 4 waves (LDS).
//   output   an entry whose sequence fits in one chunk is normalised and
//            written as fp16 directly; otherwise (m, l, o[D]) partials go to
//            the workspace and attn_merge_kernel combines the chunks:
//            m* = max m_c, l = sum l_c 2^(m_c-m*), o = sum o_c 2^(m_c-m*) / (l+1e-6).
//
// Every global load of a lane uses a token index clamped into [0, n) of its
// chunk, so no load leaves the attended range; masked tokens get p = 0.
#include "kv_kernels.h"

#include "tiny_llm/hip_utils.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace tiny_llm {
namespace detail {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTokPerWaveMax = kChunkMax / kWaves; // 128

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct AttnArgs {
    const __half *q;
    __half       *out;
    float        *part_o;  // [n_work][Hq][D]
    float        *part_ml; // [n_work][Hq][2]
    KvView        kv;
    AttnPlan      plan;
    int           Hq;
    float         scale_log2; // scale * log2(e)
};

// Address of token rows of one batch entry (see KvView).
struct SeqAddr {
    const int32_t *bt_row;
    int64_t        fixed;
    int64_t        blk_stride;
    int64_t        tok_stride;
    int            log2_blk;
    int            mask;

    __device__ __forceinline__ SeqAddr(const KvView &v, int b) {
        const int row = v.seq_row ? v.seq_row[b] : b;
        bt_row = v.block_table ? v.block_table + (int64_t)row * v.bt_stride : nullptr;
        fixed = (int64_t)row * v.blk_stride;
        blk_stride = v.blk_stride;
        tok_stride = v.tok_stride;
        log2_blk = v.log2_blk;
        mask = (1 << v.log2_blk) - 1;
    }
    __device__ __forceinline__ int64_t off(int t) const {
        const int64_t blk = bt_row ? (int64_t)bt_row[t >> log2_blk] * blk_stride : fixed;
        return blk + (int64_t)(t & mask) * tok_stride;
    }
};

// Sum over the 8 lanes of each half-row (lanes 8k..8k+7); result in all 8.
__device__ __forceinline__ float sum8(float v) {
    int x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false));
    return v;
}

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc,
                                  false);
}

// Phase-1 piece of a token row owned by lane c8 (0..7): D/8 halves.
// D >= 64: 16-byte pieces at halves p*64 + 8*c8 (p < D/64), so each load
// instruction of the 8 lanes of a token covers 128 contiguous bytes.
// D == 32: one 8-byte piece at 4*c8.
template <int D>
__device__ __forceinline__ void load_p1(const __half *row, int c8, uint32_t (&r)[D / 16]) {
    if constexpr (D == 32) {
        const uint2 v = *reinterpret_cast<const uint2 *>(row + 4 * c8);
        r[0] = v.x;
        r[1] = v.y;
    } else {
#pragma unroll
        for (int p = 0; p < D / 64; ++p) {
            const uint4 v = *reinterpret_cast<const uint4 *>(row + p * 64 + 8 * c8);
            r[4 * p + 0] = v.x;
            r[4 * p + 1] = v.y;
            r[4 * p + 2] = v.z;
            r[4 * p + 3] = v.w;
        }
    }
}

__device__ __forceinline__ void h8_to_f(uint4 v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f16x2 h = __builtin_bit_cast(f16x2, w[i]);
        f[2 * i] = (float)h.x;
        f[2 * i + 1] = (float)h.y;
    }
}

template <int D, int G>
__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(AttnArgs a) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group size");
    static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head_dim");
    constexpr int NQ = D / 16;  // dwords of a token row per phase-1 lane
    constexpr int LPT = D / 8;  // phase-2 lanes per token (8 dims each)
    constexpr int TPI = 64 / LPT; // phase-2 tokens per wave step

    __shared__ float s_p[kChunkMax * G];
    __shared__ float s_mx[kWaves][G];
    __shared__ float s_sm[kWaves][G];
    __shared__ float s_acc[kWaves * G * D];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = blockIdx.y;
    const AttnPlan &pl = a.plan;

    int b, c;
    if (pl.work) {
        b = pl.work[2 * blockIdx.x];
        c = pl.work[2 * blockIdx.x + 1];
    } else {
        b = blockIdx.x / pl.nchunk;
        c = blockIdx.x - b * pl.nchunk;
    }
    const int S = pl.seq_lens ? pl.seq_lens[b] : pl.uniform_len;
    const int nch = pl.part_base ? pl.part_base[b + 1] - pl.part_base[b] : pl.nchunk;
    const int widx = pl.part_base ? pl.part_base[b] + c : (int)blockIdx.x;
    const int t0 = c * pl.chunk;
    const int n = min(pl.chunk, S - t0); // >= 1 by construction of the plan
    const int tpw = pl.chunk / kWaves;   // tokens per wave, multiple of 16
    const int wt0 = wave * tpw;

    const SeqAddr addr(a.kv, b);
    const __half *kbase = a.kv.k_base + (int64_t)g * a.kv.head_stride;
    const __half *vbase = a.kv.v_base + (int64_t)g * a.kv.head_stride;

    // ---------------- phase 1: scores ----------------
    const int tg = lane >> 3; // token within the 8-token step
    const int c8 = lane & 7;  // dim piece
    uint32_t qr[G][NQ];
    {
        const __half *qb = a.q + ((int64_t)b * a.Hq + (int64_t)g * G) * D;
#pragma unroll
        for (int h = 0; h < G; ++h) load_p1<D>(qb + h * D, c8, qr[h]);
    }

    float sc[kTokPerWaveMax / 8];
#pragma unroll
    for (int i = 0; i < kTokPerWaveMax / 8; ++i) sc[i] = -INFINITY;

#pragma unroll
    for (int ib = 0; ib < kTokPerWaveMax / 8; ib += 4) {
        if (ib * 8 < tpw && wt0 + ib * 8 < n) {
            uint32_t kr[4][NQ];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int tl = wt0 + (ib + u) * 8 + tg;
                const int tc = tl < n ? tl : n - 1;
                load_p1<D>(kbase + addr.off(t0 + tc), c8, kr[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float mine = 0.0f;
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    float s = 0.0f;
#pragma unroll
                    for (int j = 0; j < NQ; ++j) s = fdot2(qr[h][j], kr[u][j], s);
                    s = sum8(s);
                    mine = (c8 == h) ? s : mine;
                }
                const int tl = wt0 + (ib + u) * 8 + tg;
                if (tl < n) sc[ib + u] = mine * a.scale_log2;
            }
        }
    }

    // ---------------- softmax over the chunk ----------------
    const bool owner = c8 < G; // lane c8 owns head c8
    float      m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kTokPerWaveMax / 8; ++i) m = fmaxf(m, sc[i]);
    m = fmaxf(m, __shfl_xor(m, 8));
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    if (lane < G) s_mx[wave][lane] = m;
    __syncthreads();

    float mc = -INFINITY;
    if (owner) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mc = fmaxf(mc, s_mx[w][c8]);
    }
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < kTokPerWaveMax / 8; ++i) {
        if (i * 8 < tpw) {
            const float p = owner ? __builtin_amdgcn_exp2f(sc[i] - mc) : 0.0f;
            lsum += p;
            if (owner) s_p[(wt0 + i * 8 + tg) * G + c8] = p;
        }
    }
    lsum += __shfl_xor(lsum, 8);
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (lane < G) s_sm[wave][lane] = lsum;
    __syncthreads();

    // ---------------- phase 2: P.V ----------------
    const int tq = lane / LPT;
    const int dg = lane % LPT;
    float     acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;

    constexpr int kSteps = kTokPerWaveMax / TPI;
    constexpr int kBatch = kSteps < 8 ? kSteps : 8;
#pragma unroll
    for (int jb = 0; jb < kSteps; jb += kBatch) {
        if (jb * TPI < tpw && wt0 + jb * TPI < n) {
            uint4 vr[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int tl = wt0 + (jb + u) * TPI + tq;
                const int tc = tl < n ? tl : n - 1;
                vr[u] = *reinterpret_cast<const uint4 *>(vbase + addr.off(t0 + tc) + dg * 8);
            }
            const bool partial = wt0 + (jb + kBatch) * TPI > n || (jb + kBatch) * TPI > tpw;
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int tl = wt0 + (jb + u) * TPI + tq;
                if ((jb + u) * TPI >= tpw) break; // uniform: beyond this wave's range
                uint4 v = vr[u];
                if (partial && tl >= n) v = make_uint4(0u, 0u, 0u, 0u);
                float vf[8];
                h8_to_f(v, vf);
                float p[G];
                if constexpr (G >= 4) {
#pragma unroll
                    for (int h4 = 0; h4 < G; h4 += 4) {
                        const float4 pp = *reinterpret_cast<const float4 *>(&s_p[tl * G + h4]);
                        p[h4] = pp.x;
                        p[h4 + 1] = pp.y;
                        p[h4 + 2] = pp.z;
                        p[h4 + 3] = pp.w;
                    }
                } else if constexpr (G == 2) {
                    const float2 pp = *reinterpret_cast<const float2 *>(&s_p[tl * 2]);
                    p[0] = pp.x;
                    p[1] = pp.y;
                } else {
                    p[0] = s_p[tl];
                }
#pragma unroll
                for (int h = 0; h < G; ++h)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p[h], vf[e], acc[h][e]);
            }
        }
    }

    // reduce over the token lanes (same dg)
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1)
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] += __shfl_xor(acc[h][e], off);
    if (tq == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float *dst = &s_acc[(wave * G + h) * D + dg * 8];
            *reinterpret_cast<float4 *>(dst) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
            *reinterpret_cast<float4 *>(dst + 4) =
                make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
    }
    __syncthreads();

    // ---------------- combine waves, emit ----------------
    for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
        const int h = idx / D;
        const int d = idx - h * D;
        float     o = 0.0f, mh = -INFINITY, lh = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            o += s_acc[(w * G + h) * D + d];
            mh = fmaxf(mh, s_mx[w][h]);
            lh += s_sm[w][h];
        }
        const int64_t row = (int64_t)b * a.Hq + (int64_t)g * G + h;
        if (nch == 1) {
            a.out[row * D + d] = __float2half(o * (1.0f / (lh + 1e-6f)));
        } else {
            const int64_t prow = (int64_t)widx * a.Hq + (int64_t)g * G + h;
            a.part_o[prow * D + d] = o;
            if (d == 0) {
                a.part_ml[prow * 2] = mh;
                a.part_ml[prow * 2 + 1] = lh;
            }
        }
    }
}

struct MergeArgs {
    const float *part_o;
    const float *part_ml;
    __half      *out;
    AttnPlan     plan;
    int          Hq;
    int          D;
};

// One wave per (entry b, query head h): log-sum-exp merge of the chunks.
__global__ __launch_bounds__(64) void attn_merge_kernel(MergeArgs a) {
    const int b = blockIdx.x;
    const int h = blockIdx.y;
    const int lane = threadIdx.x;
    const AttnPlan &pl = a.plan;
    const int nch = pl.part_base ? pl.part_base[b + 1] - pl.part_base[b] : pl.nchunk;
    if (nch == 1) return; // written by attn_chunk_kernel
    if (nch == 0) {       // empty sequence: zero row
        for (int d = lane; d < a.D; d += 64) a.out[((int64_t)b * a.Hq + h) * a.D + d] = __float2half(0.0f);
        return;
    }
    const int     w0 = pl.part_base ? pl.part_base[b] : b * pl.nchunk;
    const int64_t cstride = (int64_t)a.Hq; // rows between consecutive chunks
    const float  *ml = a.part_ml + ((int64_t)w0 * a.Hq + h) * 2;

    float mx = -INFINITY;
    for (int c = lane; c < nch; c += 64) mx = fmaxf(mx, ml[c * cstride * 2]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));

    constexpr int kMaxPer = 4; // D <= 256
    float         o[kMaxPer] = {0.0f, 0.0f, 0.0f, 0.0f};
    float         l = 0.0f;
    const float  *po = a.part_o + ((int64_t)w0 * a.Hq + h) * a.D;
    for (int c = 0; c < nch; ++c) {
        const float wgt = __builtin_amdgcn_exp2f(ml[c * cstride * 2] - mx);
        l += ml[c * cstride * 2 + 1] * wgt;
        const float *src = po + (int64_t)c * cstride * a.D;
#pragma unroll
        for (int e = 0; e < kMaxPer; ++e) {
            const int d = lane + 64 * e;
            if (d < a.D) o[e] = fmaf(wgt, src[d], o[e]);
        }
    }
    const float inv = 1.0f / (l + 1e-6f);
    __half     *dst = a.out + ((int64_t)b * a.Hq + h) * a.D;
#pragma unroll
    for (int e = 0; e < kMaxPer; ++e) {
        const int d = lane + 64 * e;
        if (d < a.D) dst[d] = __float2half(o[e] * inv);
    }
}

template <int D, int G>
void launch_chunk(const AttnArgs &args, int n_work, int Hkv, hipStream_t stream) {
    dim3 grid((unsigned)n_work, (unsigned)Hkv);
    hipLaunchKernelGGL((attn_chunk_kernel<D, G>), grid, dim3(kThreads), 0, stream, args);
}

template <int D>
void launch_chunk_g(const AttnArgs &args, int n_work, int Hkv, int G, hipStream_t stream) {
    switch (G) {
    case 1: launch_chunk<D, 1>(args, n_work, Hkv, stream); break;
    case 2: launch_chunk<D, 2>(args, n_work, Hkv, stream); break;
    case 4: launch_chunk<D, 4>(args, n_work, Hkv, stream); break;
    case 8: launch_chunk<D, 8>(args, n_work, Hkv, stream); break;
    default: break;
    }
}

} // namespace

bool attn_shape_supported(int D, int G) {
    return (D == 32 || D == 64 || D == 128 || D == 256) && (G == 1 || G == 2 || G == 4 || G == 8);
}

size_t attn_workspace_floats(int n_work, int Hq, int D) {
    return (size_t)n_work * (size_t)Hq * (size_t)(D + 2);
}

int choose_chunk(const int32_t *lens, int n, int num_kv_heads, int uniform_len) {
    if (const char *env = std::getenv("TL_ATTN_CHUNK")) {
        int c = std::atoi(env);
        if (c >= 64 && c <= kChunkMax && c % 64 == 0) return c;
    }
    // Largest chunk that still yields >= ~8 workgroups per CU on 256 CUs.
    constexpr long kTargetWgs = 2048;
    int            chunk = kChunkMax;
    while (chunk > 64) {
        long items = 0;
        if (lens) {
            for (int i = 0; i < n; ++i) items += (lens[i] + chunk - 1) / chunk;
        } else {
            items = (long)n * ((uniform_len + chunk - 1) / chunk);
        }
        if (items * num_kv_heads >= kTargetWgs) break;
        chunk >>= 1;
    }
    return chunk;
}

void launch_attn_decode(const __half *q, const KvView &kv, const AttnPlan &plan, int B, int Hq,
                        int Hkv, int D, float scale, __half *out, float *part, hipStream_t stream) {
    const int G = Hq / Hkv;
    if (plan.n_work <= 0) return;
    AttnArgs args;
    args.q = q;
    args.out = out;
    args.part_o = part;
    args.part_ml = part ? part + (size_t)plan.n_work * Hq * D : nullptr;
    args.kv = kv;
    args.plan = plan;
    args.Hq = Hq;
    args.scale_log2 = scale * 1.4426950408889634f;

    profile_begin(KernelId::AttnChunk, stream);
    switch (D) {
    case 32: launch_chunk_g<32>(args, plan.n_work, Hkv, G, stream); break;
    case 64: launch_chunk_g<64>(args, plan.n_work, Hkv, G, stream); break;
    case 128: launch_chunk_g<128>(args, plan.n_work, Hkv, G, stream); break;
    case 256: launch_chunk_g<256>(args, plan.n_work, Hkv, G, stream); break;
    default: break;
    }
    HIP_CHECK(hipGetLastError());
    profile_end(KernelId::AttnChunk, stream);

    if (plan.any_multi || plan.any_empty) {
        MergeArgs m;
        m.part_o = args.part_o;
        m.part_ml = args.part_ml;
        m.out = out;
        m.plan = plan;
        m.Hq = Hq;
        m.D = D;
        profile_begin(KernelId::AttnMerge, stream);
        hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)B, (unsigned)Hq), dim3(64), 0, stream, m);
        HIP_CHECK(hipGetLastError());
        profile_end(KernelId::AttnMerge, stream);
    }
}

} // namespace detail
} // namespace tiny_llm
