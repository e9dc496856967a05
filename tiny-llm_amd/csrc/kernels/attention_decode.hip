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
// chunk of <= 512 tokens); each wave owns a contiguous quarter of the chunk
// and runs its own two-pass softmax over it, so waves never wait for each
// other until the final combine.  The G query heads of the group share every
// K/V byte: K and V rows are loaded once from HBM into VGPRs and used for all
// G heads.
//   phase 1  scores.  Default: MFMA v_mfma_f32_16x16x32_f16 with q as the A
//            operand (16 rows = query heads, G of them non-zero) and 16 cached
//            K rows as B (each lane loads 16 contiguous bytes of one token
//            row per k-step); the 16x16 fp32 result holds 16 tokens x G heads
//            with no cross-lane reduction.  Alternative (TL_ATTN_QK=valu):
//            v_dot2_f32_f16 over 8 lanes per token + DPP reduction.
//            Scores are scaled by scale*log2(e) so exp(s - m) = exp2(s' - m')
//            (v_exp_f32; the change of base, no CUDA math routine).
//   softmax  per-wave max over its tokens (DPP row rotations), p = exp2(s-m)
//            rounded to fp16 and stored in LDS pair-interleaved:
//            (p[h][t], p[h][t+TPI]) as one half2 per head; l = sum of the
//            rounded p, so the normaliser matches the weights used.
//   phase 2  P.V with v_dot2_f32_f16 on token pairs: a lane holds 8 dims of
//            tokens t and t+TPI (two 16-byte loads), v_perm_b32 interleaves
//            them into half2 (v[t][d], v[t+TPI][d]), one dot2 per (head, dim)
//            consumes two tokens.
//   combine  waves merged in LDS with 2^(m_w - m) weights; an entry whose
//            sequence fits in one chunk is normalised and written as fp16,
//            otherwise (m, l, o[D]) partials go to the workspace and
//            attn_merge_kernel combines the chunks.
//   append   (decode calls) the workgroup holding the last chunk of entry b
//            first copies the new token's K/V row of head g into the cache at
//            position S_b - 1 -- the bytes of appendKV(n=1) -- then reads it
//            like any other token.
//
// Every global load uses a token index clamped into [0, n) of its chunk, so
// no load leaves the attended range; masked tokens get p = 0.
#include "kv_kernels.h"

#include "tiny_llm/hip_utils.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

namespace tiny_llm {
namespace detail {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTokPerWaveMax = kChunkMax / kWaves; // 128

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));

struct AttnArgs {
    const __half *q;
    __half       *out;
    float        *part_o;  // [n_work][Hq][D]
    float        *part_ml; // [n_work][Hq][2]
    const __half *new_k;   // fused append source [B][Hkv][D] or null
    const __half *new_v;
    KvView        kv;
    AttnPlan      plan;
    int           Hq;
    int           Hkv;
    float         scale_log2; // scale * log2(e)
};

// Byte addressing of the token rows of one (entry, kv head).
template <bool PAGED>
struct RowAddr {
    const char    *kbase; // K of head g (and of the entry's block when not paged)
    const char    *vbase;
    const int32_t *bt_row;
    int64_t        blk_bytes;
    uint32_t       tok_bytes;
    int            log2_blk;
    uint32_t       mask;

    __device__ __forceinline__ RowAddr(const KvView &v, int b, int g) {
        const int     row = v.seq_row ? v.seq_row[b] : b;
        const int64_t head = (int64_t)g * v.head_stride * 2;
        blk_bytes = v.blk_stride * 2;
        tok_bytes = (uint32_t)(v.tok_stride * 2);
        log2_blk = v.log2_blk;
        mask = (1u << v.log2_blk) - 1u;
        if constexpr (PAGED) {
            bt_row = v.block_table + (int64_t)row * v.bt_stride;
            kbase = reinterpret_cast<const char *>(v.k_base) + head;
            vbase = reinterpret_cast<const char *>(v.v_base) + head;
        } else {
            bt_row = nullptr;
            kbase = reinterpret_cast<const char *>(v.k_base) + head + (int64_t)row * blk_bytes;
            vbase = reinterpret_cast<const char *>(v.v_base) + head + (int64_t)row * blk_bytes;
        }
    }
    // Base of the block holding token t0 (t0 wave-uniform); tokens of one
    // 16-aligned group share it.
    __device__ __forceinline__ int64_t block_off(int t0) const {
        if constexpr (PAGED) {
            const int j = __builtin_amdgcn_readfirstlane(t0 >> log2_blk);
            return (int64_t)bt_row[j] * blk_bytes;
        } else {
            return 0;
        }
    }
    __device__ __forceinline__ uint32_t in_block(int t) const {
        if constexpr (PAGED) return ((uint32_t)t & mask) * tok_bytes;
        else return (uint32_t)t * tok_bytes;
    }
    // Per-lane full offset (token may lie in any block).
    __device__ __forceinline__ int64_t lane_off(int t) const {
        if constexpr (PAGED) return (int64_t)bt_row[t >> log2_blk] * blk_bytes + in_block(t);
        else return in_block(t);
    }
};

__device__ __forceinline__ uint4 ld16(const char *p) { return *reinterpret_cast<const uint4 *>(p); }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Streaming load of cache bytes that are read once per call: the
// non-temporal hint keeps them from displacing reusable lines in L2 / MALL.
__device__ __forceinline__ uint4 ld16nt(const char *p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc,
                                  false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, false));
}
// Reductions over the 16 lanes of a DPP row (row_ror 8, 4, 2, 1).
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp_f<0x128>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x122>(v));
    v = fmaxf(v, dpp_f<0x121>(v));
    return v;
}
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f<0x128>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x122>(v);
    v += dpp_f<0x121>(v);
    return v;
}
__device__ __forceinline__ uint16_t f2h_bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ __forceinline__ float h_bits2f(uint16_t x) { return (float)__builtin_bit_cast(_Float16, x); }

// Shared memory of one workgroup.
template <int D, int G>
struct Smem {
    uint16_t pp[kWaves][kTokPerWaveMax * G]; // fp16 p, pair-interleaved per wave
    float    o[kWaves][G * D];               // per-wave P.V partial
    float    m[kWaves][G];
    float    l[kWaves][G];
};

// Index (in halves) of p[h][t] in the pair-interleaved layout of a wave:
// tokens t = 2*TPI*blk + hi*TPI + q pair up as (q, hi = 0/1).
template <int G, int TPI>
__device__ __forceinline__ int pp_index(int t, int h) {
    const int blk = t / (2 * TPI);
    const int r = t - blk * 2 * TPI;
    const int q = r % TPI;
    const int hi = r / TPI;
    return ((blk * TPI + q) * G + h) * 2 + hi;
}

// ---------------------------------------------------------------- phase 1
// Both variants leave, for the wave: pp (fp16 p), s.m[wave][h], s.l[wave][h].

template <int D, int G, bool PAGED>
__device__ __forceinline__ void scores_mfma(const AttnArgs &a, const RowAddr<PAGED> &ra, Smem<D, G> &s,
                                            int b, int g, int t0, int n, int wt0, int tpw, int lane,
                                            int wave) {
    constexpr int KS = D / 32;         // k-steps of 32 dims
    constexpr int TPI = 64 / (D / 8);  // phase-2 tokens per step
    constexpr int NG = kTokPerWaveMax / 16;
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    // A = q: row r16 = head, k = 32*s + 8*kq .. +8
    f16x8 qa[KS];
    {
        const __half *qp = a.q + ((int64_t)b * a.Hq + (int64_t)g * G + r16) * D + 8 * kq;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (r16 < G) v = *reinterpret_cast<const uint4 *>(qp + 32 * ks);
            qa[ks] = __builtin_bit_cast(f16x8, v);
        }
    }
    f32x4 sc[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) sc[j] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};

    // Groups of 16 tokens; loads of 2 groups in flight per batch.
#pragma unroll
    for (int j0 = 0; j0 < NG; j0 += 2) {
        if (j0 * 16 < tpw && wt0 + j0 * 16 < n) {
            uint4 kr[2][KS];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int gs = wt0 + (j0 + u) * 16; // group start (chunk-local)
                const int tl = gs + r16;
                const int tc = tl < n ? tl : n - 1;
                const int gsc = gs < n ? gs : n - 1;
                const char *base = ra.kbase + ra.block_off(t0 + gsc);
                const uint32_t off = ra.in_block(t0 + tc) + 16u * kq;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) kr[u][ks] = ld16(base + off + 64u * ks);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                if ((j0 + u) * 16 < tpw) {
                    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks)
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[ks], __builtin_bit_cast(f16x8, kr[u][ks]),
                                                                     acc, 0, 0, 0);
                    const int tl = wt0 + (j0 + u) * 16 + r16;
                    const bool ok = tl < n;
#pragma unroll
                    for (int i = 0; i < 4; ++i) sc[j0 + u][i] = ok ? acc[i] * a.scale_log2 : -INFINITY;
                }
            }
        }
    }
    // acc[i] of lane (kq, r16) = score of head 4*kq + i for token r16 of the group.
    float mh[4], lh[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < NG; ++j) m = fmaxf(m, sc[j][i]);
        mh[i] = row_max16(m);
        lh[i] = 0.0f;
    }
    uint16_t *pp = s.pp[wave];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        if (j * 16 < tpw) {
            const int tw = j * 16 + r16; // wave-local token
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int h = 4 * kq + i;
                if (h < G) {
                    const float    p = sc[j][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[j][i] - mh[i]);
                    const uint16_t ph = f2h_bits(p);
                    lh[i] += h_bits2f(ph);
                    pp[pp_index<G, TPI>(tw, h)] = ph;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float l = row_sum16(lh[i]);
        const int   h = 4 * kq + i;
        if (r16 == 0 && h < G) {
            s.m[wave][h] = mh[i];
            s.l[wave][h] = l;
        }
    }
}

// Sum over the LPR lanes that hold one token row (LPR = 4, 8, 16 or 32).
template <int LPR>
__device__ __forceinline__ float row_reduce_sum(float v) {
    v += dpp_f<0xB1>(v);                              // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);                              // quad_perm [2,3,0,1]
    if constexpr (LPR >= 8) v += dpp_f<0x141>(v);     // row_half_mirror
    if constexpr (LPR >= 16) v += dpp_f<0x140>(v);    // row_mirror
    if constexpr (LPR >= 32) v += __shfl_xor(v, 16);
    return v;
}

// Phase 1 on the VALU with the load pattern of phase 2: LPR = D/8 lanes per
// token row, 16 contiguous bytes (8 dims) per lane, TPI = 64/LPR rows per
// load instruction, non-temporal.  Each lane dots its 8 dims with the G
// query heads (v_dot2_f32_f16), the row's LPR lanes are summed with DPP, and
// lane p of the row keeps the score of heads h with h % LPR == p.
template <int D, int G, bool PAGED>
__device__ __forceinline__ void scores_rows(const AttnArgs &a, const RowAddr<PAGED> &ra, Smem<D, G> &s,
                                            int b, int g, int t0, int n, int wt0, int tpw, int lane,
                                            int wave) {
    constexpr int LPR = D / 8;
    constexpr int TPI = 64 / LPR;
    constexpr int NSTEP = kTokPerWaveMax / TPI;
    constexpr int HPL = (G + LPR - 1) / LPR; // heads owned per lane
    constexpr int SB = NSTEP < 8 ? NSTEP : 8; // steps per load batch
    const int     r = lane / LPR;
    const int     p = lane % LPR;
    uint4         qv[G];
    {
        const __half *qb = a.q + ((int64_t)b * a.Hq + (int64_t)g * G) * D + 8 * p;
#pragma unroll
        for (int h = 0; h < G; ++h) qv[h] = *reinterpret_cast<const uint4 *>(qb + h * D);
    }
    float sc[HPL][NSTEP];
#pragma unroll
    for (int hh = 0; hh < HPL; ++hh)
#pragma unroll
        for (int i = 0; i < NSTEP; ++i) sc[hh][i] = -INFINITY;

#pragma unroll
    for (int s0 = 0; s0 < NSTEP; s0 += SB) {
        if (s0 * TPI < tpw && wt0 + s0 * TPI < n) {
            uint4 kr[SB];
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                const int   ss = wt0 + (s0 + u) * TPI; // step start (chunk-local)
                const int   ssc = ss < n ? ss : n - 1;
                const int   tl = ss + r;
                const int   tc = tl < n ? tl : n - 1;
                const char *base = ra.kbase + ra.block_off(t0 + ssc);
                kr[u] = ld16nt(base + ra.in_block(t0 + tc) + 16 * p);
            }
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                if ((s0 + u) * TPI < tpw) {
                    float mine[HPL];
#pragma unroll
                    for (int hh = 0; hh < HPL; ++hh) mine[hh] = 0.0f;
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        float d = fdot2(qv[h].x, kr[u].x, 0.0f);
                        d = fdot2(qv[h].y, kr[u].y, d);
                        d = fdot2(qv[h].z, kr[u].z, d);
                        d = fdot2(qv[h].w, kr[u].w, d);
                        d = row_reduce_sum<LPR>(d);
                        if (h % LPR == p) mine[h / LPR] = d;
                    }
                    const bool ok = wt0 + (s0 + u) * TPI + r < n;
#pragma unroll
                    for (int hh = 0; hh < HPL; ++hh)
                        sc[hh][s0 + u] = ok ? mine[hh] * a.scale_log2 : -INFINITY;
                }
            }
        }
    }
    // per-head max / sum over the wave: across the rows r for a fixed p
    uint16_t *pp = s.pp[wave];
#pragma unroll
    for (int hh = 0; hh < HPL; ++hh) {
        const int h = hh * LPR + p;
        float     m = -INFINITY;
#pragma unroll
        for (int i = 0; i < NSTEP; ++i) m = fmaxf(m, sc[hh][i]);
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        float l = 0.0f;
        if (h < G) {
#pragma unroll
            for (int i = 0; i < NSTEP; ++i) {
                if (i * TPI < tpw) {
                    const float    pv = sc[hh][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[hh][i] - m);
                    const uint16_t ph = f2h_bits(pv);
                    l += h_bits2f(ph);
                    // token i*TPI + r: pair block i/2, half i%2, q = r
                    pp[(((i >> 1) * TPI + r) * G + h) * 2 + (i & 1)] = ph;
                }
            }
        }
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) l += __shfl_xor(l, off);
        if (r == 0 && h < G) {
            s.m[wave][h] = m;
            s.l[wave][h] = l;
        }
    }
}

// ---------------------------------------------------------------- kernel
template <int D, int G, bool PAGED, bool MFMA>
__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(AttnArgs a) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group size");
    static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head_dim");
    constexpr int LPT = D / 8;    // phase-2 lanes per token (8 dims each)
    constexpr int TPI = 64 / LPT; // phase-2 tokens per wave step
    __shared__ Smem<D, G> s;

    const int       lane = threadIdx.x & 63;
    const int       wave = threadIdx.x >> 6;
    const AttnPlan &pl = a.plan;
    // 1-D grid, kv head fastest: the Hkv workgroups that read the pieces of
    // the same token rows are dispatched together (one per XCD when Hkv = 8).
    const int       item = blockIdx.x / a.Hkv;
    const int       g = blockIdx.x - item * a.Hkv;
    int             b, c;
    if (pl.work) {
        b = pl.work[2 * item];
        c = pl.work[2 * item + 1];
    } else {
        b = item / pl.nchunk;
        c = item - b * pl.nchunk;
    }
    const int S = pl.seq_lens ? pl.seq_lens[b] : pl.uniform_len;
    const int nch = pl.part_base ? pl.part_base[b + 1] - pl.part_base[b] : pl.nchunk;
    const int widx = pl.part_base ? pl.part_base[b] + c : item;
    const int t0 = c * pl.chunk;
    const int n = min(pl.chunk, S - t0); // >= 1 by construction of the plan
    const int tpw = pl.chunk / kWaves;   // multiple of 16
    const int wt0 = wave * tpw;

    const RowAddr<PAGED> ra(a.kv, b, g);

    if (a.new_k && c == nch - 1) {
        // Fused appendKV(n=1) of head g at position S-1 (same bytes as the
        // D2D copies of kv_cache.cpp:230-233).
        constexpr int P = D / 8; // 16-byte pieces per head row
        const int     tid = threadIdx.x;
        if (tid < 2 * P) {
            const int      which = tid / P, e = tid - which * P;
            const __half  *src = (which ? a.new_v : a.new_k) + ((int64_t)b * a.Hkv + g) * D + e * 8;
            const char    *base = which ? ra.vbase : ra.kbase;
            char          *dst = const_cast<char *>(base) + ra.lane_off(S - 1) + 16 * e;
            *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(src);
        }
        __threadfence_block();
        __syncthreads();
    }

    // ---------------- phase 1 + per-wave softmax ----------------
    const bool active = wt0 < n; // wave has tokens
    if (active) {
        if constexpr (MFMA) scores_mfma<D, G, PAGED>(a, ra, s, b, g, t0, n, wt0, tpw, lane, wave);
        else scores_rows<D, G, PAGED>(a, ra, s, b, g, t0, n, wt0, tpw, lane, wave);
    } else if (lane < G) {
        s.m[wave][lane] = -INFINITY;
        s.l[wave][lane] = 0.0f;
    }

    // ---------------- phase 2: P.V on token pairs ----------------
    const int tq = lane / LPT;
    const int dg = lane % LPT;
    float     acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;

    if (active) {
        // pp was written by other lanes of this wave.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        constexpr int NB = kTokPerWaveMax / (2 * TPI); // pair blocks per wave
        constexpr int BB = NB < 4 ? NB : 4;            // blocks per load batch
        const uint16_t *pp = s.pp[wave];
        constexpr bool uniform_blk = (2 * TPI <= 16);  // a pair block sits in one 16-token block
#pragma unroll
        for (int jb = 0; jb < NB; jb += BB) {
            if (jb * 2 * TPI < tpw && wt0 + jb * 2 * TPI < n) {
                uint4 va[BB], vb[BB];
#pragma unroll
                for (int u = 0; u < BB; ++u) {
                    const int bs = wt0 + (jb + u) * 2 * TPI; // block start (chunk-local)
                    const int ta = bs + tq, tb = bs + TPI + tq;
                    const int tca = ta < n ? ta : n - 1, tcb = tb < n ? tb : n - 1;
                    if constexpr (uniform_blk) {
                        const int   bsc = bs < n ? bs : n - 1;
                        const char *base = ra.vbase + ra.block_off(t0 + bsc);
                        va[u] = ld16nt(base + ra.in_block(t0 + tca) + 16 * dg);
                        vb[u] = ld16nt(base + ra.in_block(t0 + tcb) + 16 * dg);
                    } else {
                        va[u] = ld16nt(ra.vbase + ra.lane_off(t0 + tca) + 16 * dg);
                        vb[u] = ld16nt(ra.vbase + ra.lane_off(t0 + tcb) + 16 * dg);
                    }
                }
#pragma unroll
                for (int u = 0; u < BB; ++u) {
                    if ((jb + u) * 2 * TPI < tpw) {
                        // p pairs of the G heads for (block jb+u, q = tq)
                        uint32_t pw[G];
                        const uint32_t *src = reinterpret_cast<const uint32_t *>(pp) + ((jb + u) * TPI + tq) * G;
                        if constexpr (G >= 4) {
#pragma unroll
                            for (int h4 = 0; h4 < G; h4 += 4) {
                                const uint4 v = *reinterpret_cast<const uint4 *>(src + h4);
                                pw[h4] = v.x;
                                pw[h4 + 1] = v.y;
                                pw[h4 + 2] = v.z;
                                pw[h4 + 3] = v.w;
                            }
                        } else if constexpr (G == 2) {
                            const uint2 v = *reinterpret_cast<const uint2 *>(src);
                            pw[0] = v.x;
                            pw[1] = v.y;
                        } else {
                            pw[0] = src[0];
                        }
                        const uint32_t wa[4] = {va[u].x, va[u].y, va[u].z, va[u].w};
                        const uint32_t wb[4] = {vb[u].x, vb[u].y, vb[u].z, vb[u].w};
                        uint32_t       vp[8]; // (v[ta][d], v[tb][d]) for the lane's 8 dims
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            vp[2 * i] = __builtin_amdgcn_perm(wb[i], wa[i], 0x05040100u);
                            vp[2 * i + 1] = __builtin_amdgcn_perm(wb[i], wa[i], 0x07060302u);
                        }
#pragma unroll
                        for (int h = 0; h < G; ++h)
#pragma unroll
                            for (int e = 0; e < 8; ++e) acc[h][e] = fdot2(pw[h], vp[e], acc[h][e]);
                    }
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
    }
    if (tq == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float *dst = &s.o[wave][h * D + dg * 8];
            *reinterpret_cast<float4 *>(dst) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
            *reinterpret_cast<float4 *>(dst + 4) = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
    }
    __syncthreads();

    // ---------------- combine waves, emit ----------------
    for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
        const int h = idx / D;
        const int d = idx - h * D;
        float     mh = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mh = fmaxf(mh, s.m[w][h]);
        float o = 0.0f, lh = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wgt = s.m[w][h] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s.m[w][h] - mh);
            o = fmaf(wgt, s.o[w][h * D + d], o);
            lh = fmaf(wgt, s.l[w][h], lh);
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
    const float   *part_o;  // [n_work][Hq][D]
    const float   *part_ml; // [n_work][Hq][2]
    __half        *out;
    const int32_t *part_base;
    int            nchunk;
    int            Hq;
    int            Hkv;
};

constexpr int kMergeMaxChunks = 64;

// One workgroup per (entry b, kv head g): log-sum-exp merge of the chunk
// partials of the G query heads,
//   m* = max m_c, l = sum l_c 2^(m_c-m*), o = sum o_c 2^(m_c-m*) / (l+1e-6).
// The chunk weights go through LDS; every thread then issues the o loads of
// all chunks back to back.  Entries with no tokens get a zero row.
template <int D, int G>
__global__ __launch_bounds__(256) void attn_merge_kernel(MergeArgs a) {
    __shared__ float s_w[kMergeMaxChunks][G];
    __shared__ float s_m[G], s_l[G];
    const int        b = blockIdx.x / a.Hkv;
    const int        g = blockIdx.x - b * a.Hkv;
    const int        nch = a.part_base ? a.part_base[b + 1] - a.part_base[b] : a.nchunk;
    __half          *dst = a.out + ((int64_t)b * a.Hq + (int64_t)g * G) * D;
    if (nch == 1) return; // written by attn_chunk_kernel
    if (nch == 0) {
        for (int i = threadIdx.x; i < G * D; i += 256) dst[i] = __float2half(0.0f);
        return;
    }
    const int w0 = a.part_base ? a.part_base[b] : b * a.nchunk;
    for (int c0 = 0; c0 < nch; c0 += kMergeMaxChunks) {
        const int cn = min(kMergeMaxChunks, nch - c0);
        for (int i = threadIdx.x; i < cn * G; i += 256) {
            const int c = i / G, h = i - c * G;
            s_w[c][h] = a.part_ml[((int64_t)(w0 + c0 + c) * a.Hq + (int64_t)g * G + h) * 2];
        }
        __syncthreads();
        if (threadIdx.x < G) { // running max and sum of head threadIdx.x
            const int h = threadIdx.x;
            float     mx = c0 ? s_m[h] : -INFINITY, mnew = mx;
            for (int c = 0; c < cn; ++c) mnew = fmaxf(mnew, s_w[c][h]);
            float l = c0 ? s_l[h] * __builtin_amdgcn_exp2f(mx - mnew) : 0.0f;
            for (int c = 0; c < cn; ++c) {
                const float wgt = __builtin_amdgcn_exp2f(s_w[c][h] - mnew);
                l = fmaf(wgt, a.part_ml[((int64_t)(w0 + c0 + c) * a.Hq + (int64_t)g * G + h) * 2 + 1], l);
                s_w[c][h] = wgt;
            }
            s_l[h] = l;
            s_m[h] = mnew;
        }
        __syncthreads();
        if (c0 == 0 && nch <= kMergeMaxChunks) {
            for (int idx = threadIdx.x; idx < G * D; idx += 256) {
                const int     h = idx / D;
                const float  *po = a.part_o + ((int64_t)w0 * a.Hq + (int64_t)g * G) * D + idx;
                const int64_t rs = (int64_t)a.Hq * D;
                float         o = 0.0f;
#pragma unroll 16
                for (int c = 0; c < cn; ++c) o = fmaf(s_w[c][h], po[c * rs], o);
                dst[idx] = __float2half(o * (1.0f / (s_l[h] + 1e-6f)));
            }
            return;
        }
        __syncthreads();
    }
    // More than kMergeMaxChunks chunks: weights relative to the final max.
    for (int idx = threadIdx.x; idx < G * D; idx += 256) {
        const int     h = idx / D;
        const float  *ml = a.part_ml + ((int64_t)w0 * a.Hq + (int64_t)g * G + h) * 2;
        const float  *po = a.part_o + ((int64_t)w0 * a.Hq + (int64_t)g * G) * D + idx;
        const int64_t rs = (int64_t)a.Hq;
        float         o = 0.0f;
        for (int c = 0; c < nch; ++c)
            o = fmaf(__builtin_amdgcn_exp2f(ml[c * rs * 2] - s_m[h]), po[c * rs * D], o);
        dst[idx] = __float2half(o * (1.0f / (s_l[h] + 1e-6f)));
    }
}

template <int D>
void launch_merge_g(const MergeArgs &m, int B, int Hkv, int G, hipStream_t stream) {
    const dim3 grid((unsigned)(B * Hkv));
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_merge_kernel<D, 1>), grid, dim3(256), 0, stream, m); break;
    case 2: hipLaunchKernelGGL((attn_merge_kernel<D, 2>), grid, dim3(256), 0, stream, m); break;
    case 4: hipLaunchKernelGGL((attn_merge_kernel<D, 4>), grid, dim3(256), 0, stream, m); break;
    case 8: hipLaunchKernelGGL((attn_merge_kernel<D, 8>), grid, dim3(256), 0, stream, m); break;
    default: break;
    }
}

template <int D, int G>
void launch_chunk(const AttnArgs &args, int n_work, int Hkv, bool paged, bool mfma, hipStream_t stream) {
    dim3 grid((unsigned)n_work * (unsigned)Hkv);
    if (paged) {
        if (mfma) hipLaunchKernelGGL((attn_chunk_kernel<D, G, true, true>), grid, dim3(kThreads), 0, stream, args);
        else hipLaunchKernelGGL((attn_chunk_kernel<D, G, true, false>), grid, dim3(kThreads), 0, stream, args);
    } else {
        if (mfma) hipLaunchKernelGGL((attn_chunk_kernel<D, G, false, true>), grid, dim3(kThreads), 0, stream, args);
        else hipLaunchKernelGGL((attn_chunk_kernel<D, G, false, false>), grid, dim3(kThreads), 0, stream, args);
    }
}

template <int D>
void launch_chunk_g(const AttnArgs &args, int n_work, int Hkv, int G, bool paged, bool mfma,
                    hipStream_t stream) {
    switch (G) {
    case 1: launch_chunk<D, 1>(args, n_work, Hkv, paged, mfma, stream); break;
    case 2: launch_chunk<D, 2>(args, n_work, Hkv, paged, mfma, stream); break;
    case 4: launch_chunk<D, 4>(args, n_work, Hkv, paged, mfma, stream); break;
    case 8: launch_chunk<D, 8>(args, n_work, Hkv, paged, mfma, stream); break;
    default: break;
    }
}

// Score variant: VALU rows unless TL_ATTN_QK=mfma.
bool use_mfma_scores() {
    static const bool mfma = [] {
        const char *e = std::getenv("TL_ATTN_QK");
        return e && std::strcmp(e, "mfma") == 0;
    }();
    return mfma;
}

} // namespace

bool attn_shape_supported(int D, int G) {
    return (D == 32 || D == 64 || D == 128 || D == 256) && (G == 1 || G == 2 || G == 4 || G == 8);
}

size_t attn_workspace_floats(int n_work, int Hq, int D) {
    return (size_t)n_work * (size_t)Hq * (size_t)(D + 2);
}

int choose_chunk(const int32_t *lens, int n, int num_kv_heads, int uniform_len, int head_dim) {
    // A wave's quarter of the chunk must hold whole pair blocks of 2*TPI
    // tokens (TPI = 512 / head_dim) and whole 16-token score groups.
    const int min_chunk = std::max(64, kWaves * 2 * (512 / head_dim));
    if (const char *env = std::getenv("TL_ATTN_CHUNK")) {
        const int c = std::atoi(env);
        if (c >= min_chunk && c <= kChunkMax && c % min_chunk == 0) return c;
    }
    // Largest chunk that still yields >= ~8 workgroups per CU on 256 CUs.
    constexpr long kTargetWgs = 2048;
    int            chunk = kChunkMax;
    while (chunk > min_chunk) {
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
                        int Hkv, int D, float scale, __half *out, float *part, const __half *new_k,
                        const __half *new_v, hipStream_t stream) {
    const int G = Hq / Hkv;
    if (plan.n_work <= 0 && !plan.any_empty) return;
    AttnArgs args;
    args.q = q;
    args.out = out;
    args.part_o = part;
    args.part_ml = part ? part + (size_t)plan.n_work * Hq * D : nullptr;
    args.new_k = new_k;
    args.new_v = new_v;
    if (plan.any_multi && !part)
        throw std::invalid_argument("attention: a multi-chunk plan needs the partials workspace");
    args.kv = kv;
    args.plan = plan;
    args.Hq = Hq;
    args.Hkv = Hkv;
    args.scale_log2 = scale * 1.4426950408889634f;
    const bool paged = kv.block_table != nullptr;
    const bool mfma = use_mfma_scores();
    if (plan.chunk % std::max(64, kWaves * 2 * (512 / D)) != 0 || plan.chunk > kChunkMax)
        throw std::invalid_argument("attention: chunk length does not fit the head size");
    if (!paged && (int64_t)plan.max_len * kv.tok_stride * 2 > (int64_t)UINT32_MAX)
        throw std::invalid_argument("attention: token offsets exceed 32 bits (max_len * row bytes)");

    if (plan.n_work > 0) {
        profile_begin(KernelId::AttnChunk, stream);
        switch (D) {
        case 32: launch_chunk_g<32>(args, plan.n_work, Hkv, G, paged, mfma, stream); break;
        case 64: launch_chunk_g<64>(args, plan.n_work, Hkv, G, paged, mfma, stream); break;
        case 128: launch_chunk_g<128>(args, plan.n_work, Hkv, G, paged, mfma, stream); break;
        case 256: launch_chunk_g<256>(args, plan.n_work, Hkv, G, paged, mfma, stream); break;
        default: break;
        }
        HIP_CHECK(hipGetLastError());
        profile_end(KernelId::AttnChunk, stream);
    }

    if (plan.any_multi || plan.any_empty) {
        MergeArgs m;
        m.part_o = args.part_o;
        m.part_ml = args.part_ml;
        m.out = out;
        m.part_base = plan.part_base;
        m.nchunk = plan.nchunk;
        m.Hq = Hq;
        m.Hkv = Hkv;
        profile_begin(KernelId::AttnMerge, stream);
        switch (D) {
        case 32: launch_merge_g<32>(m, B, Hkv, G, stream); break;
        case 64: launch_merge_g<64>(m, B, Hkv, G, stream); break;
        case 128: launch_merge_g<128>(m, B, Hkv, G, stream); break;
        case 256: launch_merge_g<256>(m, B, Hkv, G, stream); break;
        default: break;
        }
        HIP_CHECK(hipGetLastError());
        profile_end(KernelId::AttnMerge, stream);
    }
}

} // namespace detail
} // namespace tiny_llm
