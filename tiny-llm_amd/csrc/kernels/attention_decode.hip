// Split-K flash-decoding GQA attention over the KV cache, for gfx950.
//
// Computes, for every batch entry b and query head h (kv head g = h / G):
//   s_t = (q_h . k_{g,t}) * scale,  p_t = exp(s_t - max s),
//   o_h = (sum_t p_t v_{g,t}) / (sum_t p_t + 1e-6)           t in [0, S_b)
// which is the arithmetic of attention_decode_kernel (kernels/attention.cu:
// 11-112: scores, max, expf, 1/(sum+1e-6f), P.V, RNE fp16 output), extended to
// GQA over the token-major cache of kv_cache.cpp:226-233.
//
// Work decomposition.  One workgroup of NW wave64 per work item (entry b, kv
// head g, chunk of the sequence), 8 waves resident per CU: one 8-wave
// workgroup, or two 4-wave workgroups whose ramp-up and drain overlap each
// other's streaming (chosen per launch: 8 waves when every CU gets at most two
// workgroups in turn, 4 waves for longer work lists).  The planner sizes
// chunks so that work items roughly match the resident workgroup slots of the
// device, which for long sequences usually means one chunk per sequence and
// no split-K partials at all (partials are HBM writes interleaved with the
// read stream, which costs far more than their byte count), and orders the
// work list longest first.  Inside a chunk the waves take interleaved 64-token
// tiles (wave w: tiles w, w+NW, ...) and keep a running softmax
// (max m, sum l, o[G][D]) in registers, rescaling by 2^(m_old - m_new) from
// tile to tile.  The G query heads of the group share every K/V byte: each
// K/V row is loaded once into VGPRs and used for all G heads.
//
// Head-fused plans (head_dim 128, near-uniform lengths, planner's choice): an
// 8-wave workgroup takes H = 2, 4 or 8 kv heads of an entry instead of one,
// wave w head w % H and tile slice w / H, so the workgroup reads H heads'
// 256-byte pieces of each token row together (per-head workgroups read them
// from H different CUs).  An entry's nch work items interleave its tiles
// (slice s of item c: tiles c*NS+s, + nch*NS, ... with NS = 8 / H) instead of
// taking chunks, and the planner picks H and nch so that the launch is one
// workgroup per CU; for 64 entries of 8 kv heads on 256 CUs that is H = 2
// and one item per entry, so no partials and no merge launch.
//
// Per tile:
//   loads    K and V rows are read with LPR = D/8 lanes per token row, 16
//            contiguous bytes per lane, TPI = 64/LPR rows per instruction,
//            non-temporal (read once).  Batches are double-buffered: the next
//            batch (and, at phase ends, the first batch of the next phase or
//            tile) is in flight while the current one is consumed.
//   scores   VALU path: v_dot2_f32_f16 of the lane's 8 dims with the G heads,
//            DPP sum over the row's LPR lanes; lane p keeps heads h%LPR == p
//            (16 lanes per row, G >= 2: a transposing DPP reduction, lane p
//            keeps head f(p); see ValuScorer).
//            MFMA path: the K rows of 16 tokens go through a padded LDS tile
//            and are read back in the B layout of v_mfma_f32_16x16x32_f16
//            with q as the A operand (G of its 16 rows non-zero).
//            Scores are scaled by scale*log2(e) so exp(s - m) = exp2(s' - m')
//            (v_exp_f32; the change of base, no CUDA math routine).
//   softmax  tile max per head, new running max, alpha = 2^(m_old - m_new);
//            p = exp2(s - m_new) rounded to fp16 into LDS, pair-interleaved:
//            (p[h][t], p[h][t+TPI]) as one half2 per head; l accumulates the
//            rounded p, so the normaliser matches the weights used.
//   P.V      v_dot2_f32_f16 on token pairs: a lane holds 8 dims of tokens t
//            and t+TPI, v_perm_b32 interleaves them into half2
//            (v[t][d], v[t+TPI][d]); one dot2 per (head, dim) takes two tokens.
//            At head_dim 128 and groups 2-8 (kMfmaPV) instead on MFMA: the
//            V rows go to a two-quarter ring in the wave's LDS as loaded, and
//            per staged 16-token quarter O^T += V^T P^T by
//            v_mfma_f32_16x16x16f16, V^T by the transposing ds_read_b64_tr_b16,
//            P^T from p stored [head][token].  V batches are 8 tokens, 16 for
//            the head-fused chunk items of ragged plans.
// End: per-wave (m, l, o) combined across the NW waves (head-fused: the NS
// waves of each head) in LDS; a work item that
// covers its whole sequence is normalised and written as fp16, otherwise
// (m, l, o[D]) partials go to the workspace and attn_merge_kernel combines
// the chunks: m* = max m_c, l = sum l_c 2^(m_c-m*), o = sum o_c 2^(m_c-m*)/(l+1e-6).
// Append (decode calls): the workgroup holding the last chunk (head-fused: the
// last tile) of entry b first copies the new token's K/V row of head g into
// the cache at position S_b - 1 -- the bytes of appendKV(n=1) -- then reads it
// like any other token.
//
// Every global load uses a token index clamped into its tile's valid range,
// so no load leaves the attended range; masked tokens get p = 0.
#include "kv_kernels.h"

#include "tiny_llm/hip_utils.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace tiny_llm {
namespace detail {

namespace {

// Resident waves per SIMD the kernels ask the register allocator for (8 per
// CU: one 8-wave or two 4-wave workgroups); the planner's slot count is
// expressed in 4-wave workgroups.
constexpr int kWavesPerEU = 2;
constexpr int kTile = 64;             // tokens per wave tile
constexpr int kVmcntAll = 0x0F70;     // s_waitcnt vmcnt(0)
constexpr int kQuantum = kPlanQuantum; // chunk lengths are multiples of this
static_assert(kTile == kPlanTile && kPlanSlotsPerCU == kWavesPerEU, "planner geometry");

// Tuning (compile-time): K load steps per batch, V pair blocks per batch.
#ifndef TL_ATTN_KB
#define TL_ATTN_KB 2
#endif
#ifndef TL_ATTN_VB
#define TL_ATTN_VB 1
#endif

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
    InlineMeta    meta;       // used when meta.n > 0
    // Merge in the launch: one counter per (entry, kv head), zero between
    // launches; the workgroup that completes an entry's last chunk of a head
    // block merges its partials (fused_merge).  Null: attn_merge_kernel does.
    int          *counters;
};
static_assert(sizeof(AttnArgs) <= 4096, "kernel arguments");

// Work item `item` of the launch: entry b, chunk c of nch, attended length
// S, partial row widx and cache row (slot) row, from the inline metadata
// (full or compact encoding, see InlineMeta) or the plan's device arrays.
// A macro, expanded in each kernel body on the by-value kernel argument `a`:
// passing the argument by reference to a function makes the compiler copy
// the whole 3.7 KB struct into per-lane scratch memory.
#define ATTN_WORK_ITEM(a, item, b, c, S, nch, widx, row)                                           \
    do {                                                                                           \
        if ((a).meta.n && (a).meta.compact) { /* one chunk per entry */                            \
            const uint32_t ord_ = (uint32_t)(a).meta.w[(a).meta.off_work + ((item) >> 1)];         \
            b = (int)((ord_ >> (((item) & 1) * 16)) & 0xffffu);                                    \
            const uint32_t e_ = (uint32_t)(a).meta.w[b];                                           \
            S = (int)(e_ & 0xffffu);                                                               \
            row = (int)(e_ >> 16);                                                                 \
            c = 0;                                                                                 \
            nch = 1;                                                                               \
            widx = b;                                                                              \
        } else if ((a).meta.n) { /* full encoding */                                               \
            b = (a).meta.w[(a).meta.off_work + 2 * (item)];                                        \
            c = (a).meta.w[(a).meta.off_work + 2 * (item) + 1];                                    \
            S = (a).meta.w[b];                                                                     \
            const int pb_ = (a).meta.w[(a).meta.off_part + b];                                     \
            nch = (a).meta.w[(a).meta.off_part + b + 1] - pb_;                                     \
            widx = pb_ + c;                                                                        \
            row = (a).meta.has_rows ? (a).meta.w[(a).meta.off_rows + b] : b;                       \
        } else {                                                                                   \
            if ((a).plan.work) {                                                                   \
                b = (a).plan.work[2 * (item)];                                                     \
                c = (a).plan.work[2 * (item) + 1];                                                 \
            } else {                                                                               \
                b = (item) / (a).plan.nchunk;                                                      \
                c = (item) - b * (a).plan.nchunk;                                                  \
            }                                                                                      \
            S = (a).plan.seq_lens ? (a).plan.seq_lens[b] : (a).plan.uniform_len;                   \
            nch = (a).plan.part_base ? (a).plan.part_base[b + 1] - (a).plan.part_base[b]           \
                                     : (a).plan.nchunk;                                            \
            widx = (a).plan.part_base ? (a).plan.part_base[b] + c : (item);                        \
            row = (a).kv.seq_row ? (a).kv.seq_row[b] : b;                                          \
        }                                                                                          \
    } while (0)

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

    __device__ __forceinline__ RowAddr(const KvView &v, int row, int g) {
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
    // Block ids of the four 16-token quarters of one tile [t_first, t_last]
    // (t_first is a multiple of kTile and blocks hold >= 16 tokens, so each
    // quarter lies in one block): lane k < 4 holds the block of token
    // min(t_first + 16k, t_last).  Loaded one tile ahead, so the address
    // arithmetic of the loads never waits on the block table.
    __device__ __forceinline__ int tile_blocks(int t_first, int t_last, int lane) const {
        static_assert(kTile == 64, "four 16-token quarters per tile");
        if constexpr (PAGED) {
            return lane < 4 ? bt_row[min(t_first + 16 * lane, t_last) >> log2_blk] : 0;
        } else {
            return 0;
        }
    }
    // Byte offsets of the quarters' blocks, wave-uniform (scalar registers):
    // four readlanes per tile, after which every load step picks its
    // quarter's offset by a compile-time index.
    struct Quarters {
        int64_t o[4];
    };
    __device__ __forceinline__ Quarters quarters(int btv) const {
        Quarters q;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            q.o[k] = PAGED ? (int64_t)__builtin_amdgcn_readlane(btv, k) * blk_bytes : 0;
        return q;
    }
    __device__ __forceinline__ uint32_t in_block(int t) const {
        if constexpr (PAGED) return ((uint32_t)t & mask) * tok_bytes;
        else return (uint32_t)t * tok_bytes;
    }
    // Per-lane full offset straight from the block table (one-off accesses).
    __device__ __forceinline__ int64_t lane_off(int t) const {
        if constexpr (PAGED) return (int64_t)bt_row[t >> log2_blk] * blk_bytes + in_block(t);
        else return in_block(t);
    }
};

// A global-memory pointer that is the same in every lane, moved to scalar
// registers (its arithmetic then runs on the scalar unit); typed as global so
// that the loads through it stay global loads, not flat ones.
typedef const __attribute__((address_space(1))) char *gptr;
__device__ __forceinline__ gptr uniform_ptr(const char *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<gptr>(((uint64_t)hi << 32) | lo);
}

// Streaming load of cache bytes that are read once per call: the
// non-temporal hint keeps them from displacing reusable lines in L2 / MALL.
__device__ __forceinline__ uint4 ld16nt(gptr p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const __attribute__((address_space(1))) u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc,
                                  false);
}

// The G heads' scores over the lane's 8 fp16 pairs of k, accumulated in fp32
// in pair order: d[h] = dot2(q_h.w, k.w, dot2(q_h.z, k.z, dot2(q_h.y, k.y,
// dot2(q_h.x, k.x, 0)))), as the builtin chains give.  Written out so that
// each chain starts with the three-operand v_dot2_f32_f16 and an inline zero:
// from the builtin the compiler starts every chain with a v_mov of 0 for the
// two-operand accumulating v_dot2c_f32_f16 (one VALU instruction per chain).
// One statement per pair position, the G chains interleaved: a v_dot2c may
// read the v_dot2 result it accumulates only 3 wait states after it, which
// G - 1 >= 3 other instructions provide (an s_nop for G = 2); same-opcode
// v_dot2c chains need none; the closing s_nop covers the compiler's next
// reader of d, which does not see what the statement holds.
template <int G>
__device__ __forceinline__ void dot_heads(const uint4 (&q)[G], const uint4 &k, float (&d)[G]);
template <>
__device__ __forceinline__ void dot_heads<2>(const uint4 (&q)[2], const uint4 &k, float (&d)[2]) {
    asm("v_dot2_f32_f16 %0, %2, %4, 0\n\tv_dot2_f32_f16 %1, %3, %4, 0\n\ts_nop 1"
        : "=&v"(d[0]), "=&v"(d[1])
        : "v"(q[0].x), "v"(q[1].x), "v"(k.x));
    asm("v_dot2c_f32_f16 %0, %2, %4\n\tv_dot2c_f32_f16 %1, %3, %4"
        : "+v"(d[0]), "+v"(d[1])
        : "v"(q[0].y), "v"(q[1].y), "v"(k.y));
    asm("v_dot2c_f32_f16 %0, %2, %4\n\tv_dot2c_f32_f16 %1, %3, %4"
        : "+v"(d[0]), "+v"(d[1])
        : "v"(q[0].z), "v"(q[1].z), "v"(k.z));
    asm("v_dot2c_f32_f16 %0, %2, %4\n\tv_dot2c_f32_f16 %1, %3, %4\n\ts_nop 2"
        : "+v"(d[0]), "+v"(d[1])
        : "v"(q[0].w), "v"(q[1].w), "v"(k.w));
}
template <>
__device__ __forceinline__ void dot_heads<4>(const uint4 (&q)[4], const uint4 &k, float (&d)[4]) {
    asm("v_dot2_f32_f16 %0, %4, %8, 0\n\tv_dot2_f32_f16 %1, %5, %8, 0\n\tv_dot2_f32_f16 %2, %6, %8, 0\n\tv_dot2_f32_f16 %3, %7, %8, 0"
        : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3])
        : "v"(q[0].x), "v"(q[1].x), "v"(q[2].x), "v"(q[3].x), "v"(k.x));
    asm("v_dot2c_f32_f16 %0, %4, %8\n\tv_dot2c_f32_f16 %1, %5, %8\n\tv_dot2c_f32_f16 %2, %6, %8\n\tv_dot2c_f32_f16 %3, %7, %8"
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3])
        : "v"(q[0].y), "v"(q[1].y), "v"(q[2].y), "v"(q[3].y), "v"(k.y));
    asm("v_dot2c_f32_f16 %0, %4, %8\n\tv_dot2c_f32_f16 %1, %5, %8\n\tv_dot2c_f32_f16 %2, %6, %8\n\tv_dot2c_f32_f16 %3, %7, %8"
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3])
        : "v"(q[0].z), "v"(q[1].z), "v"(q[2].z), "v"(q[3].z), "v"(k.z));
    asm("v_dot2c_f32_f16 %0, %4, %8\n\tv_dot2c_f32_f16 %1, %5, %8\n\tv_dot2c_f32_f16 %2, %6, %8\n\tv_dot2c_f32_f16 %3, %7, %8\n\ts_nop 2"
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3])
        : "v"(q[0].w), "v"(q[1].w), "v"(q[2].w), "v"(q[3].w), "v"(k.w));
}
template <>
__device__ __forceinline__ void dot_heads<8>(const uint4 (&q)[8], const uint4 &k, float (&d)[8]) {
    asm("v_dot2_f32_f16 %0, %8, %16, 0\n\tv_dot2_f32_f16 %1, %9, %16, 0\n\tv_dot2_f32_f16 %2, %10, %16, 0\n\tv_dot2_f32_f16 %3, %11, %16, 0\n\tv_dot2_f32_f16 %4, %12, %16, 0\n\tv_dot2_f32_f16 %5, %13, %16, 0\n\tv_dot2_f32_f16 %6, %14, %16, 0\n\tv_dot2_f32_f16 %7, %15, %16, 0"
        : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3]), "=&v"(d[4]), "=&v"(d[5]), "=&v"(d[6]), "=&v"(d[7])
        : "v"(q[0].x), "v"(q[1].x), "v"(q[2].x), "v"(q[3].x), "v"(q[4].x), "v"(q[5].x), "v"(q[6].x), "v"(q[7].x), "v"(k.x));
    asm("v_dot2c_f32_f16 %0, %8, %16\n\tv_dot2c_f32_f16 %1, %9, %16\n\tv_dot2c_f32_f16 %2, %10, %16\n\tv_dot2c_f32_f16 %3, %11, %16\n\tv_dot2c_f32_f16 %4, %12, %16\n\tv_dot2c_f32_f16 %5, %13, %16\n\tv_dot2c_f32_f16 %6, %14, %16\n\tv_dot2c_f32_f16 %7, %15, %16"
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]), "+v"(d[6]), "+v"(d[7])
        : "v"(q[0].y), "v"(q[1].y), "v"(q[2].y), "v"(q[3].y), "v"(q[4].y), "v"(q[5].y), "v"(q[6].y), "v"(q[7].y), "v"(k.y));
    asm("v_dot2c_f32_f16 %0, %8, %16\n\tv_dot2c_f32_f16 %1, %9, %16\n\tv_dot2c_f32_f16 %2, %10, %16\n\tv_dot2c_f32_f16 %3, %11, %16\n\tv_dot2c_f32_f16 %4, %12, %16\n\tv_dot2c_f32_f16 %5, %13, %16\n\tv_dot2c_f32_f16 %6, %14, %16\n\tv_dot2c_f32_f16 %7, %15, %16"
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]), "+v"(d[6]), "+v"(d[7])
        : "v"(q[0].z), "v"(q[1].z), "v"(q[2].z), "v"(q[3].z), "v"(q[4].z), "v"(q[5].z), "v"(q[6].z), "v"(q[7].z), "v"(k.z));
    asm("v_dot2c_f32_f16 %0, %8, %16\n\tv_dot2c_f32_f16 %1, %9, %16\n\tv_dot2c_f32_f16 %2, %10, %16\n\tv_dot2c_f32_f16 %3, %11, %16\n\tv_dot2c_f32_f16 %4, %12, %16\n\tv_dot2c_f32_f16 %5, %13, %16\n\tv_dot2c_f32_f16 %6, %14, %16\n\tv_dot2c_f32_f16 %7, %15, %16\n\ts_nop 2"
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]), "+v"(d[6]), "+v"(d[7])
        : "v"(q[0].w), "v"(q[1].w), "v"(q[2].w), "v"(q[3].w), "v"(q[4].w), "v"(q[5].w), "v"(q[6].w), "v"(q[7].w), "v"(k.w));
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
// Sum over the LPR lanes that hold one token row (LPR = 4, 8, 16 or 32).
template <int LPR>
__device__ __forceinline__ float row_reduce_sum(float v) {
    v += dpp_f<0xB1>(v);                           // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);                           // quad_perm [2,3,0,1]
    if constexpr (LPR >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
    if constexpr (LPR >= 16) v += dpp_f<0x140>(v); // row_mirror
    if constexpr (LPR >= 32) v += __shfl_xor(v, 16);
    return v;
}
__device__ __forceinline__ uint16_t f2h_bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ __forceinline__ float h_bits2f(uint16_t x) { return (float)__builtin_bit_cast(_Float16, x); }
__device__ __forceinline__ float bcast(float v, int src_lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src_lane));
}
typedef _Float16 f16x4m __attribute__((ext_vector_type(4)));
typedef short    s16x4m __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __attribute__((address_space(3))) s16x4m *mma_lds(const uint16_t *p) {
    return (__attribute__((address_space(3))) s16x4m *)(p);
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// P.V on MFMA (v_mfma_f32_16x16x16f16, O^T += V^T P^T, G of the 16 columns
// live) instead of v_dot2 on token pairs: the VALU score path at head_dim 128
// and groups 2 to 8.  P.V's v_dot2 (64 G per lane and tile) give way to 32
// MFMAs, 32 transposing LDS reads and 8 LDS stores of the V rows, and the
// accumulators shrink to 32 VGPRs.  Measured: Llama-3-8B decode (group 4)
// 322 -> 311 us per step, group 8 and group 2 batches 3-8% faster; group 1,
// one live column in 16, was 1.5% slower and keeps v_dot2.
// Building with -DTL_ATTN_PV_DOT2 (make EXTRA=-DTL_ATTN_PV_DOT2) keeps P.V on
// v_dot2 token pairs everywhere: the comparison build behind that choice.
#ifdef TL_ATTN_PV_DOT2
template <int D, int G, bool MFMA>
constexpr bool kMfmaPV = false;
#else
template <int D, int G, bool MFMA>
constexpr bool kMfmaPV = !MFMA && D == 128 && G >= 2;
#endif
// The V stage of the MFMA P.V is a ring of two 16-token quarters per wave
// (8 KB at head_dim 128, 69 KB an 8-wave workgroup at group 4): a quarter's
// MFMAs run as soon as its rows are staged, while the next V batch loads.
// Against a whole-tile stage (16 KB a wave, 132 KB a workgroup, which leaves
// no room for a second workgroup's LDS on the CU) it measured level on
// Llama-3-8B decode and 0.3-1.5% faster per step on ragged, churn and
// group-8 batches.
constexpr int kVStageQuarters = 2;

// Dynamic shared memory of one workgroup.  Per wave one region that holds,
// in turn, the K transpose tile of the MFMA score path (16 rows of D halves,
// padded by 8 halves so that column reads of 16 rows fall in distinct bank
// groups) or the tile's fp16 p (and, with the MFMA P.V, the ring of staged
// V quarters after it), and at the end the wave's o[G][D] for the combine.
template <int D, int G, bool MFMA, int kNW>
struct Smem {
    static constexpr int kKt = MFMA ? 16 * (D + 8) * 2 : 0; // bytes
    static constexpr int kPp = kTile * G * 2;
    static constexpr int kO = G * D * 4;
    static constexpr int kV = kMfmaPV<D, G, MFMA> ? kVStageQuarters * 16 * D * 2 : 0; // V stage of the MFMA P.V
    static constexpr int kA = (kKt > kPp ? kKt : kPp) + kV;
    static constexpr int kWave = kA > kO ? kA : kO;
    __device__ static char  *vstage(char *wave_base) { return wave_base + kPp; }
    static constexpr int kBytes = kNW * kWave + 2 * kNW * G * 4;
    __device__ static char  *wave(char *base, int w) { return base + w * kWave; }
    __device__ static float *m(char *base) { return reinterpret_cast<float *>(base + kNW * kWave); }
    __device__ static float *l(char *base) { return m(base) + kNW * G; }
};

// ------------------------------------------------------------------ scorers
// A scorer owns the q registers and the running softmax state of the heads a
// lane is responsible for; it turns the K batches of a tile into fp16 p in
// LDS and hands the per-head rescale factors to the P.V stage.

// One step of the transposing row reduction: the N slots of every lane are
// halved by adding the partner's (DPP CTRL) upper half onto the lower half;
// with one slot left, the partner's slot is added.
template <int CTRL, int N>
__device__ __forceinline__ void xpose_step(float *d) {
    if constexpr (N >= 2) {
#pragma unroll
        for (int k = 0; k < N / 2; ++k) d[k] += dpp_f<CTRL>(d[k + N / 2]);
    } else {
        d[0] += dpp_f<CTRL>(d[0]);
    }
}

// VALU: lane (r = lane / LPR, p = lane % LPR); owner of heads h % LPR == p.
// With 16 (or 8) lanes per row and G a power of two in [2, LPR] (XP), the G
// head sums are instead reduced transposingly: lane p's slot k holds head
// k ^ f(p), so that adding the partner's upper half of the slots (partners
// p ^ 15, p ^ 7, p ^ 2, p ^ 1 -- row_mirror, row_half_mirror, quad_perm; the
// first only with 16 lanes) onto the lower half leaves lane p with the row's
// full sum for head f(p) after G - 1 + (log2 LPR - log2 G) DPP adds instead
// of G log2 LPR.  f is linear in p's bits with f(15) = G/2, f(7) = G/4,
// f(2) = G/8, f(1) = G/16 for 16 lanes (f(7) = G/2, f(2) = G/4, f(1) = G/8
// for 8; integer division), which is what makes the partner's slot k + N/2
// hold the same head as slot k at every step; the LPR/G lanes of a head are
// the p that differ in the low log2(LPR/G) bits, and the one with those bits
// zero owns it.
template <int D, int G>
struct ValuScorer {
    static constexpr int LPR = D / 8;
    static constexpr int TPI = 64 / LPR;
    static constexpr int NSTEP = kTile / TPI;
    static constexpr int HPL = (G + LPR - 1) / LPR;
    static constexpr bool XP = (LPR == 16 || LPR == 8) && G >= 2 && G <= LPR && (G & (G - 1)) == 0;
    // f at the partner masks (16 lanes: 15, 7, 2, 1; 8 lanes: 7, 2, 1)
    static constexpr int F15 = LPR == 16 ? G / 2 : 0;
    static constexpr int F7 = LPR == 16 ? G / 4 : G / 2;
    static constexpr int F2 = LPR == 16 ? G / 8 : G / 4;
    static constexpr int F1 = LPR == 16 ? G / 16 : G / 8;
    static __host__ __device__ constexpr int fhead(int q) {
        return ((q & 1) ? F1 : 0) ^ ((q & 2) ? F2 : 0) ^ ((q & 4) ? (F7 ^ F1 ^ F2) : 0) ^
               ((q & 8) ? (F15 ^ F7) : 0); // bit 3 only with 16 lanes
    }
    struct Owners {
        int lane[16];
    };
    static constexpr Owners owners() { // lane of head h with the low bits zero
        Owners o{};
        for (int q = LPR - 1; q >= 0; --q)
            if ((q & (LPR / G - 1)) == 0) o.lane[fhead(q)] = q;
        return o;
    }
    static constexpr Owners kOwners = owners();
    uint4 qv[G];
    float sc[HPL][NSTEP];
    float mrun[HPL], lrun[HPL], alpha[HPL];
    int   r, p;

    // Head of the lane's slot hh, and whether the lane writes its results.
    __device__ __forceinline__ int lane_head(int hh) const { return XP ? fhead(p) : hh * LPR + p; }
    __device__ __forceinline__ bool lane_owns(int hh) const {
        return XP ? (p & (LPR / G - 1)) == 0 : hh * LPR + p < G;
    }

    __device__ __forceinline__ void init(const __half *qrow, int lane) {
        r = lane / LPR;
        p = lane % LPR;
        const int f = XP ? fhead(p) : 0;
#pragma unroll
        for (int h = 0; h < G; ++h) qv[h] = *reinterpret_cast<const uint4 *>(qrow + (h ^ f) * D + 8 * p);
#pragma unroll
        for (int hh = 0; hh < HPL; ++hh) {
            mrun[hh] = -INFINITY;
            lrun[hh] = 0.0f;
        }
    }
    // Scores of load step s (tokens s*TPI + r of the tile) from the lane's row piece.
    __device__ __forceinline__ void step(int s, uint4 k, bool valid, float scale_log2) {
        if constexpr (XP) {
            float d[G];
            dot_heads<G>(qv, k, d);
            constexpr int N0 = LPR == 16 ? G : 2 * G; // slots before the p ^ 7 step
            if constexpr (LPR == 16) xpose_step<0x140, G>(d); // row_mirror: p ^ 15
            xpose_step<0x141, (N0 / 2 > 1 ? N0 / 2 : 1)>(d);     // row_half_mirror: p ^ 7
            xpose_step<0x4E, (N0 / 4 > 1 ? N0 / 4 : 1)>(d);      // quad_perm [2,3,0,1]: p ^ 2
            xpose_step<0xB1, (N0 / 8 > 1 ? N0 / 8 : 1)>(d);      // quad_perm [1,0,3,2]: p ^ 1
            sc[0][s] = valid ? d[0] * scale_log2 : -INFINITY;
            return;
        }
        float mine[HPL];
#pragma unroll
        for (int hh = 0; hh < HPL; ++hh) mine[hh] = 0.0f;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float d = fdot2(qv[h].x, k.x, 0.0f);
            d = fdot2(qv[h].y, k.y, d);
            d = fdot2(qv[h].z, k.z, d);
            d = fdot2(qv[h].w, k.w, d);
            d = row_reduce_sum<LPR>(d);
            if (h % LPR == p) mine[h / LPR] = d;
        }
#pragma unroll
        for (int hh = 0; hh < HPL; ++hh) sc[hh][s] = valid ? mine[hh] * scale_log2 : -INFINITY;
    }
    // After all steps: running max/sum update, p -> LDS (pair layout).
    __device__ __forceinline__ void softmax(uint16_t *pp) {
#pragma unroll
        for (int hh = 0; hh < HPL; ++hh) {
            const int h = lane_head(hh);
            float     m = -INFINITY;
#pragma unroll
            for (int s = 0; s < NSTEP; ++s) m = fmaxf(m, sc[hh][s]);
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
            const float mnew = fmaxf(mrun[hh], m);
            alpha[hh] = mrun[hh] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrun[hh] - mnew);
            mrun[hh] = mnew;
            float l = 0.0f;
            if (lane_owns(hh)) {
#pragma unroll
                for (int s = 0; s < NSTEP; ++s) {
                    const float    pv = sc[hh][s] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[hh][s] - mnew);
                    const uint16_t ph = f2h_bits(pv);
                    l += h_bits2f(ph);
                    if constexpr (kMfmaPV<D, G, false>) { // [head][token]
                        pp[h * kTile + s * TPI + r] = ph;
                    } else { // token s*TPI + r: pair block s/2, half s%2, q = r
                        pp[(((s >> 1) * TPI + r) * G + h) * 2 + (s & 1)] = ph;
                    }
                }
            }
            lrun[hh] = lrun[hh] * alpha[hh] + l;
        }
    }
    // Rescale factor of head h, broadcast to every lane.
    __device__ __forceinline__ float head_alpha(int h) const {
        if constexpr (XP) return bcast(alpha[0], kOwners.lane[h]);
        else return bcast(alpha[h / LPR], h % LPR);
    }
    // Final (m, l) of the lane's heads into LDS.
    __device__ __forceinline__ void finish(float *sm, float *sl) {
#pragma unroll
        for (int hh = 0; hh < HPL; ++hh) {
            float l = lrun[hh];
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) l += __shfl_xor(l, off);
            const int h = lane_head(hh);
            if (r == 0 && lane_owns(hh)) {
                sm[h] = mrun[hh];
                sl[h] = l;
            }
        }
    }
};

// MFMA: lane (kq = lane >> 4, r16 = lane & 15); lane holds heads 4*kq + i.
template <int D, int G>
struct MfmaScorer {
    static constexpr int LPR = D / 8;
    static constexpr int TPI = 64 / LPR;
    static constexpr int SPG = 16 / TPI; // load steps per 16-token group
    static constexpr int NG = kTile / 16;
    static constexpr int KS = D / 32;
    static constexpr int KR = D + 8; // padded tile row (halves)
    f16x8 qa[KS];
    float sc[NG][4];
    float mrun[4], lrun[4], alpha[4];
    int   r, p, r16, kq;

    __device__ __forceinline__ void init(const __half *qrow, int lane) {
        r = lane / LPR;
        p = lane % LPR;
        r16 = lane & 15;
        kq = lane >> 4;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (r16 < G) v = *reinterpret_cast<const uint4 *>(qrow + r16 * D + 8 * kq + 32 * ks);
            qa[ks] = __builtin_bit_cast(f16x8, v);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            mrun[i] = -INFINITY;
            lrun[i] = 0.0f;
        }
    }
    // Group j (steps j*SPG .. +SPG) of the tile: kr holds those steps' rows.
    __device__ __forceinline__ void group(int j, const uint4 *kr, uint16_t *kt, int nt,
                                          float scale_log2) {
#pragma unroll
        for (int u = 0; u < SPG; ++u)
            *reinterpret_cast<uint4 *>(kt + (r + TPI * u) * KR + 8 * p) = kr[u];
        wave_sync_lds();
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint4 kb = *reinterpret_cast<const uint4 *>(kt + r16 * KR + 8 * kq + 32 * ks);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[ks], __builtin_bit_cast(f16x8, kb), acc, 0,
                                                         0, 0);
        }
        wave_sync_lds();
        const bool ok = j * 16 + r16 < nt;
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[j][i] = ok ? acc[i] * scale_log2 : -INFINITY;
    }
    __device__ __forceinline__ void softmax(uint16_t *pp) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = 4 * kq + i;
            float     m = -INFINITY;
#pragma unroll
            for (int j = 0; j < NG; ++j) m = fmaxf(m, sc[j][i]);
            m = row_max16(m);
            const float mnew = fmaxf(mrun[i], m);
            alpha[i] = mrun[i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrun[i] - mnew);
            mrun[i] = mnew;
            float l = 0.0f;
            if (h < G) {
#pragma unroll
                for (int j = 0; j < NG; ++j) {
                    const float    pv = sc[j][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[j][i] - mnew);
                    const uint16_t ph = f2h_bits(pv);
                    l += h_bits2f(ph);
                    const int t = j * 16 + r16; // tile-local token
                    const int blk = t / (2 * TPI), rr = t - blk * 2 * TPI;
                    pp[((blk * TPI + rr % TPI) * G + h) * 2 + rr / TPI] = ph;
                }
            }
            lrun[i] = lrun[i] * alpha[i] + l;
        }
    }
    __device__ __forceinline__ float head_alpha(int h) const {
        float a = alpha[0];
        if (h % 4 == 1) a = alpha[1];
        if (h % 4 == 2) a = alpha[2];
        if (h % 4 == 3) a = alpha[3];
        return bcast(a, 16 * (h / 4));
    }
    __device__ __forceinline__ void finish(float *sm, float *sl) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float l = row_sum16(lrun[i]);
            const int   h = 4 * kq + i;
            if (r16 == 0 && h < G) {
                sm[h] = mrun[i];
                sl[h] = l;
            }
        }
    }
};

// Merge of an entry's chunk partials inside the attention launch, for the R
// query heads row0 .. row0 + R - 1 (the kv heads of one workgroup).  Every
// chunk's workgroup calls this after writing its partials.  Each wave waits
// for its own stores; after the workgroup barrier one thread releases them at
// device scope (the chunks run on any XCD, whose L2s are not coherent with
// each other: the fence writes this XCD's L2 back) and counts the chunk in
// *counter.  The thread that counts the last one acquires (invalidating this
// CU's and XCD's caches) before the barrier that lets its workgroup read the
// other chunks' partials and write the output rows; it resets the counter,
// so it is zero again for the next launch.  One device-scope fence per
// workgroup, two for the merging one (a fence in every wave made the launch
// 1.7x longer).  No workgroup waits for another.  Off by default
// (fused_merge_enabled): even so the launch's tail grows by more than the
// merge launch costs.  The
// arithmetic is attn_merge_kernel's, term for term (same bits):
//   m* = max m_c, l = sum l_c 2^(m_c-m*) (in blocks of kMergeMaxChunks,
//   rescaled between blocks), o = sum o_c 2^(m_c-m*) / (l + 1e-6).
// flag: an LDS word no thread reads or writes at the call.
constexpr int kMergeMaxChunks = 64;

template <int D, int R, int NT>
__device__ __forceinline__ void fused_merge(int *counter, int *flag, const float *part_o,
                                            const float *part_ml, __half *out, int Hq, int b,
                                            int row0, int pb0, int nch) {
    __builtin_amdgcn_s_waitcnt(kVmcntAll); // this wave's partial stores are done
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const bool last =
            __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nch - 1;
        if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        *flag = last;
    }
    __syncthreads();
    if (!*flag) return;
    const int64_t cs_ml = (int64_t)Hq * 2, cs_o = (int64_t)Hq * D; // chunk strides
    for (int idx = threadIdx.x; idx < R * D; idx += NT) {
        const int    h = idx / D, d = idx - h * D;
        const float *ml = part_ml + ((int64_t)pb0 * Hq + row0 + h) * 2;
        const float *po = part_o + ((int64_t)pb0 * Hq + row0 + h) * D + d;
        float        mx = -INFINITY, l = 0.0f;
        for (int c0 = 0; c0 < nch; c0 += kMergeMaxChunks) {
            const int cn = min(kMergeMaxChunks, nch - c0);
            float     mnew = mx;
            for (int c = c0; c < c0 + cn; ++c) mnew = fmaxf(mnew, ml[c * cs_ml]);
            l = c0 ? l * __builtin_amdgcn_exp2f(mx - mnew) : 0.0f;
            for (int c = c0; c < c0 + cn; ++c)
                l = fmaf(__builtin_amdgcn_exp2f(ml[c * cs_ml] - mnew), ml[c * cs_ml + 1], l);
            mx = mnew;
        }
        float o = 0.0f;
#pragma unroll 8
        for (int c = 0; c < nch; ++c) o = fmaf(__builtin_amdgcn_exp2f(ml[c * cs_ml] - mx), po[c * cs_o], o);
        out[((int64_t)b * Hq + row0 + h) * D + d] = __float2half(o * (1.0f / (l + 1e-6f)));
    }
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ kernel
template <int D, int G, bool PAGED, bool MFMA, int kNW, int HPW, int VBO = 0>
__global__ __launch_bounds__(kNW * 64)
__attribute__((amdgpu_waves_per_eu(kWavesPerEU))) void attn_decode_kernel(AttnArgs a) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group size");
    static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head_dim");
    static_assert(kNW == 4 || kNW == 8, "waves per workgroup");
    static_assert(HPW == 0 || (kNW % HPW == 0 && (HPW == 2 || HPW == 4 || HPW == 8)), "head block");
    constexpr bool HF = HPW > 0;                // head-fused
    constexpr int  H1 = HF ? HPW : 1;           // heads per workgroup
    constexpr int  NS = kNW / H1;               // waves sharing one kv head (tile slices)
    constexpr bool SOLO = HF && NS == 1;        // one wave per head: no cross-wave combine
    constexpr int kThreads = kNW * 64;
    using SM = Smem<D, G, MFMA, kNW>;
    using Scorer = typename std::conditional<MFMA, MfmaScorer<D, G>, ValuScorer<D, G>>::type;
    constexpr int  LPR = D / 8;
    constexpr int  TPI = 64 / LPR;
    constexpr int  NSTEP = kTile / TPI;      // K load steps per tile
    constexpr int  NBLK = kTile / (2 * TPI); // V pair blocks per tile
    constexpr int  SPG = MFMA ? 16 / TPI : 1; // steps consumed together
    constexpr int  KB0 = TL_ATTN_KB < NSTEP ? TL_ATTN_KB : NSTEP;
    constexpr int  KB = KB0 < SPG ? SPG : KB0; // steps per K batch
    constexpr int  NKB = NSTEP / KB;
    constexpr int  VB0 = VBO ? VBO : TL_ATTN_VB;
    constexpr int  VB = VB0 < NBLK ? VB0 : NBLK; // pair blocks per V batch
    constexpr int  NVB = NBLK / VB;
    extern __shared__ __align__(16) char smem[];

    const int       lane = threadIdx.x & 63;
    const int       wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // wave-uniform: scalar tile math
    const AttnPlan &pl = a.plan;
    // 1-D grid.  Per head (HPW = 0): kv head fastest, so the Hkv workgroups
    // reading the pieces of the same token rows are dispatched together.
    // Head-fused: block hb * n_work + item takes kv heads hb * HPW .. + HPW - 1
    // of the item, wave w head hb * HPW + w % HPW and tile slice w / HPW, so
    // the workgroup reads HPW heads' pieces of each token row at once; items
    // fastest, so that an entry's head blocks are dealt to one XCD when
    // n_work is a multiple of the XCD count.
    // (Head-fused over chunk items: head block fastest, keeping the work
    // list's longest-first order.)
    const bool ilv = HF && !pl.fused_chunked; // items interleave an entry's tiles
    const int  hbn = a.Hkv / H1;              // head blocks per item
    const int  item = !HF ? blockIdx.x / a.Hkv
                      : ilv ? (int)(blockIdx.x % (unsigned)pl.n_work)
                            : (int)(blockIdx.x / (unsigned)hbn);
    const int  hb = !HF ? 0 : ilv ? (int)(blockIdx.x / (unsigned)pl.n_work) : (int)(blockIdx.x % (unsigned)hbn);
    const int slice = wave / H1;
    const int g = HF ? hb * HPW + wave % H1 : blockIdx.x - item * a.Hkv;
    int       b, c, S, nch, widx, row;
    ATTN_WORK_ITEM(a, item, b, c, S, nch, widx, row);
    // One value per workgroup; the device-array path reads them with vector
    // loads (the kernel's stores could alias them, which rules out scalar
    // loads), so they are moved to scalar registers here: the tile loop and
    // the token addresses then run on the scalar unit.
    b = __builtin_amdgcn_readfirstlane(b);
    c = __builtin_amdgcn_readfirstlane(c);
    S = __builtin_amdgcn_readfirstlane(S);
    nch = __builtin_amdgcn_readfirstlane(nch);
    widx = __builtin_amdgcn_readfirstlane(widx);
    row = __builtin_amdgcn_readfirstlane(row);
    // HF: the nch items of an entry interleave its tiles in slices: slice s
    // of item c takes tiles u, u + nch * NS, ... with u = c * NS + s, instead
    // of contiguous chunks.
    const int t0 = ilv ? 0 : c * pl.chunk;
    const int n = ilv ? S : min(pl.chunk, S - t0); // >= 1 by construction of the plan
    const int ntiles = (n + kTile - 1) / kTile;
    // Tile order: wave w walks tiles tile_of(j), j = w, w + NW, ... (head-fused:
    // j = c * NS + slice, + nch * NS, ...) -- every tile once, rotated by an
    // offset that depends on the entry.  Entries of
    // equal length stream in lockstep; without the rotation their concurrent
    // reads sit a multiple of the slot stride apart, which for some strides
    // (max_seq_len 8256 or 8704 at 8 kv heads x 128 dims) maps them onto the
    // same HBM channels and cost 5% of the stream.
    const int rot = ntiles > 1 ? (int)((((uint32_t)b * 2654435761u) >> 8) % (uint32_t)ntiles) : 0;
    auto tile_of = [&](int j_) { const int x = j_ + rot; return x < ntiles ? x : x - ntiles; };
    // HF: the item holding the last tile appends (it reads token S-1).
    const int app_c = ilv ? ((ntiles - 1 - rot + ntiles) % ntiles) % (nch * NS) / NS : nch - 1;

    const RowAddr<PAGED> ra(a.kv, row, g);

    if (a.new_k && c == app_c) {
        // Fused appendKV(n=1) of head g at position S-1 (same bytes as the
        // D2D copies of kv_cache.cpp:230-233); HF: each slice-0 wave its own head.
        constexpr int P = D / 8; // 16-byte pieces per head row
        const int     tid = !HF ? (int)threadIdx.x : slice == 0 ? lane : kThreads;
        if (tid < 2 * P) {
            const int     which = tid / P, e = tid - which * P;
            const __half *src = (which ? a.new_v : a.new_k) + ((int64_t)b * a.Hkv + g) * D + e * 8;
            const char   *base = which ? ra.vbase : ra.kbase;
            char         *dst = const_cast<char *>(base) + ra.lane_off(S - 1) + 16 * e;
            *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(src);
        }
        __threadfence_block();
        __syncthreads();
    }

    char     *wbuf = SM::wave(smem, wave);
    uint16_t *pp = reinterpret_cast<uint16_t *>(wbuf);
    uint16_t *kt = reinterpret_cast<uint16_t *>(wbuf);
    const int r = lane / LPR; // row (token) within a load step
    const int p = lane % LPR; // 16-byte piece of the row

    Scorer sco;
    sco.init(a.q + ((int64_t)b * a.Hq + (int64_t)g * G) * D, lane);
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
    // MFMA P.V: O^T (dims x heads) in v_mfma_f32_16x16x16f16 tiles, lane
    // (hc, kq) holding dims 16 dt + 4 kq .. + 3 of head hc; the tile's V rows
    // go, a 16-token quarter at a time, through the wave's LDS stage (16-byte
    // piece x of the quarter's row t at slot t * KP + (x ^ t)) and come back
    // as V^T fragments by the transposing read, P^T from the [head][token] p
    // the scorer writes.
    constexpr bool MPV = kMfmaPV<D, G, MFMA>;
    constexpr int  DT = D / 16;
    constexpr int  KPV = D / 8;
    f32x4          oacc[MPV ? DT : 1];
#pragma unroll
    for (int dt = 0; dt < (MPV ? DT : 1); ++dt) oacc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int hc = lane & 15, kq = lane >> 4;
    uint16_t *vst = reinterpret_cast<uint16_t *>(SM::vstage(wbuf));
    auto vslot = [](int t, int x) { return t * KPV + (x ^ (t & (KPV - 1))); };
    // V batches per staged quarter, quarters per V batch.  A slot of the ring
    // is rewritten only after the MFMAs of the quarter staged in between,
    // which wait for that quarter's reads and so for every older LDS read.
    constexpr int kVBT = VB * 2 * TPI; // tokens per V batch
    constexpr int kBPQ = kVBT < 16 ? 16 / kVBT : 1;
    constexpr int kQPB = kVBT < 16 ? 1 : kVBT / 16;
    static_assert(!MPV || (kVBT % 16 == 0 || 16 % kVBT == 0), "V batches and quarters");
    static_assert(!MPV || kVStageQuarters >= 2 * kQPB, "V stage ring");

    uint4     kb[2][KB];
    uint4     va[2][VB], vb[2][VB];
    // Tile at chunk offset ts; tokens below tend are valid; q: the tile's
    // quarter block offsets.  A load step's TPI <= 16 tokens lie in one
    // quarter, known at compile time; tokens past the end are clamped to the
    // last valid one, which lies in the same quarter or in the block of the
    // tile's last token, the block that quarters past the end name.
    // The clamp runs on the scalar unit: a step's TPI tokens from ss (a
    // multiple of TPI) lie in one block, so with ssc = min(ss, lim) the row
    // of token min(ss + r, lim) sits min(r * tok_bytes, (lim - ssc) *
    // tok_bytes) bytes past row ssc -- one vector min and add per load over
    // a wave-uniform base (the work item's values are scalar, see above).
    using Quarters = typename RowAddr<PAGED>::Quarters;
    const uint32_t rtb = (uint32_t)r * ra.tok_bytes, p16 = 16u * (uint32_t)p;
    const gptr     kbu = uniform_ptr(ra.kbase), vbu = uniform_ptr(ra.vbase);
    auto step_ptr = [&](gptr base, int64_t qo, int ss, int lim) __attribute__((always_inline)) {
        const int      ssc = min(ss, lim);
        const uint32_t lim_off = (uint32_t)(lim - ssc) * ra.tok_bytes;
        return base + qo + ra.in_block(ssc) + (min(rtb, lim_off) + p16);
    };
    // (Tile starts and ends are wave-uniform; readfirstlane keeps them in
    // scalar registers where register pressure would move them to vector
    // ones.)
    auto kload = [&](int ts, int tend, int bi, uint4(&buf)[KB], const Quarters &q) {
        const int tb = __builtin_amdgcn_readfirstlane(t0 + ts);
        const int lim = __builtin_amdgcn_readfirstlane(t0 + tend - 1);
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int ss = tb + (bi * KB + u) * TPI; // step start (global token)
            buf[u] = ld16nt(step_ptr(kbu, q.o[(bi * KB + u) * TPI / 16], ss, lim));
        }
    };
    auto vload = [&](int ts, int tend, int bj, uint4(&bufa)[VB], uint4(&bufb)[VB], const Quarters &q) {
        const int tb = __builtin_amdgcn_readfirstlane(t0 + ts);
        const int lim = __builtin_amdgcn_readfirstlane(t0 + tend - 1);
#pragma unroll
        for (int u = 0; u < VB; ++u) {
            const int ob = (bj * VB + u) * 2 * TPI; // pair block start in the tile
            const int bs = tb + ob;
            bufa[u] = ld16nt(step_ptr(vbu, q.o[ob / 16], bs, lim));
            bufb[u] = ld16nt(step_ptr(vbu, q.o[(ob + TPI) / 16], bs + TPI, lim));
        }
    };
    // Quarter block ids of the wave's tile ti (paged views only).
    auto tile_bt = [&](int ti_) {
        return ra.tile_blocks(t0 + ti_ * kTile, t0 + min(n, ti_ * kTile + kTile) - 1, lane);
    };

    const int JS = !HF ? kNW : ilv ? nch * NS : NS;         // tile stride of a wave
    const int j0 = !HF ? wave : ilv ? c * NS + slice : slice; // its first tile
    int       j = j0;
    int       bt_cur = 0, bt_next = 0;
    if (j < ntiles) {
        const int tf = tile_of(j);
        bt_cur = tile_bt(tf);
        kload(tf * kTile, min(n, tf * kTile + kTile), 0, kb[0], ra.quarters(bt_cur));
    }
    for (; j < ntiles; j += JS) {
        const int      ts = tile_of(j) * kTile;
        const int      tend = min(n, ts + kTile);
        const int      nt = tend - ts;
        const Quarters qc = ra.quarters(bt_cur);
        if (PAGED && j + JS < ntiles) bt_next = tile_bt(tile_of(j + JS)); // consumed one tile later
        // ---- scores
#pragma unroll
        for (int bi = 0; bi < NKB; ++bi) {
            if (bi + 1 < NKB) kload(ts, tend, bi + 1, kb[(bi + 1) & 1], qc);
            else vload(ts, tend, 0, va[0], vb[0], qc);
            if constexpr (MFMA) {
#pragma unroll
                for (int u = 0; u < KB; u += SPG)
                    sco.group((bi * KB + u) / SPG, &kb[bi & 1][u], kt, nt, a.scale_log2);
            } else {
#pragma unroll
                for (int u = 0; u < KB; ++u) {
                    const int s = bi * KB + u;
                    sco.step(s, kb[bi & 1][u], s * TPI + r < nt, a.scale_log2);
                }
            }
            // Keep the scheduler from hoisting later batches' loads (which
            // would hold a whole tile in VGPRs): one batch in flight.
            __builtin_amdgcn_sched_barrier(0);
        }
        // ---- softmax; rescale the running P.V sums
        sco.softmax(pp);
        if constexpr (MPV) { // the lane's head hc (rows of heads >= G stay zero)
            float al = 0.0f;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float ah = sco.head_alpha(h);
                al = hc == h ? ah : al;
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) oacc[dt] *= al;
        } else {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float al = sco.head_alpha(h);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] *= al;
            }
        }
        wave_sync_lds();
        // ---- P.V on token pairs
#pragma unroll
        for (int bj = 0; bj < NVB; ++bj) {
            if (bj + 1 < NVB) {
                vload(ts, tend, bj + 1, va[(bj + 1) & 1], vb[(bj + 1) & 1], qc);
            } else if (j + JS < ntiles) {
                const int tn = tile_of(j + JS) * kTile;
                kload(tn, min(n, tn + kTile), 0, kb[0], ra.quarters(bt_next));
            }
#pragma unroll
            for (int u = 0; u < VB; ++u) {
                const int blk = bj * VB + u;
                if constexpr (MPV) { // the pair block's rows into their quarter's slot
                    const int t = blk * 2 * TPI + r; // t and t + TPI: one quarter
                    uint16_t *vq = vst + ((t >> 4) % kVStageQuarters) * (16 * D);
                    *reinterpret_cast<uint4 *>(vq + vslot(t & 15, p) * 8) = va[bj & 1][u];
                    *reinterpret_cast<uint4 *>(vq + vslot((t + TPI) & 15, p) * 8) = vb[bj & 1][u];
                    continue;
                }
                uint32_t        pw[G];
                const uint32_t *src = reinterpret_cast<const uint32_t *>(pp) + (blk * TPI + r) * G;
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
                const uint4    xa = va[bj & 1][u], xb = vb[bj & 1][u];
                const uint32_t wa[4] = {xa.x, xa.y, xa.z, xa.w};
                const uint32_t wb[4] = {xb.x, xb.y, xb.z, xb.w};
                uint32_t       vp[8]; // (v[t][d], v[t+TPI][d]) for the lane's 8 dims
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
            if constexpr (MPV) { // O^T += V^T P^T over each quarter this batch completed
                if ((bj + 1) % kBPQ == 0) {
                    wave_sync_lds(); // the quarter's rows are staged
#pragma unroll
                    for (int q = (bj + 1) / kBPQ * kQPB - kQPB; q < (bj + 1) / kBPQ * kQPB; ++q) {
                        f16x4m pb = {0, 0, 0, 0};
                        if (hc < G)
                            pb = __builtin_bit_cast(f16x4m, *reinterpret_cast<const uint2 *>(pp + hc * kTile + 16 * q + 4 * kq));
                        const uint16_t *vq = vst + (q % kVStageQuarters) * (16 * D);
                        const int       vr = 4 * kq + (hc >> 2), vh = 4 * (hc & 1);
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) {
                            const int    vx = 2 * dt + ((hc & 3) >> 1);
                            const s16x4m vf = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                mma_lds(vq + vslot(vr, vx) * 8 + vh));
                            oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4m, vf), pb,
                                                                             oacc[dt], 0, 0, 0);
                        }
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        wave_sync_lds(); // pp / kt / the V stage are rewritten by the next tile
        bt_cur = bt_next;
    }

    // ---- per-wave results -> LDS
    if constexpr (!MPV) {
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] += __shfl_xor(acc[h][e], off);
    }
    float *sm = SM::m(smem), *sl = SM::l(smem);
    if (j0 < ntiles) {
        sco.finish(sm + wave * G, sl + wave * G);
    } else if (lane < G) {
        sm[wave * G + lane] = -INFINITY;
        sl[wave * G + lane] = 0.0f;
    }
    float *so = reinterpret_cast<float *>(wbuf);
    if constexpr (MPV) {
        if (hc < G) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                *reinterpret_cast<float4 *>(so + hc * D + 16 * dt + 4 * kq) =
                    make_float4(oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3]);
        }
    } else if (r == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float *dst = so + h * D + p * 8;
            *reinterpret_cast<float4 *>(dst) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
            *reinterpret_cast<float4 *>(dst + 4) = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
    }
    if constexpr (SOLO) wave_sync_lds(); // the wave's own head: no other wave to wait for
    else __syncthreads();

    // ---- combine the waves of each head (SOLO: the wave alone), emit
    constexpr int NH = SOLO || !HF ? 1 : HPW; // heads this loop covers
    for (int idx = SOLO ? lane : (int)threadIdx.x; idx < NH * G * D; idx += SOLO ? 64 : kThreads) {
        const int hs = SOLO ? wave : idx / (G * D); // head slot in the workgroup (HF)
        const int e = SOLO || !HF ? idx : idx - hs * (G * D);
        const int h = e / D;
        const int d = e - h * D;
        const int gh = HF ? hb * HPW + hs : g; // kv head of this output
        float     mh = -INFINITY;
#pragma unroll
        for (int w0 = 0; w0 < NS; ++w0) {
            const int w = HF ? hs + HPW * w0 : w0;
            mh = fmaxf(mh, sm[w * G + h]);
        }
        float o = 0.0f, lh = 0.0f;
#pragma unroll
        for (int w0 = 0; w0 < NS; ++w0) {
            const int   w = HF ? hs + HPW * w0 : w0;
            const float mw = sm[w * G + h];
            const float wgt = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - mh);
            o = fmaf(wgt, reinterpret_cast<const float *>(SM::wave(smem, w))[e], o);
            lh = fmaf(wgt, sl[w * G + h], lh);
        }
        const int64_t row = (int64_t)b * a.Hq + (int64_t)gh * G + h;
        if (nch == 1) {
            a.out[row * D + d] = __float2half(o * (1.0f / (lh + 1e-6f)));
        } else {
            const int64_t prow = (int64_t)widx * a.Hq + (int64_t)gh * G + h;
            a.part_o[prow * D + d] = o;
            if (d == 0) {
                a.part_ml[prow * 2] = mh;
                a.part_ml[prow * 2 + 1] = lh;
            }
        }
    }
    if (a.counters && nch > 1) { // the workgroup's kv heads: g (per head), hb * HPW .. + HPW - 1
        const int gh0 = HF ? hb * HPW : g;
        fused_merge<D, H1 * G, kThreads>(a.counters + (int64_t)b * a.Hkv + gh0, reinterpret_cast<int *>(sm),
                                         a.part_o, a.part_ml, a.out, a.Hq, b, gh0 * G, widx - c, nch);
    }
}

// ----------------------------------------------------------------- MMA path
// Decode attention with both contractions on MFMA (head_dim 64 and 128).
// Each wave streams 16-token quarters of its tiles (wave w: tiles w, w+NW,
// ...) straight from HBM into its own LDS with the LDS DMA load
// (global_load_lds, 16 bytes per lane, whole rows per instruction), the next
// quarter in flight in the other buffer while the current one is computed;
// no workgroup barrier until the final combine.  Per quarter:
//   S^T = K Q^T   v_mfma_f32_16x16x32_f16, A = K rows (token l%16, dims
//                 8(l/16) + 32ks), B = q (head l%16, same dims; zero for heads
//                 >= G) -> lane: tokens 4(l/16)+i of head l%16
//   softmax       per head column in the log2 domain, lazy rescale (the
//                 reference point moves only on jumps above 2^8)
//   O^T += V^T P^T  v_mfma_f32_16x16x16_f16, A = V^T (dim l%16, tokens
//                 4(l/16)..+3) by ds_read_b64_tr_b16 from the row-major V
//                 rows, B = P^T exactly as the S^T fragment holds it.
// The combine across waves, the partials and the fused append are those of
// attn_decode_kernel.
constexpr float kMmaLazy = 8.0f;


template <int D, int G, bool PAGED, int kNW>
__global__ __launch_bounds__(kNW * 64) void attn_decode_mma_kernel(AttnArgs a) {
    static_assert(D == 64 || D == 128, "head_dim");
    static_assert(G >= 1 && G <= 8, "group size");
    constexpr int kThreads = kNW * 64;
    constexpr int KP = D / 8;          // 16-byte pieces per row
    constexpr int QH = 16 * D;         // halves of one 16-row quarter (K or V)
    constexpr int NQI = 16 * KP / 64;  // DMA pieces per lane per quarter and operand
    constexpr int KS = D / 32;         // k steps of S^T
    constexpr int DT = D / 16;         // dim tiles of O^T
    // Two buffers as distinct arrays (quarter k uses buffer k & 1), so the
    // compiler sees that the DMA into one does not alias reads of the other.
    __shared__ __align__(16) uint16_t qk0[kNW * QH], qv0[kNW * QH], qk1[kNW * QH], qv1[kNW * QH];
    __shared__ float sm_m[kNW * G], sm_l[kNW * G];
    // piece x of quarter row r at slot r * KP + (x ^ (r % KP))
    auto slot = [](int r, int x) { return r * KP + (x ^ (r & (KP - 1))); };

    const int       lane = threadIdx.x & 63;
    // wave-uniform in a scalar register: the quarter loop's branches then
    // stay scalar, and the compiler's vmcnt bookkeeping survives them
    const int       wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const AttnPlan &pl = a.plan;
    const int       item = blockIdx.x / a.Hkv;
    const int       g = blockIdx.x - item * a.Hkv;
    int             b, c, S, nch, widx, row;
    ATTN_WORK_ITEM(a, item, b, c, S, nch, widx, row);
    const int t0 = c * pl.chunk;
    const int n = __builtin_amdgcn_readfirstlane(min(pl.chunk, S - t0));
    const RowAddr<PAGED> ra(a.kv, row, g);

    if (a.new_k && c == nch - 1) {
        // Fused appendKV(n=1) of head g at position S-1 (kv_cache.cpp:230-233).
        const int tid = threadIdx.x;
        if (tid < 2 * KP) {
            const int     which = tid / KP, e = tid - which * KP;
            const __half *src = (which ? a.new_v : a.new_k) + ((int64_t)b * a.Hkv + g) * D + e * 8;
            const char   *base = which ? ra.vbase : ra.kbase;
            char         *dst = const_cast<char *>(base) + ra.lane_off(S - 1) + 16 * e;
            *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(src);
        }
        __threadfence_block();
        __syncthreads();
    }

    // q as the B operand of S^T: head l%16 (< G), dims 8(l/16) + 32ks
    const int hc = lane & 15, kq = lane >> 4;
    f16x8     qb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (hc < G)
            v = *reinterpret_cast<const uint4 *>(a.q + ((int64_t)b * a.Hq + (int64_t)g * G + hc) * D +
                                                 8 * kq + 32 * ks);
        qb[ks] = __builtin_bit_cast(f16x8, v);
    }
    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    // The wave's quarters: k -> tile wave + kNW * (k / 4), quarter k % 4.
    auto qstart = [&](int k) { return (wave + kNW * (k >> 2)) * kTile + 16 * (k & 3); };
    uint16_t *k0 = qk0 + wave * QH, *v0 = qv0 + wave * QH, *k1 = qk1 + wave * QH, *v1 = qv1 + wave * QH;
    // DMA of quarter k: K rows into kbuf, V rows into vbuf.
    auto issue = [&](int k, uint16_t *kbuf, uint16_t *vbuf) {
        const int qs = min(qstart(k), n - 1); // past the end: the last row again (a harmless re-read)
        int64_t   blk = 0;
        if constexpr (PAGED) blk = (int64_t)ra.bt_row[(t0 + qs) >> ra.log2_blk] * ra.blk_bytes; // uniform
#pragma unroll
        for (int u = 0; u < NQI; ++u) {
            const int    sl = u * 64 + lane;
            const int    r = sl / KP, x = (sl % KP) ^ (r & (KP - 1));
            const int    t = t0 + min(qs + r, n - 1);
            const int64_t off = blk + (int64_t)ra.in_block(t) + 16 * x;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(ra.kbase + off),
                                             (__attribute__((address_space(3))) void *)(kbuf + u * 512), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(ra.vbase + off),
                                             (__attribute__((address_space(3))) void *)(vbuf + u * 512), 16, 0, 0);
        }
    };
    // The fragments of one quarter from LDS: K rows as the A operand of S^T
    // (token hc, pieces kq + 4ks) and V^T by the transposing read (lane i of
    // each 16-lane group names 4 dims of one V row; afterwards lane i holds
    // dim 16dt + i of rows 4kq .. 4kq+3).
    struct Frags {
        f16x8  kf[KS];
        s16x4m vf[DT];
    };
    auto read_frags = [&](const uint16_t *kb, const uint16_t *vb, Frags &f) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) f.kf[ks] = *reinterpret_cast<const f16x8 *>(&kb[slot(hc, kq + 4 * ks) * 8]);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int vr = 4 * kq + (hc >> 2), vx = 2 * dt + ((hc & 3) >> 1), vh = 4 * (hc & 1);
            f.vf[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(mma_lds(&vb[slot(vr, vx) * 8 + vh]));
        }
    };
    // One quarter from its fragments.
    auto quarter = [&](int k, const Frags &f) __attribute__((always_inline)) {
        const int qs = qstart(k);
        f32x4     st = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.kf[ks], qb[ks], st, 0, 0, 0);
        float sv[4];
        float mq = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[i] = qs + 4 * kq + i < n ? st[i] * a.scale_log2 : -INFINITY;
            mq = fmaxf(mq, sv[i]);
        }
        mq = fmaxf(mq, __shfl_xor(mq, 16));
        mq = fmaxf(mq, __shfl_xor(mq, 32));
        if (__any(mq > m_run + kMmaLazy)) {
            const float m_new = fmaxf(m_run, mq);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new); // 0 on the first quarter
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
            l_run *= alpha;
            m_run = m_new;
        }
        f16x4m pb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float    pv = sv[i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv[i] - m_run);
            const _Float16 ph = (_Float16)pv;
            l_run += (float)ph; // the normaliser sums the weights the MFMA uses
            pb[i] = ph;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4m, f.vf[dt]), pb, acc[dt], 0, 0,
                                                            0);
    };

    // Quarter k: wait for its DMA (the only one in flight), read its
    // fragments, issue quarter k+1's DMA into the other buffers, compute.
    // The reads precede the next DMA, so nothing in flight can alias them.
    if (qstart(0) < n) {
        issue(0, k0, v0);
        Frags f;
        for (int k = 0;; k += 2) {
            __builtin_amdgcn_s_waitcnt(kVmcntAll);
            read_frags(k0, v0, f);
            const bool more1 = qstart(k + 1) < n;
            if (more1) issue(k + 1, k1, v1);
            quarter(k, f);
            if (!more1) break;
            __builtin_amdgcn_s_waitcnt(kVmcntAll);
            read_frags(k1, v1, f);
            const bool more2 = qstart(k + 2) < n;
            if (more2) issue(k + 2, k0, v0);
            quarter(k + 1, f);
            if (!more2) break;
        }
    }

    // ---- per-wave (m, l, o) -> LDS, combine the waves, emit
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    __syncthreads(); // every wave is done with the quarter buffers
    float *so = reinterpret_cast<float *>(qk0) + wave * G * D;
    static_assert(G * D * 4 <= QH * 2, "a wave's o fits its quarter of qk0");
    if (hc < G) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
            *reinterpret_cast<float4 *>(so + hc * D + 16 * dt + 4 * kq) =
                make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
        if (kq == 0) {
            const bool any = qstart(0) < n;
            sm_m[wave * G + hc] = any ? m_run : -INFINITY;
            sm_l[wave * G + hc] = any ? l_run : 0.0f;
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
        const int h = idx / D;
        const int d = idx - h * D;
        float     mh = -INFINITY;
#pragma unroll
        for (int w = 0; w < kNW; ++w) mh = fmaxf(mh, sm_m[w * G + h]);
        float o = 0.0f, lh = 0.0f;
#pragma unroll
        for (int w = 0; w < kNW; ++w) {
            const float mw = sm_m[w * G + h];
            const float wgt = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - mh);
            o = fmaf(wgt, reinterpret_cast<const float *>(qk0)[w * G * D + idx], o);
            lh = fmaf(wgt, sm_l[w * G + h], lh);
        }
        const int64_t orow = (int64_t)b * a.Hq + (int64_t)g * G + h;
        if (nch == 1) {
            a.out[orow * D + d] = __float2half(o * (1.0f / (lh + 1e-6f)));
        } else {
            const int64_t prow = (int64_t)widx * a.Hq + (int64_t)g * G + h;
            a.part_o[prow * D + d] = o;
            if (d == 0) {
                a.part_ml[prow * 2] = mh;
                a.part_ml[prow * 2 + 1] = lh;
            }
        }
    }
    if (a.counters && nch > 1)
        fused_merge<D, G, kThreads>(a.counters + (int64_t)b * a.Hkv + g, reinterpret_cast<int *>(sm_m), a.part_o,
                                    a.part_ml, a.out, a.Hq, b, g * G, widx - c, nch);
}

struct MergeArgs {
    const float   *part_o;  // [n_work][Hq][D]
    const float   *part_ml; // [n_work][Hq][2]
    __half        *out;
    const int32_t *part_base;
    int            nchunk;
    int            Hq;
    int            Hkv;
    InlineMeta     meta; // part_base from here when meta.n > 0
};

// Entries of at most this many chunks take the single-round-trip merge.
constexpr int kMergeFast = 8;

// One workgroup per (entry b, kv head g): log-sum-exp merge of the chunk
// partials of the G query heads,
//   m* = max m_c, l = sum l_c 2^(m_c-m*), o = sum o_c 2^(m_c-m*) / (l+1e-6).
// Up to kMergeFast chunks, each thread loads every chunk's (m, l) and o at
// once and weighs them itself (one memory round trip); more chunks go
// through LDS: the weights first, then every thread issues the o loads of
// all chunks back to back.  Entries with no tokens get a zero row.
template <int D, int G>
__global__ __launch_bounds__(256) void attn_merge_kernel(MergeArgs a) {
    __shared__ float s_w[kMergeMaxChunks][G];
    __shared__ float s_lc[kMergeMaxChunks][G]; // the chunks' l, loaded with their m
    __shared__ float s_m[G], s_l[G];
    const int        b = blockIdx.x / a.Hkv;
    const int        g = blockIdx.x - b * a.Hkv;
    int              pb0, nch;
    if (a.meta.n) {
        pb0 = a.meta.w[a.meta.off_part + b];
        nch = a.meta.w[a.meta.off_part + b + 1] - pb0;
    } else if (a.part_base) {
        pb0 = a.part_base[b];
        nch = a.part_base[b + 1] - pb0;
    } else {
        pb0 = b * a.nchunk;
        nch = a.nchunk;
    }
    __half          *dst = a.out + ((int64_t)b * a.Hq + (int64_t)g * G) * D;
    if (nch == 1) return; // written by attn_decode_kernel
    if (nch == 0) {
        for (int i = threadIdx.x; i < G * D; i += 256) dst[i] = __float2half(0.0f);
        return;
    }
    if (nch <= kMergeFast) {
        // One memory round trip: every thread loads its head's (m, l) pairs
        // and its o values of all chunks at once (indices clamped, unused
        // terms dropped by selects) and computes the chunk weights itself --
        // no LDS stage and no barrier.  The same terms in the same order as
        // below, so the same bits.
        for (int idx = threadIdx.x; idx < G * D; idx += 256) {
            const int    h = idx / D;
            const float *ml = a.part_ml + ((int64_t)pb0 * a.Hq + (int64_t)g * G + h) * 2;
            const float *po = a.part_o + ((int64_t)pb0 * a.Hq + (int64_t)g * G) * D + idx;
            float2       mlc[kMergeFast];
            float        pv[kMergeFast];
#pragma unroll
            for (int c = 0; c < kMergeFast; ++c) {
                const int64_t cc = min(c, nch - 1);
                mlc[c] = *reinterpret_cast<const float2 *>(ml + cc * a.Hq * 2);
                pv[c] = po[cc * a.Hq * D];
            }
            float mx = -INFINITY;
#pragma unroll
            for (int c = 0; c < kMergeFast; ++c) mx = c < nch ? fmaxf(mx, mlc[c].x) : mx;
            float l = 0.0f, o = 0.0f;
#pragma unroll
            for (int c = 0; c < kMergeFast; ++c) {
                const float wgt = __builtin_amdgcn_exp2f(mlc[c].x - mx);
                l = c < nch ? fmaf(wgt, mlc[c].y, l) : l;
                o = c < nch ? fmaf(wgt, pv[c], o) : o;
            }
            dst[idx] = __float2half(o * (1.0f / (l + 1e-6f)));
        }
        return;
    }
    const int w0 = pb0;
    for (int c0 = 0; c0 < nch; c0 += kMergeMaxChunks) {
        const int cn = min(kMergeMaxChunks, nch - c0);
        for (int i = threadIdx.x; i < cn * G; i += 256) {
            const int    c = i / G, h = i - c * G;
            const float2 ml = *reinterpret_cast<const float2 *>(
                &a.part_ml[((int64_t)(w0 + c0 + c) * a.Hq + (int64_t)g * G + h) * 2]);
            s_w[c][h] = ml.x;
            s_lc[c][h] = ml.y;
        }
        __syncthreads();
        if (threadIdx.x < G) { // running max and sum of head threadIdx.x
            const int h = threadIdx.x;
            float     mx = c0 ? s_m[h] : -INFINITY, mnew = mx;
            for (int c = 0; c < cn; ++c) mnew = fmaxf(mnew, s_w[c][h]);
            float l = c0 ? s_l[h] * __builtin_amdgcn_exp2f(mx - mnew) : 0.0f;
            for (int c = 0; c < cn; ++c) {
                const float wgt = __builtin_amdgcn_exp2f(s_w[c][h] - mnew);
                l = fmaf(wgt, s_lc[c][h], l);
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
                if (cn <= 8) { // every chunk's load in flight at once; a select keeps them up front
                    float pv[8];
#pragma unroll
                    for (int c = 0; c < 8; ++c) pv[c] = po[min(c, cn - 1) * rs];
#pragma unroll
                    for (int c = 0; c < 8; ++c) o = c < cn ? fmaf(s_w[c][h], pv[c], o) : o;
                } else {
#pragma unroll 16
                    for (int c = 0; c < cn; ++c) o = fmaf(s_w[c][h], po[c * rs], o);
                }
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
void launch_mma_dg(const AttnArgs &args, int n_work, int Hkv, bool paged, int nw, hipStream_t stream) {
    const dim3 grid((unsigned)n_work * (unsigned)Hkv);
    if (nw == 8) {
        if (paged) hipLaunchKernelGGL((attn_decode_mma_kernel<D, G, true, 8>), grid, dim3(512), 0, stream, args);
        else hipLaunchKernelGGL((attn_decode_mma_kernel<D, G, false, 8>), grid, dim3(512), 0, stream, args);
    } else {
        if (paged) hipLaunchKernelGGL((attn_decode_mma_kernel<D, G, true, 4>), grid, dim3(256), 0, stream, args);
        else hipLaunchKernelGGL((attn_decode_mma_kernel<D, G, false, 4>), grid, dim3(256), 0, stream, args);
    }
}

template <int D>
void launch_mma_d(const AttnArgs &args, int n_work, int Hkv, int G, bool paged, int nw, hipStream_t stream) {
    switch (G) {
    case 1: launch_mma_dg<D, 1>(args, n_work, Hkv, paged, nw, stream); break;
    case 2: launch_mma_dg<D, 2>(args, n_work, Hkv, paged, nw, stream); break;
    case 4: launch_mma_dg<D, 4>(args, n_work, Hkv, paged, nw, stream); break;
    case 8: launch_mma_dg<D, 8>(args, n_work, Hkv, paged, nw, stream); break;
    default: break;
    }
}

// Dynamic LDS of a decode launch: the kernel's own, raised for 8-wave
// workgroups past half of a CU's 160 KB, so that a CU holds one of them at a
// time -- the planner's model (plan_waves, plan_balanced_split: 8-wave
// workgroups one per CU, in turn).  Otherwise the occupancy would follow the
// register count: a kernel under 128 VGPRs fits two 8-wave workgroups on a CU,
// and a ragged plan then shares one CU's bandwidth between two items that its
// schedule runs one after the other (head_dim 128, group 1, 127 VGPRs: cfg2's
// balanced split 92 -> 108 us per layer).
constexpr int kCuLdsBytes = 160 * 1024;
template <int NW, int OWN>
constexpr int decode_lds_bytes() {
    return NW == 8 && OWN <= kCuLdsBytes / 2 ? kCuLdsBytes / 2 + 4096 : OWN;
}

template <int D, int G, bool PAGED, bool MFMA, int NW, int HPW = 0, int VBO = 0>
void launch_one(const AttnArgs &args, int n_work, int Hkv, hipStream_t stream) {
    using SM = Smem<D, G, MFMA, NW>;
    constexpr int         lds = decode_lds_bytes<NW, SM::kBytes>();
    auto                 *fn = attn_decode_kernel<D, G, PAGED, MFMA, NW, HPW, VBO>;
    static std::once_flag once;
    std::call_once(once, [&] {
        HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, lds));
    });
    const unsigned per = (unsigned)(Hkv / (HPW ? HPW : 1));
    hipLaunchKernelGGL(fn, dim3((unsigned)n_work * per), dim3(NW * 64), lds, stream, args);
}

// Chunk items of 2 heads per workgroup (ragged plans) load V 16 tokens a
// batch: 0.9% (cfg4-like lognormal, paged) and 1.7% (group-8 churn) faster
// per step than 8-token batches, which are 2.3% faster on the uniform
// interleaved plans.
template <int D, int G, int HPW>
void launch_fused(const AttnArgs &args, int n_work, int Hkv, bool paged, bool chunked,
                  hipStream_t stream) {
    if constexpr (HPW == 2) {
        if (chunked) {
            if (paged) launch_one<D, G, true, false, 8, HPW, 2>(args, n_work, Hkv, stream);
            else launch_one<D, G, false, false, 8, HPW, 2>(args, n_work, Hkv, stream);
            return;
        }
    }
    if (paged) launch_one<D, G, true, false, 8, HPW>(args, n_work, Hkv, stream);
    else launch_one<D, G, false, false, 8, HPW>(args, n_work, Hkv, stream);
}

template <int D, int G, bool MFMA>
void launch_dgm(const AttnArgs &args, int n_work, int Hkv, bool paged, int nw, int hpw,
                hipStream_t stream) {
    if constexpr (!MFMA && D == 128) { // the head-fused forms (VALU scores, head_dim 128)
        switch (hpw) {
        case 2: launch_fused<D, G, 2>(args, n_work, Hkv, paged, args.plan.fused_chunked, stream); return;
        case 4: launch_fused<D, G, 4>(args, n_work, Hkv, paged, args.plan.fused_chunked, stream); return;
        case 8: launch_fused<D, G, 8>(args, n_work, Hkv, paged, args.plan.fused_chunked, stream); return;
        default: break;
        }
    }
    if (nw == 8) {
        if (paged) launch_one<D, G, true, MFMA, 8>(args, n_work, Hkv, stream);
        else launch_one<D, G, false, MFMA, 8>(args, n_work, Hkv, stream);
    } else {
        if (paged) launch_one<D, G, true, MFMA, 4>(args, n_work, Hkv, stream);
        else launch_one<D, G, false, MFMA, 4>(args, n_work, Hkv, stream);
    }
}

template <int D, int G>
void launch_dg(const AttnArgs &args, int n_work, int Hkv, bool paged, bool mfma, int nw, int hpw,
               hipStream_t stream) {
    if constexpr (D <= 128) { // the MFMA score path exists for head_dim <= 128
        if (mfma) {
            launch_dgm<D, G, true>(args, n_work, Hkv, paged, nw, 0, stream);
            return;
        }
    }
    launch_dgm<D, G, false>(args, n_work, Hkv, paged, nw, hpw, stream);
}

template <int D>
void launch_d(const AttnArgs &args, int n_work, int Hkv, int G, bool paged, bool mfma, int nw,
              int hpw, hipStream_t stream) {
    switch (G) {
    case 1: launch_dg<D, 1>(args, n_work, Hkv, paged, mfma, nw, hpw, stream); break;
    case 2: launch_dg<D, 2>(args, n_work, Hkv, paged, mfma, nw, hpw, stream); break;
    case 4: launch_dg<D, 4>(args, n_work, Hkv, paged, mfma, nw, hpw, stream); break;
    case 8: launch_dg<D, 8>(args, n_work, Hkv, paged, mfma, nw, hpw, stream); break;
    default: break;
    }
}

// Score path: TL_ATTN_QK ("valu" / "mfma" / "auto" / "mma") at first use,
// else auto; tl_attn_set_score_path overrides it.  Within attn_decode_kernel
// auto resolves to VALU for every supported group: measured on the decode
// workloads (group 4 and 8, uniform and ragged contexts) its MFMA score path
// is never faster -- both are HBM-bound, and at group 8 the MFMA path's LDS
// staging and K double buffer spill a few more registers than the VALU path.
// Path 3 runs attn_decode_mma_kernel instead (use_mma_path).
std::atomic<int> g_score_path{-1};

int score_path_setting() {
    int v = g_score_path.load(std::memory_order_relaxed);
    if (v < 0) {
        const char *e = std::getenv("TL_ATTN_QK");
        v = 2;
        if (e && std::strcmp(e, "mfma") == 0) v = 1;
        if (e && std::strcmp(e, "valu") == 0) v = 0;
        if (e && std::strcmp(e, "mma") == 0) v = 3;
        g_score_path.store(v);
    }
    return v;
}

// Both contractions on MFMA (attn_decode_mma_kernel), path 3 only.  Measured
// against attn_decode_kernel (VALU scores): group 8 on the Llama-3-8B decode
// shape with 64 q heads 377 vs 397 us per step, but group 4 375 vs 334 and
// the ragged group-8 churn workload 1100 vs about 1060: each wave keeps one
// 16-token quarter in flight, which caps its stream, so auto stays on the
// VALU kernel.
bool use_mma_path(int D, int G) {
    (void)G;
    return (D == 64 || D == 128) && score_path_setting() == 3;
}

bool use_mfma_scores(int D, int G) {
    (void)G;
    if (D > 128) return false;
    return score_path_setting() == 1;
}

// Waves per workgroup: TL_ATTN_WAVES ("4" / "8" / "auto") at first use,
// else auto; tl_attn_set_waves overrides it (0 = auto).  Auto: 8-wave
// workgroups when the launch gives every CU at most two workgroups in turn
// (one resident at a time streams with all 8 waves to the end), else 4-wave
// workgroups two per CU, whose ramp-up and drain overlap.
std::atomic<int> g_waves{-1};

int waves_setting() {
    int v = g_waves.load(std::memory_order_relaxed);
    if (v < 0) {
        const char *e = std::getenv("TL_ATTN_WAVES");
        v = 0;
        if (e && std::strcmp(e, "4") == 0) v = 4;
        if (e && std::strcmp(e, "8") == 0) v = 8;
        g_waves.store(v);
    }
    return v;
}

int waves_for(int64_t workgroups) { return plan_waves(workgroups, device_cus(), waves_setting()); }

// Head-fused plans: TL_ATTN_HF ("0": off, "2" / "4" / "8": that many kv
// heads per workgroup where a plan with it applies, else auto) at first use;
// tl_attn_set_head_fuse overrides it.  0 = auto, 1 = off, 2 / 4 / 8 = forced.
std::atomic<int> g_head_fuse{-1};

int head_fuse_setting() {
    int v = g_head_fuse.load(std::memory_order_relaxed);
    if (v < 0) {
        const char *e = std::getenv("TL_ATTN_HF");
        v = 0;
        if (e && std::strcmp(e, "0") == 0) v = 1;
        if (e && (std::strcmp(e, "2") == 0 || std::strcmp(e, "4") == 0 || std::strcmp(e, "8") == 0))
            v = std::atoi(e);
        g_head_fuse.store(v);
    }
    return v;
}

} // namespace

void set_score_path(int path) { g_score_path.store(path); }
void set_waves(int waves) { g_waves.store(waves); }
void set_head_fuse(int mode) { g_head_fuse.store(mode); }
int  waves() { return waves_setting(); }
int  score_path() { return score_path_setting(); }
int  head_fuse() { return head_fuse_setting(); }

bool attn_shape_supported(int D, int G) {
    return (D == 32 || D == 64 || D == 128 || D == 256) && (G == 1 || G == 2 || G == 4 || G == 8);
}

size_t attn_workspace_floats(int n_work, int Hq, int D) {
    return (size_t)n_work * (size_t)Hq * (size_t)(D + 2);
}

int choose_chunk(const int32_t *lens, int n, int num_kv_heads, int uniform_len, int head_dim) {
    (void)head_dim;
    return plan_chunk(lens, n, num_kv_heads, uniform_len, device_cus(), chunk_override_from_env());
}

bool head_fused_kernel(int head_dim) {
    return head_dim == 128 && head_fuse_setting() != 1 && waves_setting() != 4 &&
           !use_mfma_scores(head_dim, 0) && !use_mma_path(head_dim, 0);
}

int planner_head_fuse(int head_dim) {
    const int mode = head_fuse_setting();
    return !head_fused_kernel(head_dim) ? 0 : mode == 0 ? 1 : mode;
}

void plan_work(const int32_t *lens, int n, int num_kv_heads, int head_dim, WorkList &out) {
    plan_work_list(lens, n, num_kv_heads, device_cus(), chunk_override_from_env(),
                   planner_head_fuse(head_dim), out);
}

// Merge placement: -1 until first use, then 1 (in the attention launch) or
// 0 (attn_merge_kernel, the default: the merging workgroups' device-scope
// fences and partial reads at the end of the launch cost more than the
// second launch, 99.2 against 92.2 + 4.7 us per cfg2 layer);
// TL_ATTN_MERGE=fused gives 1 at first use.
std::atomic<int> g_fused_merge{-1};

bool fused_merge_enabled() {
    int v = g_fused_merge.load(std::memory_order_relaxed);
    if (v < 0) {
        const char *e = std::getenv("TL_ATTN_MERGE");
        v = e && std::strcmp(e, "fused") == 0 ? 1 : 0;
        g_fused_merge.store(v);
    }
    return v != 0;
}

void set_fused_merge(bool on) { g_fused_merge.store(on ? 1 : 0); }

void launch_attn_decode(const __half *q, const KvView &kv, const AttnPlan &plan, int B, int Hq,
                        int Hkv, int D, float scale, __half *out, float *part, const __half *new_k,
                        const __half *new_v, hipStream_t stream, const InlineMeta *inl,
                        bool hooks, int *counters) {
    const int G = Hq / Hkv;
    if (plan.n_work <= 0 && !plan.any_empty) return;
    const bool paged = kv.block_table != nullptr;
    const bool mfma = use_mfma_scores(D, G);
    if (plan.chunk % kQuantum != 0 || plan.chunk <= 0)
        throw std::invalid_argument("attention: chunk length must be a positive multiple of " +
                                    std::to_string(kQuantum));
    // Token offsets inside a slot (contiguous) or a block (paged) are 32-bit
    // byte offsets (RowAddr::in_block).
    const int64_t span_tokens =
        paged ? std::min<int64_t>((int64_t)1 << std::min(kv.log2_blk, 62), plan.max_len) : plan.max_len;
    if (kv.log2_blk < 0 || kv.log2_blk > 30)
        throw std::invalid_argument("attention: log2_blk must be in [0, 30]");
    if (span_tokens * kv.tok_stride * 2 > (int64_t)UINT32_MAX)
        throw std::invalid_argument("attention: token offsets exceed 32 bits (tokens per " +
                                    std::string(paged ? "block" : "slot") + " * row bytes)");
    if (plan.any_multi && !part)
        throw std::invalid_argument("attention: a multi-chunk plan needs the partials workspace");
    const int  hpw = plan.fused_heads;
    const bool hf = hpw != 0;
    if (hf && (D != 128 || (hpw != 2 && hpw != 4 && hpw != 8) || Hkv % hpw != 0 ||
               (plan.any_empty && !plan.fused_chunked)))
        throw std::invalid_argument("attention: a head-fused plan needs head_dim 128, 2, 4 or 8 "
                                    "kv heads per workgroup dividing the kv heads, and (items "
                                    "interleaving tiles) no empty sequence");
    if (inl && inl->compact && (plan.any_multi || plan.any_empty || plan.n_work != inl->n))
        throw std::invalid_argument("attention: compact metadata needs one chunk per entry");
    AttnArgs args;
    args.q = q;
    args.out = out;
    args.part_o = part;
    args.part_ml = part ? part + (size_t)plan.n_work * Hq * D : nullptr;
    args.new_k = new_k;
    args.new_v = new_v;
    args.kv = kv;
    args.plan = plan;
    args.Hq = Hq;
    args.Hkv = Hkv;
    args.scale_log2 = scale * 1.4426950408889634f;
    if (inl) std::memcpy(&args.meta, inl, sizeof(InlineMeta));
    else args.meta.n = 0;
    // Merge inside the attention launch when every entry has work items (an
    // entry with none gets its zero rows from attn_merge_kernel).
    const bool fuse = counters && plan.any_multi && !plan.any_empty && fused_merge_enabled();
    args.counters = fuse ? counters : nullptr;

    if (plan.n_work > 0 && !hf && use_mma_path(D, G)) {
        const int nw = waves_for((int64_t)plan.n_work * Hkv);
        if (hooks) profile_begin(KernelId::AttnChunk, stream);
        if (D == 64) launch_mma_d<64>(args, plan.n_work, Hkv, G, paged, nw, stream);
        else launch_mma_d<128>(args, plan.n_work, Hkv, G, paged, nw, stream);
        HIP_CHECK(hipGetLastError());
        if (hooks) profile_end(KernelId::AttnChunk, stream);
    } else if (plan.n_work > 0) {
        // head-fused: 8-wave workgroups, VALU scores, whatever the settings
        const int nw = hf ? 8 : waves_for((int64_t)plan.n_work * Hkv);
        const bool mf = mfma && !hf;
        if (hooks) profile_begin(KernelId::AttnChunk, stream);
        switch (D) {
        case 32: launch_d<32>(args, plan.n_work, Hkv, G, paged, mf, nw, 0, stream); break;
        case 64: launch_d<64>(args, plan.n_work, Hkv, G, paged, mf, nw, 0, stream); break;
        case 128: launch_d<128>(args, plan.n_work, Hkv, G, paged, mf, nw, hpw, stream); break;
        case 256: launch_d<256>(args, plan.n_work, Hkv, G, paged, mf, nw, 0, stream); break;
        default: break;
        }
        HIP_CHECK(hipGetLastError());
        if (hooks) profile_end(KernelId::AttnChunk, stream);
    }

    if ((plan.any_multi || plan.any_empty) && !fuse) {
        MergeArgs m;
        m.part_o = args.part_o;
        m.part_ml = args.part_ml;
        m.out = out;
        m.part_base = plan.part_base;
        m.nchunk = plan.nchunk;
        m.Hq = Hq;
        m.Hkv = Hkv;
        if (inl) std::memcpy(&m.meta, inl, sizeof(InlineMeta));
        else m.meta.n = 0;
        if (hooks) profile_begin(KernelId::AttnMerge, stream);
        switch (D) {
        case 32: launch_merge_g<32>(m, B, Hkv, G, stream); break;
        case 64: launch_merge_g<64>(m, B, Hkv, G, stream); break;
        case 128: launch_merge_g<128>(m, B, Hkv, G, stream); break;
        case 256: launch_merge_g<256>(m, B, Hkv, G, stream); break;
        default: break;
        }
        HIP_CHECK(hipGetLastError());
        if (hooks) profile_end(KernelId::AttnMerge, stream);
    }
}

} // namespace detail
} // namespace tiny_llm
