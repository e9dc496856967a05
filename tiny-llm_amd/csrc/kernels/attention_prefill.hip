// Prefill attention for gfx950: causal attention of a block of new query
// tokens over a KV view, GQA, on MFMA; plus the reference's softmax and
// attention-weights kernels.
//
// Per query token i of a sequence whose new tokens start at position p0 and
// query head h (kv head g = h / G):
//   o_h = (sum_{p <= p0+i} e_p v_{g,p}) / (sum_{p <= p0+i} e_p + 1e-6),
//   e_p = 2^(s_p - m),  s_p = (q_h . k_{g,p}) * scale * log2(e),  m = max_p s_p
// which is the arithmetic of attention_prefill_kernel (attention.cu:131-222:
// masked keys get -FLT_MAX and contribute exp(...) = 0), reading the keys
// from the cache instead of the current token batch, and equal to decode
// attention over the first p0+i+1 keys.
//
// Workgroup: 8 waves (one workgroup per CU), one kv head g, 256 query rows =
// 256/G tokens x G heads (head_dim 256: 4 waves, 64 rows); each wave owns two
// (one) 16-row query column groups.  Keys stream in tiles of 64 tokens through double-buffered LDS,
// K and V both row-major, written by the LDS DMA load (global_load_lds,
// 16 bytes per lane) with XOR-swizzled 16-byte slots.  Per wave, group and
// tile:
//   S^T = K Q^T        v_mfma_f32_16x16x32_f16: A = K rows (token l%16,
//                      dims 8(l/16)..+7), B = Q (query l%16, same dims),
//                      D = S^T (tokens 4(l/16)+i, query l%16)
//   online softmax     per query column, over the lane's 16 scores and the
//                      4 lanes sharing the column (xor 16, 32); the reference
//                      max moves only on jumps > 8 (log2), so the running
//                      sums are rarely rescaled
//   O^T += V^T P^T     v_mfma_f32_16x16x32_f16 over 32 keys: B = P^T is the
//                      fp16 S^T fragments of two key tiles as they stand
//                      (k index 8(l/16)+j names key 4(l/16)+j of the first
//                      tile for j < 4, of the second for j >= 4); A = V^T
//                      (dim l%16) in that key order, read from the row-major
//                      V tile with ds_read_b64_tr_b16 (gfx950's transposing
//                      LDS read); D = O^T (dims 4(l/16)+i, query l%16), so
//                      the rescale by the running max is lane-local.
// The next tile's DMA runs while the current one is computed; the output
// rows go through LDS so that every store is a whole row.  Grid: work items
// x Hkv, kv head fastest, so with 8 kv heads every workgroup of head g runs
// on XCD g and the tiles it re-reads stay in that XCD's L2.
#include "prefill.h"

#include "tiny_llm/hip_utils.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

namespace tiny_llm {
namespace detail {

namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef short    s16x4 __attribute__((ext_vector_type(4)));

// LDS (address space 3) view of a pointer into a __shared__ array, the
// operand type of the transposing LDS read.
__device__ __forceinline__ __attribute__((address_space(3))) s16x4 *lds_ptr(const uint16_t *p) {
    return (__attribute__((address_space(3))) s16x4 *)(p);
}

// max(x of lane l, x of lane l ^ S) for S = 16 or 32, on the VALU: the
// gfx950 lane swaps (v_permlane16_swap / v_permlane32_swap) of x with itself
// give every lane its own value in one result and its partner's in the other
// (rows of 16 lanes: odd rows with even ones, or the two halves of the wave).
template <int S>
__device__ __forceinline__ float xor_lane_max(float x) {
    static_assert(S == 16 || S == 32, "a row or half-wave swap");
    const unsigned u = __float_as_uint(x);
    if constexpr (S == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
}

// Waves per workgroup (template argument NW): up to head_dim 128, 8 (two per
// SIMD, one workgroup per CU), so each K/V tile in LDS serves 256 query rows,
// or 4 (two workgroups per CU, 128 rows each: one's start-up -- work record,
// q, first tile -- runs under the other's tiles, which pays for launches of
// many short items; the planner's rule is prefill_waves); 4 for head_dim 256,
// whose register file allows one wave per SIMD.  (Head_dim 128 with 4 waves
// of three 16-row groups each -- a third less LDS read traffic per flop, one
// wave per SIMD -- was 1.5x slower: the second wave on each SIMD hides the LDS
// and MFMA latencies.)
// Lazy rescaling threshold of the online softmax, in log2 units.
constexpr float kLazyMax = 8.0f;
// s_waitcnt immediate (gfx9 encoding) waiting for vmcnt == 0 only.
constexpr int kVmcnt0 = 0x0F70;
constexpr int kKeyTile = 64;

struct PrefillArgs {
    const __half       *q;
    __half             *out;
    KvView              kv;
    const int32_t      *work; // kPrefillItemWords words per item, or null (uniform)
    int64_t             q_tok;
    int64_t             q_head;
    int64_t             q_entry;
    int                 uniform_b;
    int                 uniform_n;
    const __half       *new_k; // fused append source or null
    const __half       *new_v;
    int                 Hkv;
    float               scale_log2;
};

// Byte offsets of the token rows of one (cache row, kv head).
template <bool PAGED>
struct KeyRows {
    const char    *kbase;
    const char    *vbase;
    const int32_t *bt_row;
    int64_t        blk_bytes;
    int64_t        tok_bytes;
    int            log2_blk;
    int            mask;

    __device__ __forceinline__ KeyRows(const KvView &v, int row, int g) {
        const int64_t head = (int64_t)g * v.head_stride * 2;
        blk_bytes = v.blk_stride * 2;
        tok_bytes = v.tok_stride * 2;
        log2_blk = v.log2_blk;
        mask = (1 << v.log2_blk) - 1;
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
    __device__ __forceinline__ int64_t off(int t) const {
        if constexpr (PAGED) return (int64_t)bt_row[t >> log2_blk] * blk_bytes + (int64_t)(t & mask) * tok_bytes;
        else return (int64_t)t * tok_bytes;
    }
};

__device__ __forceinline__ uint4 ld16(const char *p) { return *reinterpret_cast<const uint4 *>(p); }

// 16-query column groups per wave: two share every K and V^T fragment read
// from LDS (half the LDS traffic per flop); head_dim 256 keeps one to fit
// the register file.
template <int D>
constexpr int kQueryGroups = D <= 128 ? 2 : 1;

// Rounds x to fp32 in a register before whatever consumes it: keeps the
// compiler from folding a multiply into the fp16 conversion that follows
// (v_fma_mixlo_f16 rounds once, the reference's __float2half(a * b) twice).
__device__ __forceinline__ float materialize(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

template <int D, int G, bool PAGED, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1))) void attn_prefill_kernel(PrefillArgs a) {
    static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head_dim");
    static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group size");
    static_assert(NW == 4 || (NW == 8 && D <= 128), "waves");
    constexpr int NQG = kQueryGroups<D>;    // 16-query column groups per wave
    constexpr int NT = NW * 64;             // threads
    constexpr int ROWS = NW * 16 * NQG;     // query rows per workgroup
    static_assert(ROWS == prefill_rows(D, NW), "the planner's query tile");
    constexpr int BQ = ROWS / G;            // query tokens per workgroup
    constexpr int KS = D / 32;              // k steps of S^T
    constexpr int DT = D / 16;              // dim tiles of O^T
    constexpr int KP = D / 8;               // 16-byte pieces per row
    constexpr int ROWH = D;                 // halves per LDS row (unpadded, swizzled)
    constexpr int PIECES = kKeyTile * KP;   // 16-byte pieces of a K (or V) tile
    constexpr int NKI = (PIECES + NT - 1) / NT; // K pieces per thread
    // Two buffers per operand as distinct arrays, so the compiler can tell
    // that the DMA into one does not alias the reads of the other and does
    // not wait for it before computing.
    __shared__ __align__(16) uint16_t ks0[kKeyTile * ROWH], ks1[kKeyTile * ROWH];
    __shared__ __align__(16) uint16_t vt0[kKeyTile * ROWH], vt1[kKeyTile * ROWH];
    // 16-byte piece x of key row r sits at slot x ^ swz(r) of the row, where
    // swz is the XOR-linear map r -> 2 r0 ^ 4 r1 ^ 9 r2 ^ 8 r3 of the row's
    // low four bits (mod KP; r mod 4 for KP 4).  Reads then touch distinct
    // banks whether the LDS serves 128 or 256 bytes a cycle: the 8 or 16
    // rows of a K fragment read (one piece each), and the two adjacent
    // pieces of the 4 or 8 rows a transposing V read touches (with
    // x ^ (r % KP), rows r and r ^ 1 put that pair on the same banks).  No
    // padding, so each wave's DMA of 1 KB lands contiguous.
    auto swz = [](int r) {
        if constexpr (KP <= 4) return r & (KP - 1);
        const int f = ((r & 3) << 1) ^ (((r >> 2) & 1) * 9) ^ (((r >> 3) & 1) << 3);
        return f & (KP - 1);
    };
    auto slot = [&](int r, int x) { return r * KP + (x ^ swz(r)); };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int item = blockIdx.x / a.Hkv;
    const int g = blockIdx.x - item * a.Hkv;
    int64_t   q_off;
    int       p0, n, row, qt, tok0 = 0;
    if (a.work) { // one self-contained record: a single dependent load
        const int32_t *w = a.work + (int64_t)kPrefillItemWords * item;
        q_off = (int64_t)(((uint64_t)(uint32_t)w[1] << 32) | (uint32_t)w[0]);
        p0 = w[2];
        n = w[3];
        row = w[4];
        qt = w[5];
        tok0 = w[6];
    } else { // uniform entries, the query tiles with the most keys first
        const int nqt = (a.uniform_n + BQ - 1) / BQ;
        const int b = item % a.uniform_b;
        qt = nqt - 1 - item / a.uniform_b;
        q_off = (int64_t)b * a.q_entry;
        p0 = 0;
        n = a.uniform_n;
        row = b;
    }
    const int c = lane & 15, qg = lane >> 4;
    // Transposing V^T reads: lane (c, qg) names, for dim tile dt and a
    // 16-key row group at key offset r0 (a multiple of 16), the 4 dims
    // 16dt + 4(c%4) .. +3 of key row r0 + 4qg + c/4.  The swizzle depends on
    // a row's low four bits only, and the piece 2dt + (c%4)/2 has bit 0 from
    // c alone, so the address is a lane constant, (2dt ^ vxor) pieces and an
    // immediate r0 * KP * 8: eight lane offsets instead of one register per
    // (key group, dim tile).
    const int vrow = 4 * qg + (c >> 2);
    const int vxor = ((c & 3) >> 1) ^ swz(vrow);
    const int vlane = vrow * KP * 8 + 4 * (c & 1);
    auto vt_read = [&](const uint16_t *vd, int r0, int dt) __attribute__((always_inline)) {
        return __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr(&vd[vlane + ((2 * dt) ^ vxor) * 8 + r0 * KP * 8]));
    };
    const int kend = p0 + min(n, (qt + 1) * BQ);
    const int ntile = (kend + kKeyTile - 1) / kKeyTile;
    int       pos[NQG];  // keys 0 .. pos are attended by the lane's query column
    bool      valid[NQG];
    int64_t   qrow[NQG]; // element offset of the column's query row
    f16x8     qb[NQG][KS];
#pragma unroll
    for (int j = 0; j < NQG; ++j) {
        const int r = wave * 16 * NQG + j * 16 + c;
        const int qi = qt * BQ + r / G;
        const int h = g * G + r % G;
        valid[j] = qi < n;
        const int qic = valid[j] ? qi : n - 1;
        pos[j] = p0 + qic;
        qrow[j] = q_off + (int64_t)qic * a.q_tok + (int64_t)h * a.q_head;
        // B operand of S^T: query column c, dims 32s + 8qg .. +7
        const char *qp = reinterpret_cast<const char *>(a.q + qrow[j]);
#pragma unroll
        for (int s = 0; s < KS; ++s) qb[j][s] = __builtin_bit_cast(f16x8, ld16(qp + 2 * (32 * s + 8 * qg)));
    }

    // Smallest attended position of the wave's queries: tiles ending at or
    // below it need no causal mask.
    int wave_min_pos = pos[0];
#pragma unroll
    for (int j = 1; j < NQG; ++j) wave_min_pos = min(wave_min_pos, pos[j]);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) wave_min_pos = min(wave_min_pos, __shfl_xor(wave_min_pos, o));
    wave_min_pos = __builtin_amdgcn_readfirstlane(wave_min_pos);

    const KeyRows<PAGED> kr(a.kv, row, g);
    // Byte offset of token t's row piece pc: 32 bits for a contiguous row
    // (the host checks that the rows of one cache row span < 4 GiB).
    auto roff = [&](int t, int pc) -> int64_t {
        if constexpr (PAGED) return kr.off(t) + 16 * pc;
        else return (uint32_t)t * (uint32_t)kr.tok_bytes + (uint32_t)(16 * pc);
    };
    // Tile kt of K and V straight from global memory into LDS buffer buf
    // (global_load_lds, 16 bytes per lane): thread t fills slots
    // u*256 + t, i.e. every wave instruction one contiguous 1 KB of the tile;
    // slot s holds row s / KP, piece (s % KP) ^ swz(row).  Completion is
    // tracked by vmcnt.
    auto issue_tile = [&](int kt, uint16_t *kdst, uint16_t *vdst) {
        const int t0 = kt * kKeyTile;
#pragma unroll
        for (int u = 0; u < NKI; ++u) {
            const int sl = u * NT + tid;
            if (NKI * NT > PIECES && sl >= PIECES) break; // whole waves (PIECES % 64 == 0)
            const int r = sl / KP, x = (sl % KP) ^ swz(r);
            const int t = min(t0 + r, kend - 1);
            const char *ks, *vs;
            if (a.new_k && t >= p0) { // a new token: its row in the fused append's input
                const int64_t o = ((int64_t)(tok0 + t - p0) * a.Hkv + g) * (2 * D) + 16 * x;
                ks = reinterpret_cast<const char *>(a.new_k) + o;
                vs = reinterpret_cast<const char *>(a.new_v) + o;
            } else {
                const int64_t off = roff(t, x);
                ks = kr.kbase + off;
                vs = kr.vbase + off;
            }
            const int lbase = (u * NT + wave * 64) * 8; // halves, wave-uniform
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)ks,
                                             (__attribute__((address_space(3))) void *)(&kdst[lbase]), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)vs,
                                             (__attribute__((address_space(3))) void *)(&vdst[lbase]), 16, 0, 0);
        }
    };

    f32x4 acc[NQG][DT];
#pragma unroll
    for (int j = 0; j < NQG; ++j)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[j][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // Running row sums on the MFMA: l^T += 1^T P^T (A = a 16 x 32 block of
    // ones, B = the P^T fragment), so every lane of a query column holds the
    // column's whole sum of the fp16 weights the P.V uses, with no VALU add
    // chain and no cross-lane sum at the end.
    float m_run[NQG];
    f32x4 l_run[NQG];
#pragma unroll
    for (int j = 0; j < NQG; ++j) {
        m_run[j] = -INFINITY;
        l_run[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const f16x8 ones = __builtin_bit_cast(f16x8, make_uint4(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u));

    // One tile: issue the next tile's DMA into the other buffers, compute on
    // kd/vd, wait for the DMA, barrier.
    auto tile_step = [&](int kt, const uint16_t *kd, const uint16_t *vd, uint16_t *kn, uint16_t *vn)
                         __attribute__((always_inline)) {
        if (a.new_k) {
            // Fused appendKV: the rows of this query tile's own tokens (kv
            // head g) that lie in tile kt go from LDS into the cache --
            // nothing in this launch reads them from there.
            const int lo = max(kt * kKeyTile, p0 + qt * BQ);
            const int hi = min(kt * kKeyTile + kKeyTile, p0 + min(n, qt * BQ + BQ));
            for (int e = tid; e < (hi - lo) * KP; e += NT) {
                const int     t = lo + e / KP, x = e % KP, sl = slot(t - kt * kKeyTile, x);
                const uint4   kk = *reinterpret_cast<const uint4 *>(&kd[sl * 8]);
                const uint4   vv = *reinterpret_cast<const uint4 *>(&vd[sl * 8]);
                const int64_t d = kr.off(t) + 16 * x;
                *reinterpret_cast<uint4 *>(const_cast<char *>(kr.kbase) + d) = kk;
                *reinterpret_cast<uint4 *>(const_cast<char *>(kr.vbase) + d) = vv;
            }
        }
        // the next tile lands in the other buffer during this tile's math
        if (kt + 1 < ntile) issue_tile(kt + 1, kn, vn);

        // ---- S^T = K Q^T: 16 keys x 16 queries per fragment; one K
        // fragment serves every query group of the wave
        // (two key tiles at a time: 2 x NQG independent accumulators per k
        // step keep the MFMA pipeline busy within the register budget)
        f32x4 s[NQG][4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int j = 0; j < NQG; ++j) s[j][tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int th = 0; th < 4; th += 2)
#pragma unroll
            for (int st = 0; st < KS; ++st) {
                f16x8 kf[2];
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    kf[u] = *reinterpret_cast<const f16x8 *>(&kd[slot(16 * (th + u) + c, 4 * st + qg) * 8]);
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int j = 0; j < NQG; ++j)
                        s[j][th + u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[u], qb[j][st], s[j][th + u], 0, 0, 0);
            }
        // ---- causal mask (only tiles that reach past a query of the wave),
        // online softmax per query column in the log2 domain:
        // m = scale_log2 * max s, p = 2^(s * scale_log2 - m) by one FMA.
        const int tb = kt * kKeyTile + 4 * qg;
        f16x8     pf[NQG][2]; // P^T as the B operand of a 32-key step (see below)
        if (kt * kKeyTile + kKeyTile - 1 > wave_min_pos) {
#pragma unroll
            for (int j = 0; j < NQG; ++j)
#pragma unroll
                for (int tt = 0; tt < 4; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (tb + 16 * tt + i > pos[j]) s[j][tt][i] = -INFINITY;
        }
#pragma unroll
        for (int j = 0; j < NQG; ++j) {
            float mloc = fmaxf(fmaxf(fmaxf(s[j][0][0], s[j][0][1]), fmaxf(s[j][0][2], s[j][0][3])),
                               fmaxf(fmaxf(s[j][1][0], s[j][1][1]), fmaxf(s[j][1][2], s[j][1][3])));
            mloc = fmaxf(mloc, fmaxf(fmaxf(fmaxf(s[j][2][0], s[j][2][1]), fmaxf(s[j][2][2], s[j][2][3])),
                                     fmaxf(fmaxf(s[j][3][0], s[j][3][1]), fmaxf(s[j][3][2], s[j][3][3]))));
            mloc = xor_lane_max<16>(mloc);
            mloc = xor_lane_max<32>(mloc);
            // Key 0 lies in tile 0 and every query attends it, so the max is
            // finite from the first tile on.  The reference point m_run only
            // moves when the max passes it by more than kLazyMax (log2
            // units): until then p = 2^(x - m_run) <= 2^kLazyMax, exact in
            // fp32 and fp16 range, and the final division by l cancels the
            // shift, so the running sums are rescaled only on such jumps
            // (once or twice per row instead of on most tiles).
            const float m_tile = mloc * a.scale_log2;
            if (__any(m_tile > m_run[j] + kLazyMax)) {
                const float m_new = fmaxf(m_run[j], m_tile);
                const float alpha = __builtin_amdgcn_exp2f(m_run[j] - m_new);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) acc[j][dt] *= alpha;
                l_run[j] *= alpha;
                m_run[j] = m_new;
            }
            const float m_new = m_run[j];
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                float p[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][tt][i], a.scale_log2, -m_new));
                const uint32_t lo = __builtin_bit_cast(uint32_t, __floats2half2_rn(p[0], p[1]));
                const uint32_t hi = __builtin_bit_cast(uint32_t, __floats2half2_rn(p[2], p[3]));
                uint4 w = __builtin_bit_cast(uint4, pf[j][tt >> 1]);
                if (tt & 1) {
                    w.z = lo;
                    w.w = hi;
                } else {
                    w.x = lo;
                    w.y = hi;
                }
                pf[j][tt >> 1] = __builtin_bit_cast(f16x8, w);
            }
        }
        // ---- O^T += V^T P^T on v_mfma_f32_16x16x32_f16 over 32 keys per
        // step.  Lane group qg's k index 8qg+j stands for key 32tp + 4qg + j
        // (j < 4) or 32tp + 16 + 4qg + j - 4 (j >= 4): the keys its S^T
        // fragments of tiles 2tp and 2tp+1 hold, so P^T needs no data
        // movement; the V^T fragment is read with the same key order.
        // Key step outermost: the first step's MFMAs need only the first
        // half's weights, so they can issue while the second half's are
        // still in the exponentials (each accumulator still sees step 0,
        // then step 1).
#pragma unroll
        for (int tp = 0; tp < 2; ++tp) {
#pragma unroll
            for (int j = 0; j < NQG; ++j)
                l_run[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[j][tp], l_run[j], 0, 0, 0);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                // Transposing LDS reads: lane s of each 16-lane group names
                // the 4 dims 16dt + 4(s%4) .. +3 of key row 32tp + 4qg + s/4
                // (+16 for the second read); lane i then holds dim 16dt + i
                // of keys 32tp + 4qg + j (j = 0..3), the A fragment in the key
                // order above.
                const s16x4     v0 = vt_read(vd, 32 * tp, dt);
                const s16x4     v1 = vt_read(vd, 32 * tp + 16, dt);
                const f16x8     vf = __builtin_bit_cast(
                    f16x8, make_uint4(__builtin_bit_cast(uint2, v0).x, __builtin_bit_cast(uint2, v0).y,
                                      __builtin_bit_cast(uint2, v1).x, __builtin_bit_cast(uint2, v1).y));
#pragma unroll
                for (int j = 0; j < NQG; ++j)
                    acc[j][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[j][tp], acc[j][dt], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(kVmcnt0); // this wave's part of the next tile has landed
        __syncthreads();                      // ... every wave's, and this tile's buffer is free
    };
    issue_tile(0, ks0, vt0);
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    for (int kt = 0; kt < ntile; kt += 2) {
        tile_step(kt, ks0, vt0, ks1, vt1);
        if (kt + 1 < ntile) tile_step(kt + 1, ks1, vt1, ks0, vt0);
    }

    // Output: the wave's normalised fp16 rows go through LDS (the K/V
    // buffers are free after the last barrier; wave w uses the w-th of the
    // four, rows padded by 8 halves), then every lane stores 16 contiguous
    // bytes and each group of D/8 lanes one whole row -- full cache lines
    // instead of 8-byte pieces of 16 rows per store.
    constexpr int OP = D + 8;        // staged row pitch (halves)
    constexpr int R = 16 * NQG;      // rows of the wave
    constexpr int PPR = D / 8;       // 16-byte pieces per row
    constexpr int NCH = R * PPR / 64; // pieces per lane
    // Staging: 8-wave workgroups up to head_dim 128 a region of its own (the
    // workgroup has the CU's LDS to itself); 4-wave ones (two per CU) reuse
    // the K/V buffers, one wave per buffer (head_dim 256: two).
    constexpr bool OWN = D <= 128 && NW == 8;
    __shared__ __align__(16) uint16_t own_stg[OWN ? NW * R * OP : 8];
    static_assert(OWN || ((NW + 3) / 4) * R * OP <= kKeyTile * ROWH, "staging fits the K/V buffers");
    uint16_t *stg;
    if constexpr (OWN) {
        stg = own_stg + wave * R * OP;
    } else {
        const int w4 = wave & 3;
        stg = (w4 == 0 ? ks0 : (w4 == 1 ? ks1 : (w4 == 2 ? vt0 : vt1))) + (wave >> 2) * R * OP;
    }
#pragma unroll
    for (int j = 0; j < NQG; ++j) {
        const float inv = 1.0f / (l_run[j][0] + 1e-6f);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const __half2 lo = __floats2half2_rn(acc[j][dt][0] * inv, acc[j][dt][1] * inv);
            const __half2 hi = __floats2half2_rn(acc[j][dt][2] * inv, acc[j][dt][3] * inv);
            uint2         w;
            w.x = __builtin_bit_cast(uint32_t, lo);
            w.y = __builtin_bit_cast(uint32_t, hi);
            *reinterpret_cast<uint2 *>(&stg[(j * 16 + c) * OP + 16 * dt + 4 * qg]) = w;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
        const int k = u * 64 + lane;
        const int rr = k / PPR, pc = k - rr * PPR;
        const int r = wave * R + rr; // workgroup row: token r / G, head r % G of kv group g
        const int qi = qt * BQ + r / G;
        if (qi < n) {
            const int64_t o = q_off + (int64_t)qi * a.q_tok + (int64_t)(g * G + r % G) * a.q_head + 8 * pc;
            *reinterpret_cast<uint4 *>(a.out + o) = *reinterpret_cast<const uint4 *>(&stg[rr * OP + 8 * pc]);
        }
    }
}

// softmax_kernel (attention.cu:288-343): one workgroup per row.
__global__ __launch_bounds__(256) void softmax_kernel(const __half *in, __half *out, int S) {
    __shared__ float red[8];
    const __half *x = in + (int64_t)blockIdx.x * S;
    __half       *y = out + (int64_t)blockIdx.x * S;
    const int     tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float         m = -FLT_MAX;
    for (int i = tid; i < S; i += 256) m = fmaxf(m, __half2float(x[i]));
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    constexpr float kLog2e = 1.4426950408889634f;
    float           sum = 0.0f;
    for (int i = tid; i < S; i += 256) sum += exp2f((__half2float(x[i]) - m) * kLog2e);
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    if (lane == 0) red[4 + wave] = sum;
    __syncthreads();
    sum = (red[4] + red[5]) + (red[6] + red[7]);
    const float inv = 1.0f / (sum + 1e-6f);
    for (int i = tid; i < S; i += 256)
        y[i] = __float2half(materialize(exp2f((__half2float(x[i]) - m) * kLog2e) * inv));
}

// get_attention_weights_kernel (attention.cu:240-268): one thread per
// (query, key) score, the reference's sequential fmaf order over d, then
// score * scale rounded to fp32 and to fp16.
__global__ __launch_bounds__(256) void attention_weights_kernel(const __half *q, const __half *k,
                                                                __half *w, float scale, int H,
                                                                int Lq, int Lk, int D, int causal) {
    const int     i = blockIdx.y, bh = blockIdx.z;
    const int     p = blockIdx.x * 256 + threadIdx.x;
    if (p >= Lk) return;
    const __half *qr = q + ((int64_t)bh * Lq + i) * D;
    const __half *kr = k + ((int64_t)bh * Lk + p) * D;
    float         v = 0.0f;
    if (!(causal && p > i)) {
        float score = 0.0f;
        for (int d = 0; d < D; ++d) score = fmaf(__half2float(qr[d]), __half2float(kr[d]), score);
        v = materialize(score * scale);
    }
    w[((int64_t)bh * Lq + i) * Lk + p] = __float2half(v);
    (void)H;
}

template <int D, int G, int NW>
void launch_dgw(const PrefillArgs &a, int grid, bool paged, hipStream_t stream) {
    if (paged)
        hipLaunchKernelGGL((attn_prefill_kernel<D, G, true, NW>), dim3(grid), dim3(NW * 64), 0, stream, a);
    else
        hipLaunchKernelGGL((attn_prefill_kernel<D, G, false, NW>), dim3(grid), dim3(NW * 64), 0, stream, a);
}

template <int D, int G>
void launch_dg(const PrefillArgs &a, int grid, int waves, bool paged, hipStream_t stream) {
    if constexpr (D <= 128) {
        if (waves == 8) {
            launch_dgw<D, G, 8>(a, grid, paged, stream);
            return;
        }
    }
    launch_dgw<D, G, 4>(a, grid, paged, stream);
}

template <int D>
void launch_d(const PrefillArgs &a, int grid, int G, int waves, bool paged, hipStream_t stream) {
    switch (G) {
    case 1: launch_dg<D, 1>(a, grid, waves, paged, stream); break;
    case 2: launch_dg<D, 2>(a, grid, waves, paged, stream); break;
    case 4: launch_dg<D, 4>(a, grid, waves, paged, stream); break;
    case 8: launch_dg<D, 8>(a, grid, waves, paged, stream); break;
    default: break;
    }
}

// TL_PREFILL_WAVES ("4" / "8") at first use, else auto; set_prefill_waves
// overrides it.
std::atomic<int> g_prefill_waves{-1};

// The rule of prefill_waves over the 8-wave tiling's items (x Hkv) and
// their attended keys.
int waves_rule(int D, int64_t items, int64_t keys, int Hkv, int cus) {
    if (D > 128) return 4;
    const int setting = prefill_waves_setting();
    if (setting == 4 || setting == 8) return setting;
    if (D == 64) return 4; // three 4-wave workgroups per CU against one 8-wave one
    if (D != 128 || items <= 0) return 8;
    const bool many = items * Hkv >= (int64_t)kPrefill4wItemsPerCU * std::max(1, cus);
    const bool short_items = keys <= (int64_t)kPrefill4wMeanKeys * items;
    return many && short_items ? 4 : 8;
}

} // namespace

bool prefill_shape_supported(int D, int G) {
    return (D == 32 || D == 64 || D == 128 || D == 256) && (G == 1 || G == 2 || G == 4 || G == 8);
}

void set_prefill_waves(int waves) { g_prefill_waves.store(waves); }

int prefill_waves_setting() {
    int v = g_prefill_waves.load(std::memory_order_relaxed);
    if (v < 0) {
        const char *e = std::getenv("TL_PREFILL_WAVES");
        v = 0;
        if (e && std::strcmp(e, "4") == 0) v = 4;
        if (e && std::strcmp(e, "8") == 0) v = 8;
        g_prefill_waves.store(v);
    }
    return v;
}

int prefill_waves(const PrefillEntry *entries, int n, int D, int G, int Hkv, int cus) {
    const int BQ = prefill_block_tokens(D, G, 8);
    int64_t   items = 0, keys = 0;
    for (int e = 0; e < n; ++e) {
        const int nqt = (entries[e].n + BQ - 1) / BQ;
        items += nqt;
        for (int qt = 0; qt < nqt; ++qt) keys += (int64_t)entries[e].p0 + std::min(entries[e].n, (qt + 1) * BQ);
    }
    return waves_rule(D, items, keys, Hkv, cus);
}

int prefill_waves_uniform(int B, int S, int D, int G, int Hkv, int cus) {
    const int     BQ = prefill_block_tokens(D, G, 8);
    const int64_t nqt = (S + BQ - 1) / BQ;
    int64_t       keys = 0;
    for (int64_t qt = 0; qt < nqt; ++qt) keys += std::min<int64_t>(S, (qt + 1) * BQ);
    return waves_rule(D, (int64_t)B * nqt, (int64_t)B * keys, Hkv, cus);
}

void plan_prefill(const PrefillEntry *entries, int n, int D, int G, int waves, std::vector<int32_t> &work) {
    const int BQ = prefill_block_tokens(D, G, waves);
    struct It {
        int64_t keys;
        int32_t e, qt;
    };
    std::vector<It> items;
    for (int e = 0; e < n; ++e) {
        const int nqt = (entries[e].n + BQ - 1) / BQ;
        for (int qt = 0; qt < nqt; ++qt)
            items.push_back({(int64_t)entries[e].p0 + std::min(entries[e].n, (qt + 1) * BQ), e, qt});
    }
    std::stable_sort(items.begin(), items.end(), [](const It &x, const It &y) { return x.keys > y.keys; });
    work.assign(kPrefillItemWords * items.size(), 0);
    for (size_t i = 0; i < items.size(); ++i) {
        const PrefillEntry &E = entries[items[i].e];
        int32_t            *w = &work[kPrefillItemWords * i];
        w[0] = (int32_t)(uint32_t)((uint64_t)E.q_off & 0xffffffffu);
        w[1] = (int32_t)(uint32_t)((uint64_t)E.q_off >> 32);
        w[2] = E.p0;
        w[3] = E.n;
        w[4] = E.row;
        w[5] = items[i].qt;
        w[6] = E.tok0;
    }
}

void launch_attn_prefill(const PrefillLaunch &p, const KvView &kv, int Hq, int Hkv, int D,
                         float scale, hipStream_t stream) {
    const int G = Hq / Hkv;
    int       items, waves;
    if (p.work) {
        items = p.n_items;
        waves = p.waves;
        if (waves != 4 && !(waves == 8 && D <= 128))
            throw std::invalid_argument("attention_prefill: the work list's waves per workgroup must be 4, or 8 "
                                        "up to head_dim 128");
    } else {
        waves = prefill_waves_uniform(p.uniform_b, p.uniform_n, D, G, Hkv, device_cus());
        const int BQ = prefill_block_tokens(D, G, waves);
        items = p.uniform_b * ((p.uniform_n + BQ - 1) / BQ);
    }
    if (items <= 0) return;
    PrefillArgs a;
    a.q = p.q;
    a.out = p.out;
    a.kv = kv;
    a.work = p.work;
    a.q_tok = p.q_tok_stride;
    a.q_head = p.q_head_stride;
    a.q_entry = p.q_entry_stride;
    a.uniform_b = p.uniform_b;
    a.uniform_n = p.uniform_n;
    if ((p.new_k != nullptr) != (p.new_v != nullptr) || (p.new_k && !p.work))
        throw std::invalid_argument("attention_prefill: the fused append needs new_k, new_v and a work list");
    a.new_k = p.new_k;
    a.new_v = p.new_v;
    a.Hkv = Hkv;
    a.scale_log2 = scale * 1.4426950408889634f;
    const int64_t grid = (int64_t)items * Hkv;
    if (grid > INT32_MAX) throw std::invalid_argument("attention_prefill: too many work items");
    const bool paged = kv.block_table != nullptr;
    if (!paged && (int64_t)p.max_keys * kv.tok_stride * 2 > (int64_t)UINT32_MAX)
        throw std::invalid_argument("attention_prefill: token offsets exceed 32 bits (keys * row bytes)");
    profile_begin(KernelId::AttnPrefill, stream);
    switch (D) {
    case 32: launch_d<32>(a, (int)grid, G, waves, paged, stream); break;
    case 64: launch_d<64>(a, (int)grid, G, waves, paged, stream); break;
    case 128: launch_d<128>(a, (int)grid, G, waves, paged, stream); break;
    case 256: launch_d<256>(a, (int)grid, G, waves, paged, stream); break;
    default: break;
    }
    HIP_CHECK(hipGetLastError());
    profile_end(KernelId::AttnPrefill, stream);
}

void launch_softmax(const __half *in, __half *out, int rows, int S, hipStream_t stream) {
    if (rows <= 0 || S <= 0) return;
    hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(256), 0, stream, in, out, S);
    HIP_CHECK(hipGetLastError());
}

void launch_attention_weights(const __half *q, const __half *k, __half *w, float scale, int B,
                              int H, int Lq, int Lk, int D, bool causal, hipStream_t stream) {
    if (B <= 0 || H <= 0 || Lq <= 0 || Lk <= 0 || D <= 0) return;
    dim3 grid((unsigned)((Lk + 255) / 256), (unsigned)Lq, (unsigned)(B * H));
    hipLaunchKernelGGL(attention_weights_kernel, grid, dim3(256), 0, stream, q, k, w, scale, H, Lq,
                       Lk, D, causal ? 1 : 0);
    HIP_CHECK(hipGetLastError());
}

} // namespace detail
} // namespace tiny_llm
