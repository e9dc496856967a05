// Launch interface of the prefill-side attention kernels (gfx950):
// causal attention of new query tokens over a KV view (the cache-native
// prefill, and the reference's compact attention_prefill), plus the
// reference's test-side softmax and attention-weights kernels.
#pragma once

#include "kv_kernels.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <vector>

namespace tiny_llm {
namespace detail {

// One sequence of a prefill call: its n new query tokens sit at positions
// p0 .. p0+n-1 of cache row `row`; query token i, head h is at
// q + q_off + i * q_tok_stride + h * q_head_stride (out likewise), and it
// attends to the keys at positions 0 .. p0+i of that row.  tok0: index of
// its first token in the call's token batch (the row of new_k / new_v when
// the append is fused).
struct PrefillEntry {
    int64_t q_off;
    int32_t p0;
    int32_t n;
    int32_t row;
    int32_t tok0;
};

static_assert(sizeof(PrefillEntry) == 24, "six 32-bit words per entry");

// Query rows (token, head) per workgroup of `waves` waves: 16 per query group,
// two groups per wave up to head_dim 128, one at 256.  Up to head_dim 128 a
// workgroup has 8 waves (256 rows, one workgroup per CU) or 4 (128 rows, two
// per CU); head_dim 256 has 4 (64 rows).
constexpr int prefill_rows(int D, int waves) { return waves * 16 * (D <= 128 ? 2 : 1); }
// Query tokens per workgroup: G heads of one kv group per token.
inline int prefill_block_tokens(int D, int G, int waves) { return prefill_rows(D, waves) / G; }

// Waves per workgroup of a prefill launch over `entries`, with Hkv kv heads
// (the grid is items x Hkv) on `cus` CUs: the process setting when it forces
// 4 or 8 (head_dim <= 128; head_dim 256 is always 4); else 4 at head_dim 64
// (its ~144 VGPRs per wave let a CU run three 4-wave workgroups but only one
// 8-wave one: 4 waves measured 6-24% faster on every shape tried, 32 / 8 and
// 32 / 4 heads, prompts of 256 to 8192 tokens, with and without a cached
// prefix), 8 at head_dim 32 (mixed: -16% to +28%); at head_dim 128,
// 4 when the 8-wave tiling gives every CU at least kPrefill4wItemsPerCU
// items and they attend at most kPrefill4wMeanKeys keys on average (many
// short items: a workgroup's start-up -- work record, q, first tile -- is a
// large part of each, and two 4-wave workgroups per CU run one's start-up
// under the other's tiles), else 8 (longer items pay for the 4-wave form's
// doubled K/V tile traffic per row; few items leave nothing to overlap).
// Measured at Llama-3-8B heads (32 / 8, head_dim 128), µs per launch, 8 / 4
// waves: 16 x 512 prompts 81.1 / 74.2, 32 x 256 66.1 / 60.9, 4 x 1536 99.5 /
// 96.0, 8 x 1024 96.6 / 94.5; 8 x 512 (two items per CU) 38.4 / 41.6, 4 x
// 2048 152 / 157, 1 x 8192 518 / 551, 16 x 512 after 1024 cached tokens
// 193 / 206.
constexpr int kPrefill4wItemsPerCU = 3;
constexpr int kPrefill4wMeanKeys = 800;
int prefill_waves(const PrefillEntry *entries, int n, int D, int G, int Hkv, int cus);
// The same rule for `B` entries of S new tokens each and no cached prefix.
int prefill_waves_uniform(int B, int S, int D, int G, int Hkv, int cus);
// Process setting: 0 = auto (the rule above), 4 or 8; initial value from the
// environment variable TL_PREFILL_WAVES ("4" / "8"), else 0.
void set_prefill_waves(int waves);
int  prefill_waves_setting();

// Work items (entry, query tile of prefill_block_tokens(D, G, waves) tokens),
// most keys first (LPT order for the hardware dispatcher), each a
// self-contained record of kPrefillItemWords 32-bit words: {q_off low, q_off
// high, p0, n, row, query tile, tok0, 0}, so a workgroup needs one dependent
// load before its Q and K/V loads.  The launch must use the same waves.
constexpr int kPrefillItemWords = 8;
void plan_prefill(const PrefillEntry *entries, int n, int D, int G, int waves, std::vector<int32_t> &work);

struct PrefillLaunch {
    const __half       *q = nullptr;
    __half             *out = nullptr;
    int64_t             q_tok_stride = 0;
    int64_t             q_head_stride = 0;
    // Either a device work list of n_items records (plan_prefill; 32-byte
    // aligned) with the waves per workgroup it was planned for ...
    const int32_t      *work = nullptr;
    int                 n_items = 0;
    int                 waves = 0;
    // ... or, with work == NULL, `uniform_b` entries b with p0 = 0,
    // n = uniform_n, row = b and q_off = b * q_entry_stride (waves by
    // prefill_waves_uniform).
    int                 uniform_b = 0;
    int                 uniform_n = 0;
    int64_t             q_entry_stride = 0;
    // Largest p0 + n over the entries (the offset-width check of
    // contiguous rows).
    int                 max_keys = 0;
    // Fused append (work-list launches only): the new tokens' K/V rows,
    // [tokens][Hkv * D].  Keys at positions >= p0 are then read from here,
    // and the workgroup of each query tile writes its own tokens' rows of
    // its kv head into the cache -- the bytes of appendKV -- so the cache
    // holds them when the kernel ends.  Null: every key from the cache.
    const __half       *new_k = nullptr;
    const __half       *new_v = nullptr;
};

// True when (D, G) has a prefill kernel (D in {32,64,128,256}, G in {1,2,4,8}).
bool prefill_shape_supported(int D, int G);

// Throws HipException on launch failure, std::invalid_argument when the
// token offsets of a contiguous (non-paged) view do not fit in 32 bits.
void launch_attn_prefill(const PrefillLaunch &p, const KvView &kv, int Hq, int Hkv, int D,
                         float scale, hipStream_t stream);

// softmax (attention.cu:288-354): rows of S fp16 values.
void launch_softmax(const __half *in, __half *out, int rows, int S, hipStream_t stream);

// get_attention_weights (attention.cu:240-286): [B][H][Lq][Lk] = fp16(scale * q.k),
// zero above the diagonal when causal.
void launch_attention_weights(const __half *q, const __half *k, __half *w, float scale, int B,
                              int H, int Lq, int Lk, int D, bool causal, hipStream_t stream);

} // namespace detail
} // namespace tiny_llm
