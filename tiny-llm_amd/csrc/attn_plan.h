// Host-side planner of the split-K decode attention launch: chunk length,
// work list, waves per workgroup and the kernel-argument packing of the
// per-step metadata.  Plain C++ (no HIP types), so the same code is built
// into the library and, under the address and undefined-behaviour
// sanitizers, into a host test.
#pragma once

#include <cstdint>
#include <vector>

namespace tiny_llm {
namespace detail {

constexpr int kPlanTile = 64;                  // tokens per wave tile
constexpr int kPlanQuantum = 4 * kPlanTile;    // chunk lengths are multiples of this
constexpr int kPlanSlotsPerCU = 2;             // resident 4-wave workgroups per CU
constexpr int kPlanShortLen = 2 * 8 * kPlanTile; // never split lengths up to this
constexpr int kPlanFusedWaves = 8;             // waves of a head-fused workgroup
constexpr int kPlanFusedMaxItems = 8;          // head-fused items per entry, at most
constexpr int kFusedChunkNum = 3, kFusedChunkDen = 2; // chunk scale of head-fused chunk items
constexpr int kPlanSplitCandidates = 32;       // chunk lengths plan_balanced_split tries, at most

// Host side of a ragged plan: chunk length, per-entry partial-row bases and
// the (entry, chunk) work list in longest-first order, so the hardware
// dispatcher, which hands workgroups to CUs as they free up, schedules the
// longest items first (LPT list scheduling).
// Head-fused plans (fused_heads = H > 0): an 8-wave workgroup takes H kv
// heads of an item (wave w: head w % H, tile slice w / H), and the nch items
// of an entry interleave its 64-token tiles in nch * 8 / H slices instead of
// taking chunks; `chunk` is then the longest length rounded up to the
// quantum and the work list is in chunk-major order.
struct WorkList {
    int                  chunk = 256;
    int                  n_work = 0;
    int                  max_len = 0;
    bool                 any_multi = false;
    bool                 any_empty = false;
    int                  fused_heads = 0;
    bool                 fused_chunked = false; // head-fused over the chunk plan's items
    std::vector<int32_t> part_base; // n + 1
    std::vector<int32_t> work;      // 2 * n_work
};

// Chunk length (tokens per work item, a multiple of kPlanQuantum) for the
// attended lengths lens[0..n) (or n entries of uniform_len when lens is
// NULL) on a device of `cus` compute units.  forced_chunk > 0 (a multiple
// of kPlanQuantum) overrides the choice, capped at the longest length
// rounded up to the quantum.
int plan_chunk(const int32_t *lens, int n, int num_kv_heads, int uniform_len, int cus,
               int forced_chunk);

// The head-fused plan when it applies: head_fuse != 0 (the kernel has a
// head-fused form for this shape; 2, 4 or 8 force that many kv heads per
// workgroup, 1 lets the planner choose), lengths within 10% of the longest
// and at least 1.  With H heads per workgroup (H dividing num_kv_heads) and
// g = n * num_kv_heads / H (entry, head block) pairs, at most `cus`, each
// entry gets nch = cus / g interleaved items (one workgroup per CU, the
// launch one round), fewer if the shortest length has under 8 tiles per
// wave, at most kPlanFusedMaxItems; H applies only when g * nch fills at
// least 90% of the CUs.  The planner's choice is the H in {8, 4, 2} with the
// fewest items per entry (one: no merge launch), the larger H on a tie.
// Items are listed chunk-major, (entry 0, item 0), (entry 1, item 0), ...;
// the launch deals the head blocks of the item list out item-fastest.
// Returns false (out untouched) when no H applies.
bool plan_head_fused(const int32_t *lens, int n, int num_kv_heads, int cus, int head_fuse,
                     WorkList &out);

// Ragged lengths that the chunk rule leaves whole, in per-head 8-wave
// workgroups at most two per CU, can end far from the ideal: longest-first
// can only pair each CU's two heads of two sequences (B = 16 MHA sequences
// of 657..3948 tokens: 11 tile rounds against 8.35 of work per CU).  This is
// the chunk c of a head-pair chunk plan (2 kv heads per 8-wave workgroup, 4
// waves per head, each sequence in chunks of c and a remainder) that ends
// sooner in the longest-first schedule of lpt_rounds -- in fewer whole tile
// rounds (one 64-token tile per wave), or in as many with fewer CUs busy in
// the last one -- or 0: c is a multiple of kPlanQuantum from a CU's share of
// the head pairs' tokens (shorter chunks only add workgroups, partials and
// merge work) up to the longest length, at most kPlanSplitCandidates of them
// (evenly strided by a multiple of kPlanQuantum); among the soonest the
// longest c.
// At head_dim 128 on 256 CUs a round (every CU streaming 8 tiles) takes
// ~9.7 us, the merge launch the split needs ~5 us.  (That B = 16 set, 32
// layers, kernel us per layer, (rounds, CUs in the last): whole sequences
// 94.2 (11, 32); chunks of 2560 88.0 (10, 112); 2304 92.6 (11, 32); 2816
// 91.6 (11, 80); 3072 95.3 (12, 80); 3328 99.0; 3584 102.5; end to end the
// 2560 split is the one ahead of whole sequences, also 18 steps later, when
// it is (11, 16) against (11, 64).)
int plan_balanced_split(const int32_t *lens, int n, int num_kv_heads, int cus);

// The whole ragged plan (chunk, part_base, work list) for lens[0..n): the
// head-fused plan when it applies and no chunk is forced, else chunks --
// head-fused over the chunk items (fused_chunked) when head_fuse forces 2, 4
// or 8 heads per workgroup, or, for head_fuse 1, with 2 heads per 8-wave
// workgroup where the per-head plan would take 4-wave workgroups or where
// plan_balanced_split finds a chunk (then of that length).
void plan_work_list(const int32_t *lens, int n, int num_kv_heads, int cus, int forced_chunk,
                    int head_fuse, WorkList &out);

// Waves per workgroup for a launch of `workgroups` workgroups: setting 4 or 8
// forces it; 0 (auto) gives 8 when every CU gets at most two workgroups in
// turn, else 4 (two 4-wave workgroups per CU).
int plan_waves(int64_t workgroups, int cus, int setting);

// TL_ATTN_CHUNK from the environment when it is a positive multiple of
// kPlanQuantum, else 0.
int chunk_override_from_env();

// Plan metadata small enough to travel in the kernel arguments, so that a
// launch needs no separate host-to-device copy.  Full encoding, words:
//   [lens n | part_base n+1 | work 2*n_work | rows n (if has_rows)]
// rows[b] is the cache row (slot) of entry b, replacing KvView::seq_row.
// Compact encoding (compact = 1), for plans where every entry is one work
// item (no split, no empty entry) and lengths and rows fit in 16 bits:
//   [len_b | row_b << 16, n words | launch order of the entries, 16 bits each]
// -- n + ceil(n/2) words, so up to 597 entries fit instead of 223.
constexpr int kInlineWords = 896;
struct InlineMeta {
    int32_t n = 0; // entries; 0 = metadata comes through the AttnPlan pointers
    int32_t has_rows = 0;
    int32_t off_part = 0;
    int32_t off_work = 0;
    int32_t off_rows = 0;
    int32_t compact = 0;
    int32_t w[kInlineWords];
};
// Words the full inline encoding of this plan needs.
int inline_words(const WorkList &plan, int n, bool with_rows);
// Words of the compact encoding, or -1 when the plan does not allow it.
int inline_words_compact(const int32_t *lens, const WorkList &plan, const int32_t *rows, int n);
// Packs lens / plan / rows (rows may be NULL) into out, in the full encoding
// when it fits, else in the compact one; false if neither fits.
bool pack_inline(const int32_t *lens, const WorkList &plan, const int32_t *rows, int n,
                 InlineMeta &out);

} // namespace detail
} // namespace tiny_llm
