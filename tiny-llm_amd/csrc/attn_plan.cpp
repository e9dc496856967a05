// Host-side planner of the split-K decode attention launch (see attn_plan.h).
#include "attn_plan.h"

#include <algorithm>
#include <functional>
#include <climits>
#include <cstdlib>
#include <cstring>

namespace tiny_llm {
namespace detail {

// With W = sum(lens) * Hkv token-heads of work, C CUs and P = C *
// kPlanSlotsPerCU resident workgroup slots:
//  - uniform lengths: chunks of W / C (rounded up), one round of 8-wave
//    workgroups, one per CU -- usually the whole sequence, hence no partials.
//    Where a split is needed (few long sequences), one round of items twice
//    as long beats two rounds: the second round's start-up and the shorter
//    items' ramp and drain cost more than they balance (B = 1, 32 heads,
//    8192 tokens: 26.9 against 32.8 us per call);
//  - ragged lengths no longer than the per-CU share W / C: no split (the
//    workgroups sharing a CU share its bandwidth, and longest-first ordering
//    balances the CUs without partials or a merge launch);
//  - longer ragged lengths: chunks of W / (2P), so that longest-first list
//    scheduling ends within about one small item of the ideal;
//  - but no split at all when the longest length is at most two tiles per
//    wave of an 8-wave workgroup (kPlanShortLen): the unsplit launch is then a
//    couple of tile latencies long, and a split would only add the merge
//    launch.
int plan_chunk(const int32_t *lens, int n, int num_kv_heads, int uniform_len, int cus,
               int forced_chunk) {
    int64_t total = 0;
    int     mx = 0, mn = INT_MAX;
    for (int i = 0; i < (lens ? n : 0); ++i) {
        total += lens[i];
        mx = std::max(mx, (int)lens[i]);
        mn = std::min(mn, (int)lens[i]);
    }
    if (!lens) {
        total = (int64_t)n * uniform_len;
        mx = mn = uniform_len;
    }
    const int cap = std::max(kPlanQuantum, (mx + kPlanQuantum - 1) / kPlanQuantum * kPlanQuantum);
    if (forced_chunk >= kPlanQuantum && forced_chunk % kPlanQuantum == 0)
        return std::min(forced_chunk, cap);
    const int64_t c = std::max(1, cus);
    const int64_t slots = c * kPlanSlotsPerCU;
    const int64_t work = total * num_kv_heads;
    const bool    uniform = mn >= mx - mx / 10;
    int64_t       per;
    if (mx <= kPlanShortLen) per = mx;
    else if (uniform) per = (work + c - 1) / c;
    else if (mx <= (work + c - 1) / c) per = mx;
    else per = (work + slots - 1) / slots / 2;
    const int64_t chunk = (per + kPlanQuantum - 1) / kPlanQuantum * kPlanQuantum;
    return (int)std::min<int64_t>(std::max<int64_t>(chunk, kPlanQuantum), cap);
}

namespace {

// Items per entry of a head-fused plan with hpw heads per workgroup, or 0
// when it does not apply (see plan_head_fused).
int fused_items(int n, int num_kv_heads, int cus, int mn, int hpw) {
    if (num_kv_heads % hpw != 0) return 0;
    const int64_t groups = (int64_t)n * (num_kv_heads / hpw);
    if (groups > cus) return 0;
    const int slices = kPlanFusedWaves / hpw; // waves per head
    const int nch = (int)std::min<int64_t>(std::min<int64_t>(cus / groups, kPlanFusedMaxItems),
                                           std::max(1, mn / (8 * kPlanTile * slices)));
    return groups * nch * 10 >= (int64_t)cus * 9 ? nch : 0;
}

} // namespace

bool plan_head_fused(const int32_t *lens, int n, int num_kv_heads, int cus, int head_fuse,
                     WorkList &out) {
    if (!head_fuse || !lens || n <= 0 || cus <= 0) return false;
    int mx = 0, mn = INT_MAX;
    for (int i = 0; i < n; ++i) {
        mx = std::max(mx, (int)lens[i]);
        mn = std::min(mn, (int)lens[i]);
    }
    if (mn < 1 || mn < mx - mx / 10) return false;
    int hpw = 0, nch = 0;
    if (head_fuse == 2 || head_fuse == 4 || head_fuse == 8) {
        hpw = head_fuse;
        nch = fused_items(n, num_kv_heads, cus, mn, hpw);
    } else {
        for (const int h : {8, 4, 2}) { // fewest items; more heads on a tie
            const int c = fused_items(n, num_kv_heads, cus, mn, h);
            if (c && (!nch || c < nch)) {
                hpw = h;
                nch = c;
            }
        }
    }
    if (!nch) return false;
    out.fused_heads = hpw;
    out.chunk = std::max(kPlanQuantum, (mx + kPlanQuantum - 1) / kPlanQuantum * kPlanQuantum);
    out.max_len = mx;
    out.any_multi = nch > 1;
    out.any_empty = false;
    out.n_work = n * nch;
    out.part_base.resize((size_t)n + 1);
    for (int i = 0; i <= n; ++i) out.part_base[(size_t)i] = i * nch;
    out.work.resize(2 * (size_t)out.n_work);
    size_t w = 0;
    for (int c = 0; c < nch; ++c)
        for (int i = 0; i < n; ++i) {
            out.work[w++] = i;
            out.work[w++] = c;
        }
    return true;
}

namespace {

// The chunk items of out.chunk over lens: part_base, and the work list
// sorted by item length descending (then entry, chunk).
void chunk_items(const int32_t *lens, int n, WorkList &out) {
    out.part_base.assign((size_t)std::max(n, 0) + 1, 0);
    out.any_multi = false;
    out.any_empty = false;
    out.max_len = 0;
    for (int i = 0; i < n; ++i) {
        const int c = (lens[i] + out.chunk - 1) / out.chunk;
        out.any_multi |= c > 1;
        out.any_empty |= c == 0;
        out.max_len = std::max(out.max_len, (int)lens[i]);
        out.part_base[(size_t)i + 1] = out.part_base[(size_t)i] + c;
    }
    out.n_work = out.part_base[(size_t)std::max(n, 0)];
    // (length, entry, chunk) sorted by length descending, then entry, chunk.
    std::vector<int64_t> key((size_t)out.n_work);
    size_t               k = 0;
    for (int i = 0; i < n; ++i)
        for (int c = 0; c < out.part_base[(size_t)i + 1] - out.part_base[(size_t)i]; ++c) {
            const int len = std::min(out.chunk, lens[i] - c * out.chunk);
            // larger length first; ties keep (entry, chunk) order
            key[k++] = ((int64_t)(INT32_MAX - len) << 32) | (int64_t)(out.part_base[(size_t)i] + c);
        }
    std::sort(key.begin(), key.end());
    out.work.resize(2 * (size_t)out.n_work);
    // part_base is non-decreasing: entry of partial row r = last i with part_base[i] <= r
    for (size_t w = 0; w < key.size(); ++w) {
        const int32_t row = (int32_t)(key[w] & 0xffffffff);
        const int     i = (int)(std::upper_bound(out.part_base.begin(), out.part_base.end(), row) -
                            out.part_base.begin()) - 1;
        out.work[2 * w] = i;
        out.work[2 * w + 1] = row - out.part_base[(size_t)i];
    }
}

// Longest-first schedule, in whole tile rounds (one 64-token tile per wave),
// of the workgroups of items with lengths lens_desc (longest first),
// per_item workgroups each, on `cus` CUs (one workgroup at a time each),
// where a workgroup of an item of len tokens takes ceil(ceil(len / 64) /
// waves_per_head) rounds: its makespan R and the number of CUs still busy in
// round R, as the key R * (cus + 1) + busy (smaller: ends sooner; with as
// many rounds, fewer CUs share the last one).  The hardware dispatcher hands
// the next workgroup to the first CU that frees up, which is this greedy
// assignment to the least loaded CU; loads are small integers, so the CUs are
// counted per load level.
int64_t lpt_rounds(const std::vector<int> &lens_desc, int per_item, int waves_per_head, int cus) {
    cus = std::max(1, cus);
    std::vector<int> at(1, cus); // at[l]: CUs with load l
    int              lo = 0, top = 0;
    for (const int len : lens_desc) {
        const int w = ((len + kPlanTile - 1) / kPlanTile + waves_per_head - 1) / waves_per_head;
        for (int k = 0; k < per_item; ++k) {
            while (at[(size_t)lo] == 0) ++lo;
            --at[(size_t)lo];
            const int l = lo + w;
            if ((int)at.size() <= l) at.resize((size_t)l + 1, 0);
            ++at[(size_t)l];
            top = std::max(top, l);
        }
    }
    return (int64_t)top * (cus + 1) + at[(size_t)top];
}

// Items of chunk c over lens: per entry, full chunks of c tokens and the
// remainder, longest first.
std::vector<int> chunk_lengths(const int32_t *lens, int n, int c) {
    std::vector<int> v;
    for (int i = 0; i < n; ++i) {
        for (int t = 0; t < lens[i]; t += c) v.push_back(std::min(c, lens[i] - t));
    }
    std::sort(v.begin(), v.end(), std::greater<int>());
    return v;
}

} // namespace

int plan_balanced_split(const int32_t *lens, int n, int num_kv_heads, int cus) {
    if (!lens || n <= 0 || cus <= 0 || num_kv_heads % 2 != 0) return 0;
    int64_t total = 0;
    int     mx = 0;
    for (int i = 0; i < n; ++i) {
        total += std::max(0, (int)lens[i]);
        mx = std::max(mx, (int)lens[i]);
    }
    if (mx <= kPlanShortLen) return 0;
    std::vector<int> whole(lens, lens + n);
    std::sort(whole.begin(), whole.end(), std::greater<int>());
    const int64_t r0 = lpt_rounds(whole, num_kv_heads, 8, cus);
    // a CU's share of the head pairs' tokens, rounded up
    const int64_t share = (total * (num_kv_heads / 2) + cus - 1) / cus;
    int64_t       lo = (share + kPlanQuantum - 1) / kPlanQuantum * kPlanQuantum;
    lo = std::max<int64_t>(lo, kPlanQuantum);
    // at most kPlanSplitCandidates chunk lengths, evenly strided (host cost)
    const int64_t stride = std::max<int64_t>(
        kPlanQuantum, ((mx - lo) / kPlanSplitCandidates + kPlanQuantum - 1) / kPlanQuantum * kPlanQuantum);
    int           best = 0;
    int64_t       best_r = r0;
    for (int64_t c = lo; c < mx; c += stride) {
        const int64_t r = lpt_rounds(chunk_lengths(lens, n, (int)c), num_kv_heads / 2, 4, cus);
        if (r < best_r || (r == best_r && best)) { // ends soonest; the longest chunk on a tie
            best_r = r;
            best = (int)c;
        }
    }
    return best; // nonzero only when it ends before the whole sequences
}

void plan_work_list(const int32_t *lens, int n, int num_kv_heads, int cus, int forced_chunk,
                    int head_fuse, WorkList &out) {
    if (forced_chunk == 0 && plan_head_fused(lens, n, num_kv_heads, cus, head_fuse, out)) {
        out.fused_chunked = false;
        return;
    }
    out.fused_heads = 0;
    out.fused_chunked = false;
    out.chunk = plan_chunk(lens, n, num_kv_heads, 0, cus, forced_chunk);
    chunk_items(lens, n, out);
    // Whole sequences in per-head 8-wave workgroups at most two per CU: a
    // head-pair chunk plan when its longest-first schedule ends sooner
    // (plan_balanced_split).
    if (forced_chunk == 0 && head_fuse == 1 && !out.any_multi && out.n_work > 0 &&
        plan_waves((int64_t)out.n_work * num_kv_heads, cus, 0) == 8) {
        const int c = plan_balanced_split(lens, n, num_kv_heads, cus);
        if (c) {
            out.chunk = c;
            chunk_items(lens, n, out);
            out.fused_heads = 2;
            out.fused_chunked = true;
            return;
        }
    }
    // Head-fused over the chunk items: forced heads per workgroup, or (auto)
    // two heads per 8-wave workgroup where the per-head plan takes 4-wave
    // workgroups -- as many waves per head, two heads' pieces of each row
    // read together.  (Where per-head workgroups have 8 waves, fusing would
    // halve the workgroups and unbalance ragged lengths.)
    if ((head_fuse == 2 || head_fuse == 4 || head_fuse == 8) && num_kv_heads % head_fuse == 0) {
        out.fused_heads = head_fuse;
        out.fused_chunked = true;
    } else if (head_fuse == 1 && num_kv_heads % 2 == 0 && out.n_work > 0 &&
               plan_waves((int64_t)out.n_work * num_kv_heads, cus, 0) == 4) {
        out.fused_heads = 2;
        out.fused_chunked = true;
        // These workgroups run one per CU where the per-head ones ran two:
        // chunks kFusedChunkNum / kFusedChunkDen as long (capped at the
        // longest length), fewer items and partials.
        if (forced_chunk == 0 && out.any_multi) {
            const int64_t c2 = ((int64_t)out.chunk * kFusedChunkNum / kFusedChunkDen + kPlanQuantum - 1) /
                               kPlanQuantum * kPlanQuantum;
            const int cap = (out.max_len + kPlanQuantum - 1) / kPlanQuantum * kPlanQuantum;
            const int chunk = (int)std::min<int64_t>(c2, cap);
            if (chunk != out.chunk) {
                out.chunk = chunk;
                chunk_items(lens, n, out);
            }
        }
    }
}

int plan_waves(int64_t workgroups, int cus, int setting) {
    if (setting == 4 || setting == 8) return setting;
    return workgroups <= 2 * (int64_t)std::max(1, cus) ? 8 : 4;
}

int chunk_override_from_env() {
    const char *env = std::getenv("TL_ATTN_CHUNK");
    if (!env) return 0;
    const int c = std::atoi(env);
    return c >= kPlanQuantum && c % kPlanQuantum == 0 ? c : 0;
}

int inline_words(const WorkList &plan, int n, bool with_rows) {
    return n + (n + 1) + 2 * plan.n_work + (with_rows ? n : 0);
}

int inline_words_compact(const int32_t *lens, const WorkList &plan, const int32_t *rows, int n) {
    if (n <= 0 || n > 0xffff || plan.any_multi || plan.any_empty || plan.n_work != n) return -1;
    for (int i = 0; i < n; ++i) {
        if (lens[i] < 0 || lens[i] > 0xffff) return -1;
        const int r = rows ? rows[i] : i;
        if (r < 0 || r > 0xffff) return -1;
    }
    return n + (n + 1) / 2;
}

bool pack_inline(const int32_t *lens, const WorkList &plan, const int32_t *rows, int n,
                 InlineMeta &out) {
    const int words = inline_words(plan, n, rows != nullptr);
    if (n > 0 && words > kInlineWords) {
        const int cw = inline_words_compact(lens, plan, rows, n);
        if (cw < 0 || cw > kInlineWords) return false;
        out.n = n;
        out.compact = 1;
        out.has_rows = 1;
        out.off_part = 0;
        out.off_rows = 0;
        out.off_work = n;
        for (int i = 0; i < n; ++i)
            out.w[i] = (int32_t)((uint32_t)lens[i] | ((uint32_t)(rows ? rows[i] : i) << 16));
        for (int k = 0; k < (n + 1) / 2; ++k) out.w[n + k] = 0;
        for (int k = 0; k < n; ++k) {
            const uint32_t e = (uint32_t)plan.work[2 * (size_t)k]; // chunk 0 of entry e
            out.w[n + k / 2] = (int32_t)((uint32_t)out.w[n + k / 2] | (e << ((k & 1) * 16)));
        }
        return true;
    }
    if (n <= 0) return false;
    out.n = n;
    out.compact = 0;
    out.has_rows = rows ? 1 : 0;
    out.off_part = n;
    out.off_work = 2 * n + 1;
    out.off_rows = out.off_work + 2 * plan.n_work;
    std::memcpy(out.w, lens, (size_t)n * 4);
    std::memcpy(out.w + out.off_part, plan.part_base.data(), (size_t)(n + 1) * 4);
    if (plan.n_work) std::memcpy(out.w + out.off_work, plan.work.data(), (size_t)plan.n_work * 8);
    if (rows) std::memcpy(out.w + out.off_rows, rows, (size_t)n * 4);
    return true;
}

} // namespace detail
} // namespace tiny_llm
