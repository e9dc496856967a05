"""CPU: the decode attention launch planner (csrc/attn_plan.cpp) through the C
ABI (tl_attn_plan; host only, no GPU).

The plan decides which kernel path runs: chunk length (tokens per work
item), work items, waves per workgroup, split-K merge or not, metadata in the
kernel arguments or a device copy.  These tests pin the plans of the five
benchmark configurations on a 256-CU MI355X (the values the bench reports
and the GPU parity tests assert), and check the plan's invariants on random
length sets: every token of every sequence is covered by exactly one work
item, the work list is ordered longest first, and longest-first list
scheduling of the items on the device's workgroup slots ends within one
item of the ideal."""
import heapq

import numpy as np
import pytest

import workloads

CUS = 256


@pytest.fixture(scope="module")
def tl():
    import tinyllm_kv
    tinyllm_kv.load()
    return tinyllm_kv


def churn_snapshot(n_live=585, seed=5):
    """Attended lengths of a config-5 step with n_live live sequences:
    prompts U{256..4096} plus up to 600 decoded tokens each."""
    rng = np.random.default_rng(workloads.seed(5, 3) + seed)
    return (rng.integers(256, 4097, n_live) + rng.integers(0, 600, n_live) + 1).astype(np.int32)


# (config, attended lengths, kv heads) -> expected (chunk, items, waves,
# merge launch, inline words or -1)
def cases():
    out = {}
    for c in (1, 2, 3, 4):
        cfg = workloads.config(c)
        out[f"cfg{c}"] = (cfg.contexts.astype(np.int32) + 1, cfg.hkv)
    out["cfg5"] = (churn_snapshot(), 8)
    return out


EXPECTED = {
    # cfg1: 4 MHA sequences of 129..513 tokens, at most two tiles per wave of
    # an 8-wave workgroup: no split (a merge launch would cost more than it
    # saves), one 768-token chunk each
    "cfg1": dict(chunk_tokens=768, work_items=4, waves=8, any_multi=0, inline_words=21),
    # cfg2: ragged, every length within the per-CU share: one chunk each
    "cfg2": dict(chunk_tokens=4096, work_items=16, waves=8, any_multi=0, inline_words=81),
    # cfg3 (headline): 64 x 8193 tokens, one 8448-token chunk per sequence,
    # 512 workgroups of 8 waves, metadata in the kernel arguments
    "cfg3": dict(chunk_tokens=8448, work_items=64, waves=8, any_multi=0, inline_words=321),
    # cfg4: lognormal lengths up to 27370 split into 3328-token chunks
    "cfg4": dict(chunk_tokens=3328, work_items=195, waves=4, any_multi=1, inline_words=775),
    # cfg5: ~585 live sequences: one chunk each (the longest, 4601 tokens,
    # rounded up); the full metadata (2926 words) would need a device copy,
    # the compact encoding fits: 585 + 293 words
    "cfg5": dict(chunk_tokens=4608, work_items=585, waves=4, any_multi=0, inline_words=878,
                 inline_compact=1),
}


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_benchmark_config_plans(tl, name):
    lens, hkv = cases()[name]
    p = tl.attn_plan(lens, hkv, num_cus=CUS, head_fuse="off")
    got = {k: p[k] for k in EXPECTED[name]}
    assert got == EXPECTED[name]
    assert p["max_len"] == int(lens.max())
    check_invariants(p, lens, hkv, CUS)


# Head-fused plans, which the entry points allow for head_dim 128 on the VALU
# score path (every benchmark configuration's shape).  cfg3: 64 sequences of
# 8 kv heads; 2 heads per workgroup gives 256 (sequence, head pair) blocks,
# one per CU, so one item per sequence (4 heads: 2 items, 8 heads: 4) -- 64
# items, no merge, metadata 64 + 65 + 2 * 64 + 64 words.  The ragged
# configurations keep their chunk plans; cfg4 and cfg5, whose per-head
# workgroups would have 4 waves, run them with 2 heads per 8-wave workgroup,
# cfg4's split sequences in chunks 3/2 as long (3328 * 3/2 = 4992, rounded
# up to 5120 tokens: 163 items).  cfg2's whole sequences in per-head 8-wave
# workgroups end at 11 tile rounds; head pairs in chunks of 2560 end at 10
# (plan_balanced_split): 16 sequences, 5 of them over 2560 tokens, 21 items.
EXPECTED_FUSED = {
    "cfg3": dict(chunk_tokens=8448, work_items=64, waves=8, any_multi=0, inline_words=321,
                 head_fused=2, fused_chunked=0),
    "cfg1": dict(EXPECTED["cfg1"], head_fused=0, fused_chunked=0),
    "cfg2": dict(EXPECTED["cfg2"], chunk_tokens=2560, work_items=21, any_multi=1, inline_words=91,
                 head_fused=2, fused_chunked=1),
    "cfg4": dict(EXPECTED["cfg4"], chunk_tokens=5120, work_items=163, inline_words=711, waves=8,
                 head_fused=2, fused_chunked=1),
    "cfg5": dict(EXPECTED["cfg5"], waves=8, head_fused=2, fused_chunked=1),
}


def fused_chunk_plan(per_head, lens):
    """(chunk, items, any_multi) of the automatic 2-heads-per-workgroup
    chunk plan: where the per-head plan splits a sequence, chunks 3/2 as long,
    rounded up to 256 tokens and capped at the longest length."""
    lens = np.asarray(lens, dtype=np.int64)
    chunk = per_head["chunk_tokens"]
    if per_head["any_multi"]:
        cap = -(-int(lens.max()) // 256) * 256
        chunk = min(-(-(chunk * 3 // 2) // 256) * 256, cap)
    per_entry = -(-lens // chunk)
    return chunk, int(per_entry.sum()), int((per_entry > 1).any())


def lpt_rounds_py(items_desc, per_item, waves_per_head, cus):
    """Longest-first list scheduling (a heap of CU loads) of per_item
    workgroups per item, in whole tile rounds (ceil(ceil(len / 64) /
    waves_per_head) per workgroup): (makespan R, CUs busy in round R)."""
    h = [0] * cus
    for L in items_desc:
        w = -(-(-(-int(L) // 64)) // waves_per_head)
        for _ in range(per_item):
            heapq.heapreplace(h, h[0] + w)
    return max(h), h.count(max(h))


def balanced_split_py(lens, hkv, cus):
    """plan_balanced_split restated: the chunk c (a multiple of 256 from a
    CU's share of the head pairs' tokens up to the longest length, at most 32
    of them, evenly strided) whose
    head-pair plan (hkv / 2 workgroups per item, 4 waves per head) ends before
    whole sequences in per-head 8-wave workgroups -- fewer tile rounds, or as
    many with fewer CUs in the last -- the longest c among the soonest; else 0."""
    lens = [int(x) for x in lens]
    if hkv % 2 or max(lens) <= 1024:
        return 0
    best, best_r = 0, lpt_rounds_py(sorted(lens, reverse=True), hkv, 8, cus)
    share = -(-(sum(lens) * (hkv // 2)) // cus)
    lo = max(256, -(-share // 256) * 256)
    stride = max(256, -(-((max(lens) - lo) // 32) // 256) * 256)  # at most 32 candidates
    for c in range(lo, max(lens), stride):
        items = sorted((min(c, L - t) for L in lens for t in range(0, L, c)), reverse=True)
        r = lpt_rounds_py(items, hkv // 2, 4, cus)
        if r < best_r or (r == best_r and best):
            best, best_r = c, r
    return best


def test_balanced_split_rounds_examples(tl):
    """cfg2's lengths (16 MHA sequences), (tile rounds, CUs in the last):
    whole sequences (11, 32); head pairs in chunks of 2304 (11, 32), 2560
    (10, 112), 2816 (11, 80) -- the kernel measured 92.6, 88.0 and 91.6 us
    per layer against 94.2, and only the 2560 split beat whole sequences end
    to end -- so 2560 is the split.  18 steps later (lengths + 18) whole
    sequences are (11, 64) and 2560 (11, 16): still the split (measured over
    40 steps: 2913 us per step with it throughout, 2992 without).  Uniform
    lengths and short ones never split."""
    lens, hkv = cases()["cfg2"]
    ls = [int(x) for x in lens]
    assert lpt_rounds_py(sorted(ls, reverse=True), 32, 8, CUS) == (11, 32)
    for c, r in ((2304, (11, 32)), (2560, (10, 112)), (2816, (11, 80)), (3072, (12, 80))):
        items = sorted((min(c, L - t) for L in ls for t in range(0, L, c)), reverse=True)
        assert lpt_rounds_py(items, 16, 4, CUS) == r, c
    assert balanced_split_py(ls, 32, CUS) == 2560
    later = [L + 18 for L in ls]
    assert lpt_rounds_py(sorted(later, reverse=True), 32, 8, CUS) == (11, 64)
    assert balanced_split_py(later, 32, CUS) == 2560
    for grow in (0, 18, 39):
        p = tl.attn_plan(lens + grow, hkv, num_cus=CUS, head_fuse="auto")
        assert (p["chunk_tokens"], p["head_fused"], p["fused_chunked"]) == (2560, 2, 1), grow
    # the per-head-only plan (head_fuse off) and a forced chunk keep their chunks
    assert tl.attn_plan(lens, hkv, num_cus=CUS, head_fuse="off")["chunk_tokens"] == 4096
    assert tl.attn_plan(lens, hkv, num_cus=CUS, head_fuse="auto", forced_chunk=3072)["chunk_tokens"] == 3072
    assert balanced_split_py([1000] * 16, 32, CUS) == 0


@pytest.mark.parametrize("name", sorted(EXPECTED_FUSED))
def test_benchmark_config_plans_head_fused(tl, name):
    lens, hkv = cases()[name]
    p = tl.attn_plan(lens, hkv, num_cus=CUS, head_fuse="auto")
    got = {k: p[k] for k in EXPECTED_FUSED[name]}
    assert got == EXPECTED_FUSED[name]
    if p["head_fused"] and not p["fused_chunked"]:
        check_fused(p, lens, hkv, CUS, *fused_choice(lens, hkv, CUS))
    else:
        check_invariants(p, lens, hkv, CUS)


def fused_items(lens, hkv, cus, h):
    """Items per sequence with h kv heads per workgroup, 0 if h does not apply."""
    if hkv % h:
        return 0
    groups = lens.size * hkv // h
    if groups > cus:
        return 0
    nch = min(cus // groups, 8, max(1, int(lens.min()) // (512 * (8 // h))))
    return nch if groups * nch * 10 >= cus * 9 else 0


def fused_choice(lens, hkv, cus, force=1):
    """(heads per workgroup, items per sequence) of the head-fused plan, or
    None: lengths within 10% of the longest; forced h, or the h in (8, 4, 2)
    with the fewest items, the larger h on a tie."""
    lens = np.asarray(lens, dtype=np.int64)
    mx, mn = int(lens.max()), int(lens.min())
    if mn < 1 or mn < mx - mx // 10:
        return None
    if force in (2, 4, 8):
        c = fused_items(lens, hkv, cus, force)
        return (force, c) if c else None
    best = None
    for h in (8, 4, 2):
        c = fused_items(lens, hkv, cus, h)
        if c and (best is None or c < best[1]):
            best = (h, c)
    return best


def check_fused(p, lens, hkv, cus, hpw, nch):
    lens = np.asarray(lens, dtype=np.int64)
    n = lens.size
    assert p["head_fused"] == hpw and p["work_items"] == n * nch
    assert n * (hkv // hpw) * nch <= cus
    assert p["chunk_tokens"] == -(-int(lens.max()) // 256) * 256
    assert p["waves"] == 8 and p["any_multi"] == int(nch > 1) and p["any_empty"] == 0
    assert np.array_equal(p["part_base"], np.arange(n + 1) * nch)
    # chunk-major: (0, 0), (1, 0), ..., (n-1, 0), (0, 1), ...
    want = np.array([(i, c) for c in range(nch) for i in range(n)], dtype=np.int32).reshape(-1, 2)
    assert np.array_equal(p["work"], want)
    # slice s of item c takes tiles u, u + nch * S, ... (u = c * S + s, S = 8 / hpw
    # waves per head): every tile exactly once
    S = 8 // hpw
    for L in {int(lens.min()), int(lens.max())}:
        tiles = -(-L // 64)
        covered = sorted(t for u in range(nch * S) for t in range(u, tiles, nch * S))
        assert covered == list(range(tiles))


@pytest.mark.parametrize("seed", range(60))
def test_random_plans_head_fused(tl, seed):
    rng = np.random.default_rng(1000 + seed)
    hkv = int(rng.choice([2, 4, 8, 16, 32]))
    cus = int(rng.choice([80, 256, 304]))
    groups_max = max(1, cus * 4 // hkv)
    n = int(rng.integers(1, min(300, groups_max + 20)))
    top = int(rng.integers(1, 20000))
    spread = top // 10 if seed % 3 else top // 4  # within 10%, or ragged
    lens = (top - rng.integers(0, spread + 1, n)).astype(np.int32)
    force = int(rng.choice([1, 1, 2, 4, 8]))
    hf = "auto" if force == 1 else force  # force: 1 = the planner's choice
    p = tl.attn_plan(lens, hkv, num_cus=cus, head_fuse=hf)
    choice = fused_choice(lens, hkv, cus, force)
    if choice:
        check_fused(p, lens, hkv, cus, *choice)
        assert p["fused_chunked"] == 0
    else:
        # the chunk plan, over 2 (auto, where per-head workgroups would have 4
        # waves) or the forced number of heads per workgroup
        per_head = tl.attn_plan(lens, hkv, num_cus=cus, head_fuse="off")
        split = 0
        if force in (2, 4, 8):
            want = force if hkv % force == 0 else 0
        else:
            want = 2 if hkv % 2 == 0 and per_head["waves"] == 4 else 0
            if hkv % 2 == 0 and per_head["waves"] == 8 and not per_head["any_multi"]:
                split = balanced_split_py(lens, hkv, cus)
                want = 2 if split else want
        assert (p["head_fused"], p["fused_chunked"]) == (want, int(want > 0))
        got = tuple(p[k] for k in ("chunk_tokens", "work_items", "any_multi"))
        if split:
            assert got == (split, int((-(-lens.astype(np.int64) // split)).sum()), 1)
        elif force == 1 and want == 2:
            assert got == fused_chunk_plan(per_head, lens)
        else:
            assert got == tuple(per_head[k] for k in ("chunk_tokens", "work_items", "any_multi"))
        check_invariants(p, lens, hkv, cus)
    # forced 4-wave workgroups keep the per-head plan; a forced chunk the
    # chunk plan, head-fused over its items by the same rule
    assert tl.attn_plan(lens, hkv, num_cus=cus, head_fuse=hf, waves=4)["head_fused"] == 0
    pf = tl.attn_plan(lens, hkv, num_cus=cus, head_fuse=hf, forced_chunk=512)
    per_head = tl.attn_plan(lens, hkv, num_cus=cus, forced_chunk=512, head_fuse="off")
    if force in (2, 4, 8):
        want = force if hkv % force == 0 else 0
    else:
        want = 2 if hkv % 2 == 0 and per_head["waves"] == 4 else 0
    assert (pf["head_fused"], pf["fused_chunked"]) == (want, int(want > 0))
    assert pf["work_items"] == per_head["work_items"]


def test_head_fused_choice_examples(tl):
    """Fewest items per sequence, then more heads per workgroup (256 CUs)."""
    def pick(B, hkv, L):
        p = tl.attn_plan(np.full(B, L, np.int32), hkv, num_cus=CUS, head_fuse="auto")
        return p["head_fused"], p["work_items"] // B
    assert pick(64, 8, 8193) == (2, 1)     # cfg3: 256 head-pair blocks
    assert pick(128, 8, 8193) == (4, 1)    # 256 blocks of 4 heads
    assert pick(256, 8, 8193) == (8, 1)    # 256 blocks of 8 heads
    assert pick(32, 8, 8193) == (2, 2)     # 128 head-pair blocks, 2 items each
    assert pick(80, 8, 8193) == (8, 3)     # only 8 heads fill 90%: 3 x 80 = 240
    assert pick(64, 4, 8193) == (2, 2)     # 4 kv heads: pairs, 2 items
    assert pick(64, 8, 600) == (2, 1)      # short sequences: one item still fills
    p = tl.attn_plan(np.full(100, 8193, np.int32), 8, num_cus=CUS, head_fuse="auto")
    assert (p["head_fused"], p["fused_chunked"]) == (2, 1)  # no h fills 90%: chunk plan, 2 heads


def check_invariants(p, lens, hkv, cus, forced=0):
    lens = np.asarray(lens, dtype=np.int64)
    n = lens.size
    chunk = p["chunk_tokens"]
    assert chunk % 256 == 0 and chunk >= 256
    cap = max(256, -(-int(lens.max(initial=0)) // 256) * 256)
    assert chunk <= cap
    if forced:
        assert chunk == min(forced, cap)
    per_entry = -(-lens // chunk)
    assert np.array_equal(p["part_base"], np.concatenate([[0], np.cumsum(per_entry)]))
    assert p["work_items"] == int(per_entry.sum())
    assert p["any_multi"] == int((per_entry > 1).any())
    assert p["any_empty"] == int((per_entry == 0).any())
    work = p["work"]
    # exactly the (entry, chunk) pairs, each once
    pairs = sorted(map(tuple, work.tolist()))
    assert pairs == [(i, c) for i in range(n) for c in range(int(per_entry[i]))]
    # longest item first; equal lengths keep (entry, chunk) order
    item_len = [min(chunk, int(lens[i]) - c * chunk) for i, c in work.tolist()]
    assert all(a >= b for a, b in zip(item_len, item_len[1:]))
    for k in range(len(item_len) - 1):
        if item_len[k] == item_len[k + 1]:
            assert tuple(work[k]) < tuple(work[k + 1])
    # waves: 8 when every CU gets at most two workgroups in turn (head-fused
    # over the items: 8-wave workgroups of several heads, one per CU)
    fused = p.get("fused_chunked", 0) == 1
    if p["work_items"]:
        assert p["waves"] == (8 if fused or p["work_items"] * hkv <= 2 * cus else 4)
    # list scheduling of the items (x hkv heads, or head blocks) on 2 slots
    # per CU (one per CU for head blocks), longest first, finishes within one
    # item of the ideal makespan
    if p["work_items"]:
        units = hkv // p["head_fused"] if fused else hkv
        slots = [0] * (cus if fused else 2 * cus)
        for L in item_len:
            for _ in range(units):
                heapq.heapreplace(slots, slots[0] + L)
        ideal = sum(item_len) * units / len(slots)
        assert max(slots) <= ideal + max(item_len)


@pytest.mark.parametrize("seed", range(40))
def test_random_plans_keep_invariants(tl, seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 300))
    kind = seed % 4
    if kind == 0:
        lens = np.full(n, int(rng.integers(1, 20000)))
    elif kind == 1:
        lens = rng.integers(0, 40000, n)
    elif kind == 2:
        lens = np.clip(np.round(np.exp(rng.normal(np.log(2048), 1.0, n))), 1, 32768)
    else:
        lens = rng.integers(1, 600, n)
    hkv = int(rng.choice([1, 2, 8, 32]))
    cus = int(rng.choice([8, 80, 256]))
    p = tl.attn_plan(lens.astype(np.int32), hkv, num_cus=cus, head_fuse="off")
    check_invariants(p, lens, hkv, cus)


@pytest.mark.parametrize("forced", [256, 512, 4096, 1 << 20])
def test_forced_chunk_is_capped_at_the_longest_length(tl, forced):
    lens = np.array([2101, 4096, 4601, 17], dtype=np.int32)
    p = tl.attn_plan(lens, 2, num_cus=CUS, forced_chunk=forced, head_fuse="off")
    check_invariants(p, lens, 2, CUS, forced=forced)


def test_whole_sequence_chunk_gives_many_tiles_per_wave(tl):
    """A forced chunk at least as long as every sequence puts each sequence in
    one work item, so a wave of an 8-wave workgroup walks len/64/8 tiles."""
    lens = np.array([2101, 4097, 4601], dtype=np.int32)
    p = tl.attn_plan(lens, 2, num_cus=CUS, forced_chunk=4608, head_fuse="off")
    assert p["chunk_tokens"] == 4608 and p["work_items"] == 3 and p["any_multi"] == 0
    assert min(-(-int(s) // 64) // 8 for s in lens) >= 4


@pytest.mark.parametrize("S,chunk", [(8192, 1024), (2048, 256), (4096, 512), (512, 512)])
def test_uniform_split_is_one_round_of_workgroups(tl, S, chunk):
    """The reference's published attention_decode shape (B = 1, 32 heads,
    compact K/V): uniform lengths that must split take chunks of W / C, so
    the items x heads fill each CU once with an 8-wave workgroup (one round);
    512 tokens stay whole (at most two tiles per wave)."""
    p = tl.attn_plan(np.full(1, S, np.int32), 32, num_cus=CUS, head_fuse="off")
    assert p["chunk_tokens"] == chunk and p["waves"] == 8
    assert p["work_items"] * 32 == (CUS if S > 1024 else 32)
    assert p["any_multi"] == int(S > 1024)
    check_invariants(p, np.full(1, S), 32, CUS)


def test_waves_setting_and_empty_sequences(tl):
    lens = np.array([0, 5, 0], dtype=np.int32)
    p = tl.attn_plan(lens, 8, num_cus=CUS, head_fuse="off")
    assert p["any_empty"] == 1 and p["work_items"] == 1
    assert tl.attn_plan(lens, 8, num_cus=CUS, waves=4, head_fuse="off")["waves"] == 4
    assert tl.attn_plan(np.zeros(0, np.int32), 8, num_cus=CUS, head_fuse="off")["work_items"] == 0


def test_inline_metadata_limit(tl):
    """896 words travel in the kernel arguments: lens n, part_base n+1, the
    work list 2 per item, the slot row n -- or, when every sequence is one
    work item, the compact encoding: one word per sequence (16-bit length and
    slot) and 16 bits per work item."""
    fits = np.full(223, 100, dtype=np.int32)      # 223 + 224 + 446 + 0 = 893
    p = tl.attn_plan(fits, 8, num_cus=CUS, with_rows=False, head_fuse="off")
    assert (p["inline_words"], p["inline_compact"]) == (893, 0)
    p = tl.attn_plan(fits, 8, num_cus=CUS, with_rows=True, head_fuse="off")  # 1116 full words
    assert (p["inline_words"], p["inline_compact"]) == (223 + 112, 1)
    big = np.full(597, 100, dtype=np.int32)       # 597 + 299 = 896: the most that fits
    assert tl.attn_plan(big, 8, num_cus=CUS, head_fuse="off")["inline_words"] == 896
    assert tl.attn_plan(np.full(598, 100, np.int32), 8, num_cus=CUS, head_fuse="off")["inline_words"] == -1
    split = np.array([30000] + [100] * 300, dtype=np.int32)  # a split sequence: full only
    p = tl.attn_plan(split, 8, num_cus=CUS, head_fuse="off")
    assert p["any_multi"] == 1 and (p["inline_words"], p["inline_compact"]) == (-1, 0)
    long_ = np.full(300, 70000, dtype=np.int32)   # lengths beyond 16 bits: full only
    assert tl.attn_plan(long_, 1, num_cus=CUS, forced_chunk=70144, head_fuse="off")["inline_compact"] == 0


def test_plan_rejects_bad_arguments(tl):
    with pytest.raises(tl.TinyLLMError):
        tl.attn_plan(np.array([-1], np.int32), 8, head_fuse="off")
    with pytest.raises(tl.TinyLLMError):
        tl.attn_plan(np.array([1], np.int32), 0, head_fuse="off")
    with pytest.raises(tl.TinyLLMError):
        tl.attn_plan(np.array([1], np.int32), 8, waves=3, head_fuse="off")
    with pytest.raises(tl.TinyLLMError):
        tl.attn_plan(np.array([1], np.int32), 8, head_dim=96)
    with pytest.raises(ValueError):
        tl.attn_plan(np.array([1], np.int32), 8, head_fuse=True)


def test_current_mode_follows_the_process_settings(tl, monkeypatch):
    """head_fuse="current" is the entry points' plan: the head-fuse setter's
    mode, the waves setting and TL_ATTN_CHUNK, at the given head_dim; the
    explicit codes are the setter's (0 auto, 1 off, 2 / 4 / 8 forced)."""
    lens = np.full(64, 8193, np.int32)  # config 3: head-fused, 2 kv heads per workgroup
    keys = ("chunk_tokens", "work_items", "waves", "head_fused", "fused_chunked")

    def plan(**kw):
        p = tl.attn_plan(lens, 8, num_cus=CUS, **kw)
        return tuple(p[k] for k in keys)
    hf0, w0 = tl.get_head_fuse(), tl.get_waves()
    monkeypatch.delenv("TL_ATTN_CHUNK", raising=False)
    try:
        tl.set_head_fuse(0)
        tl.set_waves(0)
        assert plan(head_fuse="current") == plan(head_fuse="auto")
        assert plan(head_fuse="current")[3] == 2
        assert plan(head_fuse="current", head_dim=64) == plan(head_fuse="off", head_dim=64)
        assert plan(head_fuse="auto", head_dim=64)[3] == 0  # no head-fused form at 64
        tl.set_head_fuse(1)
        assert plan(head_fuse="current") == plan(head_fuse="off")
        assert plan(head_fuse="current")[3] == 0
        tl.set_head_fuse(4)
        assert plan(head_fuse="current") == plan(head_fuse=4)
        tl.set_head_fuse(0)
        tl.set_waves(4)
        assert plan(head_fuse="current") == plan(head_fuse="off", waves=4)
        tl.set_waves(0)
        monkeypatch.setenv("TL_ATTN_CHUNK", "1024")
        assert plan(head_fuse="current") == plan(head_fuse="auto", forced_chunk=1024)
        assert plan(head_fuse="current")[0] == 1024
    finally:
        tl.set_head_fuse(hf0)
        tl.set_waves(w0)


# Prefill workgroup size (prefill_waves, attention_prefill.hip): the shapes
# timed on one box at Llama-3-8B heads (32 q / 8 kv, head_dim 128), 8- against
# 4-wave workgroups, us per launch: (prompts, new tokens, cached prefix) ->
# the faster form.  4 waves won 2-8.5% where it is expected, 8 waves 3-10%
# elsewhere.
PREFILL_MEASURED = {
    (64, 128, 0): 4,     # 51.4 / 49.8
    (32, 256, 0): 4,     # 66.1 / 60.9
    (16, 512, 0): 4,     # 81.1 / 74.2
    (16, 768, 0): 4,     # 127.4 / 121.7
    (8, 1024, 0): 4,     # 96.6 / 94.5
    (16, 1024, 0): 4,    # 207.5 / 202.6
    (4, 1536, 0): 4,     # 99.5 / 96.0
    (8, 512, 0): 8,      # 38.4 / 41.6: two items per CU
    (4, 2048, 0): 8,     # 152 / 157
    (2, 4096, 0): 8,     # 278.6 / 287.2
    (1, 8192, 0): 8,     # 518 / 551
    (16, 512, 1024): 8,  # 192.8 / 205.8: long items (cached prefix)
    (8, 512, 4096): 8,   # 276.4 / 304.8
}


@pytest.mark.parametrize("shape", sorted(PREFILL_MEASURED))
def test_prefill_waves_follow_the_measured_shapes(tl, shape):
    b, n, p0 = shape
    old = tl.get_prefill_waves()
    tl.set_prefill_waves(0)
    try:
        assert tl.prefill_plan_waves([p0] * b, [n] * b, 32, 8, 128, CUS) == PREFILL_MEASURED[shape]
    finally:
        tl.set_prefill_waves(old)


def test_prefill_waves_rule_boundaries_and_settings(tl):
    old = tl.get_prefill_waves()
    try:
        tl.set_prefill_waves(0)
        # items = 4 x 8 kv heads x 24 query tiles = 768 = 3 per CU, mean keys
        # exactly 800: both limits inclusive
        assert tl.prefill_plan_waves([0] * 4, [1536] * 4, 32, 8, 128, CUS) == 4
        # one item per CU fewer than 3 per CU: 8 waves
        assert tl.prefill_plan_waves([0] * 4, [1536] * 4, 32, 8, 128, CUS + 1) == 8
        # a cached prefix long enough to lift the mean past 800 keys
        assert tl.prefill_plan_waves([64] * 4, [1536] * 4, 32, 8, 128, CUS) == 8
        # head_dim 64: always 4 (three workgroups per CU); 32: 8; 256 has the
        # 4-wave form only
        for n, p0 in ((512, 0), (8192, 0), (512, 1024)):
            assert tl.prefill_plan_waves([p0] * 16, [n] * 16, 32, 8, 64, CUS) == 4
            assert tl.prefill_plan_waves([p0] * 16, [n] * 16, 32, 8, 32, CUS) == 8
        assert tl.prefill_plan_waves([0] * 16, [512] * 16, 32, 8, 256, CUS) == 4
        for forced in (4, 8):
            tl.set_prefill_waves(forced)
            assert tl.get_prefill_waves() == forced
            for d in (32, 64, 128):
                assert tl.prefill_plan_waves([0], [8192], 32, 8, d, CUS) == forced
            assert tl.prefill_plan_waves([0], [8192], 32, 8, 256, CUS) == 4
        with pytest.raises(tl.TinyLLMError, match="waves must be"):
            tl.set_prefill_waves(2)
        with pytest.raises(tl.TinyLLMError, match="invalid lengths"):
            tl.prefill_plan_waves([0], [0], 32, 8, 128, CUS)
        with pytest.raises(tl.TinyLLMError, match="unsupported"):
            tl.prefill_plan_waves([0], [16], 32, 8, 96, CUS)
    finally:
        tl.set_prefill_waves(old)
