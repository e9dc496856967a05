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
    # cfg1: 4 MHA sequences of 129..513 tokens; 513 > 256 spans 3 chunks
    "cfg1": dict(chunk_tokens=256, work_items=8, waves=8, any_multi=1, inline_words=29),
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
    p = tl.attn_plan(lens, hkv, num_cus=CUS)
    got = {k: p[k] for k in EXPECTED[name]}
    assert got == EXPECTED[name]
    assert p["max_len"] == int(lens.max())
    check_invariants(p, lens, hkv, CUS)


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
    # waves: 8 when every CU gets at most two workgroups in turn
    if p["work_items"]:
        assert p["waves"] == (8 if p["work_items"] * hkv <= 2 * cus else 4)
    # list scheduling of the items (x hkv heads) on 2 slots per CU, longest
    # first, finishes within one item of the ideal makespan
    if p["work_items"]:
        slots = [0] * (2 * cus)
        for L in item_len:
            for _ in range(hkv):
                heapq.heapreplace(slots, slots[0] + L)
        ideal = sum(item_len) * hkv / (2 * cus)
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
    p = tl.attn_plan(lens.astype(np.int32), hkv, num_cus=cus)
    check_invariants(p, lens, hkv, cus)


@pytest.mark.parametrize("forced", [256, 512, 4096, 1 << 20])
def test_forced_chunk_is_capped_at_the_longest_length(tl, forced):
    lens = np.array([2101, 4096, 4601, 17], dtype=np.int32)
    p = tl.attn_plan(lens, 2, num_cus=CUS, forced_chunk=forced)
    check_invariants(p, lens, 2, CUS, forced=forced)


def test_whole_sequence_chunk_gives_many_tiles_per_wave(tl):
    """A forced chunk at least as long as every sequence puts each sequence in
    one work item, so a wave of an 8-wave workgroup walks len/64/8 tiles."""
    lens = np.array([2101, 4097, 4601], dtype=np.int32)
    p = tl.attn_plan(lens, 2, num_cus=CUS, forced_chunk=4608)
    assert p["chunk_tokens"] == 4608 and p["work_items"] == 3 and p["any_multi"] == 0
    assert min(-(-int(s) // 64) // 8 for s in lens) >= 4


def test_waves_setting_and_empty_sequences(tl):
    lens = np.array([0, 5, 0], dtype=np.int32)
    p = tl.attn_plan(lens, 8, num_cus=CUS)
    assert p["any_empty"] == 1 and p["work_items"] == 1
    assert tl.attn_plan(lens, 8, num_cus=CUS, waves=4)["waves"] == 4
    assert tl.attn_plan(np.zeros(0, np.int32), 8, num_cus=CUS)["work_items"] == 0


def test_inline_metadata_limit(tl):
    """896 words travel in the kernel arguments: lens n, part_base n+1, the
    work list 2 per item, the slot row n -- or, when every sequence is one
    work item, the compact encoding: one word per sequence (16-bit length and
    slot) and 16 bits per work item."""
    fits = np.full(223, 100, dtype=np.int32)      # 223 + 224 + 446 + 0 = 893
    p = tl.attn_plan(fits, 8, num_cus=CUS, with_rows=False)
    assert (p["inline_words"], p["inline_compact"]) == (893, 0)
    p = tl.attn_plan(fits, 8, num_cus=CUS, with_rows=True)  # 1116 full words
    assert (p["inline_words"], p["inline_compact"]) == (223 + 112, 1)
    big = np.full(597, 100, dtype=np.int32)       # 597 + 299 = 896: the most that fits
    assert tl.attn_plan(big, 8, num_cus=CUS)["inline_words"] == 896
    assert tl.attn_plan(np.full(598, 100, np.int32), 8, num_cus=CUS)["inline_words"] == -1
    split = np.array([30000] + [100] * 300, dtype=np.int32)  # a split sequence: full only
    p = tl.attn_plan(split, 8, num_cus=CUS)
    assert p["any_multi"] == 1 and (p["inline_words"], p["inline_compact"]) == (-1, 0)
    long_ = np.full(300, 70000, dtype=np.int32)   # lengths beyond 16 bits: full only
    assert tl.attn_plan(long_, 1, num_cus=CUS, forced_chunk=70144)["inline_compact"] == 0


def test_plan_rejects_bad_arguments(tl):
    with pytest.raises(tl.TinyLLMError):
        tl.attn_plan(np.array([-1], np.int32), 8)
    with pytest.raises(tl.TinyLLMError):
        tl.attn_plan(np.array([1], np.int32), 0)
    with pytest.raises(tl.TinyLLMError):
        tl.attn_plan(np.array([1], np.int32), 8, waves=3)
