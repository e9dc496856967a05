"""GPU: head-fused decode plans.  One 8-wave workgroup takes H kv heads of a
work item (wave w: head w % H, tile slice w / H), so it reads H heads'
pieces of each token row at once, and a sequence's work items interleave its
64-token tiles; split sequences are combined by the merge launch.

Ragged lengths keep the chunk plan's items (longest first), with 2 heads per
workgroup where per-head workgroups would have 4 waves, split sequences in
chunks 3/2 as long; where per-head workgroups would have 8 waves, at most two
per CU, with whole sequences, the planner's balanced split (2 heads per
workgroup, the longest sequences in chunks).

Checked for H = 2, 4 and 8 and the planner's own choice, every group size,
contiguous and paged caches, one to eight interleaved items per sequence and
chunk items of ragged lengths:
  - one decode step (append + attention) against the oracle: attention
    <= 1e-3 normwise (test_transformer.cu:80-92), cache bytes bit-exact;
  - the same step on the per-head kernel (head fusing off) within the same
    1e-3 of the oracle, and the head-fused step run twice giving the same
    bits;
  - tl_attn_decode_gqa (the library's shared workspace) over two head-fused
    plans in a row."""
import zlib

import numpy as np
import pytest

from devutil import empty_dev, read_dev, rel_err, stream, to_dev, to_host

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture
def head_fuse(tl):
    before = tl.get_head_fuse()
    yield tl.set_head_fuse
    tl.set_head_fuse(before)


def cus():
    import torch
    return torch.cuda.get_device_properties(0).multi_processor_count


def f16bits(rng, n):
    return rng.standard_normal(n, dtype=np.float32).astype(np.float16).view(np.uint16)


# (heads per workgroup setting: 0 = the planner's choice, kv heads, batch,
#  context range, group, paged) -> (heads per workgroup, items per sequence)
# on 256 CUs
RUNS = [
    ((2, 8, 64, (2048, 2250), 4, False), (2, 1)),
    ((2, 8, 64, (2048, 2250), 8, True), (2, 1)),
    ((2, 8, 32, (4096, 4300), 2, False), (2, 2)),
    ((4, 8, 128, (1024, 1100), 4, True), (4, 1)),
    ((4, 8, 64, (2048, 2250), 1, False), (4, 2)),
    ((8, 8, 256, (200, 220), 4, False), (8, 1)),
    ((8, 8, 64, (2048, 2250), 2, True), (8, 4)),
    ((8, 16, 16, (4096, 4400), 4, False), (8, 8)),
    ((0, 8, 80, (1600, 1700), 4, True), (8, 3)),
    ((0, 8, 64, (2048, 2250), 8, False), (2, 1)),
]


@pytest.mark.parametrize("run,expect", RUNS, ids=[
    "h{}-hkv{}-b{}-g{}-{}".format(r[0], r[1], r[2], r[4], "paged" if r[5] else "slots")
    for r, _ in RUNS])
def test_head_fused_decode_step(tl, orc, head_fuse, run, expect):
    setting, Hkv, B, (lo, hi), G, paged = run
    rng = np.random.default_rng(zlib.crc32(repr(run).encode()))
    ctx = rng.integers(lo, hi + 1, B)
    lens = (ctx + 1).astype(np.int32)
    plan = tl.attn_plan(lens, Hkv, num_cus=cus(), with_rows=True, head_fuse=setting or "auto")
    nch = plan["work_items"] // B
    if cus() == 256:
        assert (plan["head_fused"], nch) == expect
    assert plan["head_fused"] in (2, 4, 8) and plan["fused_chunked"] == 0
    assert nch * B == plan["work_items"]
    decode_step_checks(tl, orc, head_fuse, rng, setting, Hkv, G, paged, ctx, plan)


# Ragged lengths keep the chunk plan; where per-head workgroups would have 4
# waves the planner runs its items with 2 heads per 8-wave workgroup (setting
# 0), or with a forced number.  (setting, kv heads, batch, group, paged)
CHUNKED = [(0, 8, 128, 4, True), (0, 8, 160, 8, False), (0, 16, 64, 2, False),
           (4, 8, 96, 2, False), (8, 8, 64, 4, True), (2, 16, 48, 1, True)]


@pytest.mark.parametrize("run", CHUNKED, ids=[
    "h{}-hkv{}-b{}-g{}-{}".format(r[0], r[1], r[2], r[3], "paged" if r[4] else "slots")
    for r in CHUNKED])
def test_head_fused_chunk_items_decode_step(tl, orc, head_fuse, run):
    setting, Hkv, B, G, paged = run
    rng = np.random.default_rng(zlib.crc32(repr(run).encode()))
    # ragged: mostly short, a few long enough to split into several chunks
    ctx = np.where(rng.random(B) < 0.1, rng.integers(3000, 4000, B), rng.integers(20, 1500, B))
    lens = (ctx + 1).astype(np.int32)
    plan = tl.attn_plan(lens, Hkv, num_cus=cus(), with_rows=True, head_fuse=setting or "auto")
    assert plan["fused_chunked"] == 1 and plan["head_fused"] == (setting or 2)
    assert plan["waves"] == 8
    per_head = tl.attn_plan(lens, Hkv, num_cus=cus(), with_rows=True, head_fuse="off")
    assert per_head["waves"] == 4
    if setting:  # forced heads per workgroup: the per-head plan's items
        assert plan["work_items"] == per_head["work_items"]
    else:  # the planner's 2 heads: split sequences in chunks 3/2 as long
        assert plan["chunk_tokens"] >= per_head["chunk_tokens"]
        assert plan["work_items"] <= per_head["work_items"]
    decode_step_checks(tl, orc, head_fuse, rng, setting, Hkv, G, paged, ctx, plan)


# Ragged lengths whose whole sequences would run in per-head 8-wave
# workgroups at most two per CU: the planner's balanced split (head pairs in
# chunks, split sequences merged).  (kv heads, batch, context range, group,
# paged)
BALANCED = [(16, 32, (300, 2000), 1, False), (16, 32, (300, 2000), 2, True),
            (32, 16, (512, 4096), 1, True), (8, 60, (300, 2000), 8, True)]


@pytest.mark.parametrize("run", BALANCED, ids=[
    "hkv{}-b{}-g{}-{}".format(r[0], r[1], r[3], "paged" if r[4] else "slots") for r in BALANCED])
def test_balanced_split_decode_step(tl, orc, head_fuse, run):
    Hkv, B, (lo, hi), G, paged = run
    rng = np.random.default_rng(zlib.crc32(repr(run).encode()))
    ctx = rng.integers(lo, hi + 1, B)
    lens = (ctx + 1).astype(np.int32)
    per_head = tl.attn_plan(lens, Hkv, num_cus=cus(), with_rows=True, head_fuse="off")
    plan = tl.attn_plan(lens, Hkv, num_cus=cus(), with_rows=True, head_fuse="auto")
    if cus() == 256:
        assert (per_head["waves"], per_head["any_multi"]) == (8, 0)
        assert (plan["head_fused"], plan["fused_chunked"], plan["any_multi"]) == (2, 1, 1)
        assert plan["chunk_tokens"] < per_head["chunk_tokens"]
    decode_step_checks(tl, orc, head_fuse, rng, 0, Hkv, G, paged, ctx, plan)


def decode_step_checks(tl, orc, head_fuse, rng, setting, Hkv, G, paged, ctx, plan):
    """One decode step on a cache holding contexts ctx: head-fused (setting)
    twice, bit-identical; per-head; both against the oracle."""
    B = len(ctx)
    M = -(-(int(ctx.max()) + 1) // 64) * 64
    slots = B + 1
    lens = (ctx + 1).astype(np.int32)
    g = tl.KVCacheManager(1, Hkv, D, M, slots)
    o = orc.KVCacheOracle(1, Hkv, D, M, slots)
    if paged:
        perm = rng.permutation(slots * (M // 16)).astype(np.int32)
        assert g.setBlockMap(16, perm) is None
    ids = []
    for S in ctx:
        sid, err = g.allocateSequence(M)
        assert err is None, err
        o.allocate(M)
        k, v = f16bits(rng, int(S) * Hkv * D), f16bits(rng, int(S) * Hkv * D)
        dk, dv = to_dev(k), to_dev(v)
        assert g.appendKV(sid, 0, dk.data_ptr(), dv.data_ptr(), int(S), stream()) is None
        del dk, dv
        o.append(sid, 0, k, v, int(S))
        g.advanceSeqLen(sid, int(S))
        o.advance(sid, int(S))
        ids.append(sid)
    Hq = Hkv * G
    q = f16bits(rng, B * Hq * D).reshape(B, Hq, D)
    nk, nv = f16bits(rng, B * Hkv * D).reshape(B, -1), f16bits(rng, B * Hkv * D).reshape(B, -1)
    dq, dnk, dnv = to_dev(q), to_dev(nk), to_dev(nv)
    scale = 1.0 / np.sqrt(D)
    batch = tl.DecodeBatch(g, B, Hq)

    def step(mode):
        head_fuse(mode)
        batch.prepare(ids, stream())
        if mode != 1:
            assert batch.info()["work_items"] == plan["work_items"]
        out = empty_dev((B, Hq, D))
        out.fill_(float("nan"))
        batch.decode(0, dq.data_ptr(), dnk.data_ptr(), dnv.data_ptr(), out.data_ptr(), scale,
                     stream())
        return to_host(out)

    fused = step(setting)
    again = step(setting)  # the same step again: the append rewrites the same bytes
    per_head = step(1)
    assert np.array_equal(fused, again), "head-fused step not deterministic"

    for i, sid in enumerate(ids):
        o.append(sid, 0, nk[i], nv[i], 1)
    if not paged:
        assert np.array_equal(read_dev(g.pool(), o.pool().size), o.pool())
    view = orc.cache_view(o.pool(), 1, Hkv, D, M, 0, [o.slot_of(s) for s in ids])
    ref32, _ = orc.attn_decode_gqa(q, view, lens, Hq, Hkv, D, scale, nthreads=8)
    for name, got in (("head-fused", fused), ("per-head", per_head)):
        g32 = got.view(np.float16).astype(np.float32)
        errs = [rel_err(g32[b], ref32[b]) for b in range(B)]
        assert max(errs) <= 1e-3, (name, max(errs))
    if paged:  # the appended token landed where the block map says
        smax = int(lens.max())
        gk = empty_dev((B, Hkv, smax, D))
        batch.gather(0, gk.data_ptr(), 0, smax, stream())
        assert np.array_equal(to_host(gk), orc.gather(view, 0, lens, Hkv, D, smax))


def test_head_fused_stateless_two_plans_in_a_row(tl, orc, head_fuse):
    """tl_attn_decode_gqa over a paged view with one slot per block: two
    interleaved items per sequence (partials and the merge launch), then one,
    then ragged lengths with an empty sequence (chunk items, 2 heads per
    workgroup; the empty sequence's zero row from the merge launch)."""
    import torch
    head_fuse(0)
    Hkv, G = 8, 4
    Hq = Hkv * G
    for B, (lo, hi), seed, nch in ((32, (4200, 4400), 1, 2), (64, (2100, 2300), 2, 1),
                                   (128, (0, 2000), 3, 0)):
        rng = np.random.default_rng(seed)
        lens = rng.integers(lo, hi + 1, B).astype(np.int32)
        p = tl.attn_plan(lens, Hkv, num_cus=cus(), with_rows=False, head_fuse="auto")
        assert p["head_fused"] in (2, 4, 8)
        if nch:  # items interleaving tiles
            assert p["fused_chunked"] == 0
            assert p["work_items"] == B * nch or cus() != 256
        else:  # ragged, an empty sequence included: chunk items, 2 heads per workgroup
            lens[7] = 0
            p = tl.attn_plan(lens, Hkv, num_cus=cus(), with_rows=False, head_fuse="auto")
            assert p["fused_chunked"] == 1 and p["any_empty"] == 1
        M = max(1, int(lens.max()))
        pool = f16bits(rng, 2 * B * M * Hkv * D)
        dpool = to_dev(pool)
        base = dpool.data_ptr()
        v_off = B * M * Hkv * D
        bt = torch.arange(B, dtype=torch.int32, device="cuda").reshape(B, 1)
        view = tl.KVView(base, base + 2 * v_off, bt.data_ptr(), 1, 30, M * Hkv * D, Hkv * D, D)
        q = f16bits(rng, B * Hq * D).reshape(B, Hq, D)
        dq = to_dev(q)
        out = empty_dev((B, Hq, D))
        out.fill_(float("nan"))
        scale = 1.0 / np.sqrt(D)
        tl.attn_decode_gqa(dq.data_ptr(), view, lens, Hq, Hkv, D, scale, out.data_ptr(), stream())
        got = to_host(out).view(np.float16).astype(np.float32)
        oview = orc.View(pool, 0, v_off, np.arange(B, dtype=np.int32).reshape(B, 1), 30,
                         M * Hkv * D, Hkv * D, D)
        ref32, _ = orc.attn_decode_gqa(q, oview, lens, Hq, Hkv, D, scale, nthreads=8)
        errs = [rel_err(got[b], ref32[b]) for b in range(B)]
        assert max(errs) <= 1e-3, (B, max(errs))
