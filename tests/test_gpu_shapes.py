"""GPU: every instantiated (head_dim, group) shape, both score paths (VALU and
MFMA), both workgroup sizes (4 and 8 waves), contiguous and paged cache
layouts, ragged lengths that span one and several split-K chunks -- one
decode step (append + attention) each, against the oracle (attention <= 1e-3
normwise, cache bytes bit-exact)."""
import numpy as np
import pytest

from devutil import empty_dev, read_dev, rel_err, stream, to_dev, to_host

pytestmark = pytest.mark.gpu

LENS = [1, 17, 67, 300, 700, 1100]


@pytest.fixture
def score_path(tl):
    before = tl.get_score_path()
    yield tl.set_score_path
    tl.set_score_path(before)


@pytest.fixture
def waves(tl):
    before = tl.get_waves()
    yield tl.set_waves
    tl.set_waves(before)


def f16bits(rng, shape):
    return rng.standard_normal(shape).astype(np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("nw", [4, 8])
@pytest.mark.parametrize("chunk", ["auto", "256"])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("path", [0, 1, 3])
def test_decode_step_all_shapes(tl, orc, score_path, waves, monkeypatch, path, D, G, paged, chunk,
                                nw):
    """chunk=256 forces the smallest work items (one 64-token tile per wave,
    most entries split into several chunks and merged); "auto" lets the
    planner choose for this small batch."""
    score_path(path)
    waves(nw)
    if chunk != "auto":
        monkeypatch.setenv("TL_ATTN_CHUNK", chunk)
    rng = np.random.default_rng(path * 1000 + D * 10 + G + (500 if paged else 0))
    Hkv, M = 2, 1152
    slots = len(LENS) + 1
    g = tl.KVCacheManager(1, Hkv, D, M, slots)
    o = orc.KVCacheOracle(1, Hkv, D, M, slots)
    if paged:
        perm = rng.permutation(slots * (M // 16)).astype(np.int32)
        assert g.setBlockMap(16, perm) is None
    ids, keep = [], []
    for S in LENS:
        sid, _ = g.allocateSequence(M)
        o.allocate(M)
        k, v = f16bits(rng, S * Hkv * D), f16bits(rng, S * Hkv * D)
        dk, dv = to_dev(k), to_dev(v)
        keep += [dk, dv]
        assert g.appendKV(sid, 0, dk.data_ptr(), dv.data_ptr(), S, stream()) is None
        o.append(sid, 0, k, v, S)
        g.advanceSeqLen(sid, S)
        o.advance(sid, S)
        ids.append(sid)
    Hq = Hkv * G
    B = len(ids)
    batch = tl.DecodeBatch(g, B, Hq)
    batch.prepare(ids, stream())
    q = f16bits(rng, (B, Hq, D))
    nk, nv = f16bits(rng, (B, Hkv * D)), f16bits(rng, (B, Hkv * D))
    dq, dnk, dnv = to_dev(q), to_dev(nk), to_dev(nv)
    out = empty_dev((B, Hq, D))
    scale = 1.0 / np.sqrt(D)
    batch.decode(0, dq.data_ptr(), dnk.data_ptr(), dnv.data_ptr(), out.data_ptr(), scale, stream())
    for i, sid in enumerate(ids):
        o.append(sid, 0, nk[i], nv[i], 1)
    if not paged:
        assert np.array_equal(read_dev(g.pool(), o.pool().size), o.pool())
    lens = np.array([S + 1 for S in LENS])
    view = orc.cache_view(o.pool(), 1, Hkv, D, M, 0, [o.slot_of(s) for s in ids])
    ref32, _ = orc.attn_decode_gqa(q, view, lens, Hq, Hkv, D, scale, nthreads=8)
    got = to_host(out).view(np.float16).astype(np.float32)
    errs = [rel_err(got[i], ref32[i]) for i in range(B)]
    assert max(errs) <= 1e-3, errs
    if paged:  # the appended token landed where the block map says
        smax = int(lens.max())
        gk = empty_dev((B, Hkv, smax, D))
        batch.gather(0, gk.data_ptr(), 0, smax, stream())
        assert np.array_equal(to_host(gk), orc.gather(view, 0, lens, Hkv, D, smax))


LONG = [2100, 4096, 4600]  # contexts; attended = context + 1 after the append


@pytest.mark.parametrize("nw", [4, 8])
@pytest.mark.parametrize("chunk", ["4608", "1024"])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("path", [0, 1, 3])
def test_decode_long_chunks_all_shapes(tl, orc, score_path, waves, monkeypatch, path, D, G, paged,
                                       chunk, nw):
    """Work items of many 64-token tiles per wave -- the plans the benchmark
    configurations run (cfg3: 8448-token chunks, 17 tiles per wave).
    chunk=4608 puts each sequence in one work item (8-wave workgroups: 4 to 9
    tiles per wave, 4-wave: 8 to 18), chunk=1024 splits them into several
    multi-tile items and merges the partials.  Every sequence holds a key
    aligned with its group's first query head about 100 tokens before its
    end, so the running maximum jumps in a late tile and the rescale of the
    earlier tiles' sums (alpha = 2^(m_old - m_new) != 1) carries about half of
    the output; the paged layout also runs the next-tile block prefetch."""
    score_path(path)
    waves(nw)
    monkeypatch.setenv("TL_ATTN_CHUNK", chunk)
    rng = np.random.default_rng(7000 + path * 1000 + D * 10 + G + (500 if paged else 0))
    Hkv, M = 2, 4608
    Hq = Hkv * G
    slots = len(LONG) + 1
    g = tl.KVCacheManager(1, Hkv, D, M, slots)
    o = orc.KVCacheOracle(1, Hkv, D, M, slots)
    if paged:
        perm = rng.permutation(slots * (M // 16)).astype(np.int32)
        assert g.setBlockMap(16, perm) is None
    q = f16bits(rng, (len(LONG), Hq, D))
    qf = q.view(np.float16).astype(np.float32)
    ids, keep = [], []
    for b, S in enumerate(LONG):
        sid, _ = g.allocateSequence(M)
        o.allocate(M)
        k = f16bits(rng, (S, Hkv, D))
        v = f16bits(rng, (S, Hkv, D))
        t_star = S - 100
        for kh in range(Hkv):  # score about 9 against query head kh*G
            k[t_star, kh] = (qf[b, kh * G] * (9.0 / np.sqrt(D))).astype(np.float16).view(np.uint16)
        k, v = k.reshape(-1), v.reshape(-1)
        dk, dv = to_dev(k), to_dev(v)
        keep += [dk, dv]
        assert g.appendKV(sid, 0, dk.data_ptr(), dv.data_ptr(), S, stream()) is None
        o.append(sid, 0, k, v, S)
        g.advanceSeqLen(sid, S)
        o.advance(sid, S)
        ids.append(sid)
    B = len(ids)
    batch = tl.DecodeBatch(g, B, Hq)
    batch.prepare(ids, stream())
    info = batch.info()
    assert info["chunk_tokens"] == int(chunk)
    lens = np.array([S + 1 for S in LONG])
    assert info["work_items"] == int(sum(-(-lens // int(chunk))))
    nk, nv = f16bits(rng, (B, Hkv * D)), f16bits(rng, (B, Hkv * D))
    dq, dnk, dnv = to_dev(q), to_dev(nk), to_dev(nv)
    out = empty_dev((B, Hq, D))
    scale = 1.0 / np.sqrt(D)
    batch.decode(0, dq.data_ptr(), dnk.data_ptr(), dnv.data_ptr(), out.data_ptr(), scale, stream())
    for i, sid in enumerate(ids):
        o.append(sid, 0, nk[i], nv[i], 1)
    if not paged:
        assert np.array_equal(read_dev(g.pool(), o.pool().size), o.pool())
    view = orc.cache_view(o.pool(), 1, Hkv, D, M, 0, [o.slot_of(s) for s in ids])
    ref32, _ = orc.attn_decode_gqa(q, view, lens, Hq, Hkv, D, scale, nthreads=8)
    got = to_host(out).view(np.float16).astype(np.float32)
    errs = [rel_err(got[i], ref32[i]) for i in range(B)]
    assert max(errs) <= 1e-3, errs
    if paged:
        smax = int(lens.max())
        gk = empty_dev((B, Hkv, smax, D))
        gv = empty_dev((B, Hkv, smax, D))
        batch.gather(0, gk.data_ptr(), gv.data_ptr(), smax, stream())
        assert np.array_equal(to_host(gk), orc.gather(view, 0, lens, Hkv, D, smax))
        assert np.array_equal(to_host(gv), orc.gather(view, 1, lens, Hkv, D, smax))


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("D,G", [(128, 4), (128, 8), (64, 2), (256, 1)])
@pytest.mark.parametrize("path", [0, 3])
def test_decode_compact_metadata(tl, orc, score_path, path, D, G, paged):
    """Batches of 400 sequences that stay one work item each carry their
    metadata in the compact encoding (16-bit length and slot per sequence,
    16-bit launch order): 400 + 200 words instead of 2001.  Slots are taken
    out of order (every other one released first), so slot != entry index."""
    score_path(path)
    rng = np.random.default_rng(9100 + D + G + (50 if paged else 0) + path)
    Hkv, M, n = 2, 320, 400
    Hq = Hkv * G
    slots = 2 * n
    g = tl.KVCacheManager(1, Hkv, D, M, slots)
    o = orc.KVCacheOracle(1, Hkv, D, M, slots)
    if paged:
        assert g.setBlockMap(16, rng.permutation(slots * (M // 16)).astype(np.int32)) is None
    sids = [g.allocateSequence(M)[0] for _ in range(slots)]
    for _ in range(slots):
        o.allocate(M)
    for s in sids[::2]:  # free every other slot; the batch uses the rest
        assert g.releaseSequence(s) is None and o.release(s) is None
    ids = sids[1::2]
    lens = rng.integers(1, M - 8, n)
    keep = []
    for s, S in zip(ids, lens):
        k, v = f16bits(rng, int(S) * Hkv * D), f16bits(rng, int(S) * Hkv * D)
        dk, dv = to_dev(k), to_dev(v)
        keep += [dk, dv]
        assert g.appendKV(s, 0, dk.data_ptr(), dv.data_ptr(), int(S), stream()) is None
        o.append(s, 0, k, v, int(S))
        g.advanceSeqLen(s, int(S))
        o.advance(s, int(S))
    plan = tl.attn_plan((lens + 1).astype(np.int32), Hkv,
                        num_cus=__import__("torch").cuda.get_device_properties(0).multi_processor_count, head_fuse="off")
    assert plan["inline_compact"] == 1 and plan["work_items"] == n
    batch = tl.DecodeBatch(g, n, Hq)
    batch.prepare(ids, stream())
    q = f16bits(rng, (n, Hq, D))
    nk, nv = f16bits(rng, (n, Hkv * D)), f16bits(rng, (n, Hkv * D))
    dq, dnk, dnv = to_dev(q), to_dev(nk), to_dev(nv)
    out = empty_dev((n, Hq, D))
    scale = 1.0 / np.sqrt(D)
    batch.decode(0, dq.data_ptr(), dnk.data_ptr(), dnv.data_ptr(), out.data_ptr(), scale, stream())
    for i, s in enumerate(ids):
        o.append(s, 0, nk[i], nv[i], 1)
    if not paged:
        assert np.array_equal(read_dev(g.pool(), o.pool().size), o.pool())
    view = orc.cache_view(o.pool(), 1, Hkv, D, M, 0, [o.slot_of(s) for s in ids])
    ref32, _ = orc.attn_decode_gqa(q, view, lens + 1, Hq, Hkv, D, scale, nthreads=8)
    got = to_host(out).view(np.float16).astype(np.float32)
    errs = [rel_err(got[i], ref32[i]) for i in range(n)]
    assert max(errs) <= 1e-3, max(errs)
