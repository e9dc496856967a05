"""GPU: a decode plan that splits a sequence into several chunks merges the
chunks' partials either inside the attention launch (the workgroup that
completes a sequence's last chunk of a kv-head block merges them, counting
in a zeroed counter it leaves at zero) or in a second launch
(attn_merge_kernel).  Both forms must give identical bits, on both kernels
(VALU / MMA score paths), head_dim 64 and 128, every group size, per-head and
head-fused plans, contiguous and paged caches; over repeated calls (the
counters start at zero again) and a larger batch after a smaller one (the
counter buffer grows); and the 1e-3 gate against the oracle."""
import numpy as np
import pytest

from devutil import empty_dev, rel_err, stream, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture
def settings(tl):
    before = (tl.get_score_path(), tl.get_head_fuse(), tl.get_fused_merge())
    yield
    tl.set_score_path(before[0])
    tl.set_head_fuse(before[1])
    tl.set_fused_merge(before[2])


def f16bits(rng, shape):
    return rng.standard_normal(shape).astype(np.float32).astype(np.float16).view(np.uint16)


def build(tl, orc, rng, lens, Hkv, D, M, paged):
    g = tl.KVCacheManager(1, Hkv, D, M, len(lens))
    o = orc.KVCacheOracle(1, Hkv, D, M, len(lens))
    if paged:
        perm = rng.permutation(len(lens) * (M // 16)).astype(np.int32)
        assert g.setBlockMap(16, perm) is None
    ids, keep = [], []
    for S in lens:
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
    return g, o, ids, keep


RAGGED = [1, 300, 1100, 2100, 4600, 700]


@pytest.mark.parametrize("lens", ["ragged", "uniform"])
@pytest.mark.parametrize("hf", [1, 0])  # head-fuse setting: 1 = off, 0 = auto
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("path", [0, 3])
def test_fused_merge_same_bits_as_merge_launch(tl, orc, settings, monkeypatch, path, D, G, paged, hf,
                                               lens):
    """Ragged lengths with 256-token chunks (most sequences split, one whole);
    uniform lengths with the planner's own plan (head-fused interleaved items
    at head_dim 128 when hf = 0)."""
    tl.set_score_path(path)
    tl.set_head_fuse(hf)
    Hkv = 2 if lens == "ragged" else 8
    if lens == "ragged":
        monkeypatch.setenv("TL_ATTN_CHUNK", "256")
        L = RAGGED
    else:
        L = [3000] * 8
    rng = np.random.default_rng(path * 1000 + D * 10 + G + (500 if paged else 0) + 50 * hf)
    M = 4608
    g, o, ids, keep = build(tl, orc, rng, L, Hkv, D, M, paged)
    Hq, B = Hkv * G, len(ids)
    batch = tl.DecodeBatch(g, B, Hq)
    batch.prepare(ids, stream())
    q = f16bits(rng, (B, Hq, D))
    nk, nv = f16bits(rng, (B, Hkv * D)), f16bits(rng, (B, Hkv * D))
    dq, dnk, dnv = to_dev(q), to_dev(nk), to_dev(nv)
    scale = 1.0 / np.sqrt(D)
    ncu = __import__("torch").cuda.get_device_properties(0).multi_processor_count
    plan = tl.attn_plan(np.array(L, dtype=np.int32) + 1, Hkv, num_cus=ncu, head_fuse="current",
                        head_dim=D)
    assert plan["any_multi"] == 1 and plan["any_empty"] == 0, plan

    def step():
        out = empty_dev((B, Hq, D))
        batch.decode(0, dq.data_ptr(), dnk.data_ptr(), dnv.data_ptr(), out.data_ptr(), scale,
                     stream())
        return to_host(out)

    tl.set_fused_merge(False)
    ref = step()
    tl.set_fused_merge(True)
    for _ in range(3):  # counters back at zero after every launch
        assert np.array_equal(step(), ref)
    for i, sid in enumerate(ids):
        o.append(sid, 0, nk[i], nv[i], 1)
    view = orc.cache_view(o.pool(), 1, Hkv, D, M, 0, [o.slot_of(s) for s in ids])
    ref32, _ = orc.attn_decode_gqa(q, view, np.array(L) + 1, Hq, Hkv, D, scale, nthreads=8)
    got = ref.view(np.float16).astype(np.float32)
    errs = [rel_err(got[i], ref32[i]) for i in range(B)]
    assert max(errs) <= 1e-3, errs


def test_fused_merge_counters_grow(tl, orc, settings, monkeypatch):
    """tl_attn_decode_gqa (the library's shared workspace): a 4-sequence call,
    then 200 sequences x 8 kv heads (1600 counters, past the first buffer's
    1024), then the small call again; each against the second-launch merge."""
    monkeypatch.setenv("TL_ATTN_CHUNK", "256")
    rng = np.random.default_rng(7)
    Hkv, G, D = 8, 4, 64
    Hq = Hkv * G
    for B in (4, 200, 4):
        lens = rng.integers(300, 1200, B).astype(np.int32)
        smax = int(lens.max())
        row = Hkv * D
        k = f16bits(rng, B * smax * row)
        v = f16bits(rng, B * smax * row)
        dk, dv = to_dev(k), to_dev(v)
        view = tl.KVView(dk.data_ptr(), dv.data_ptr(), None, 0, 30, smax * row, row, D)
        q = f16bits(rng, (B, Hq, D))
        dq = to_dev(q)
        outs = []
        for fused in (False, True, True):
            tl.set_fused_merge(fused)
            out = empty_dev((B, Hq, D))
            tl.attn_decode_gqa(dq.data_ptr(), view, lens, Hq, Hkv, D, 1.0 / np.sqrt(D),
                               out.data_ptr(), stream())
            outs.append(to_host(out))
        assert np.array_equal(outs[1], outs[0]) and np.array_equal(outs[2], outs[0])
        pool = np.concatenate([k, v])
        oview = orc.View(pool, 0, k.size, None, 30, smax * row, row, D)
        ref32, _ = orc.attn_decode_gqa(q, oview, lens, Hq, Hkv, D, 1.0 / np.sqrt(D), nthreads=8)
        got = outs[1].view(np.float16).astype(np.float32)
        assert max(rel_err(got[b], ref32[b]) for b in range(B)) <= 1e-3
