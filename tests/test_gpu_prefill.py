"""GPU: prefill attention (the reference's compact attention_prefill and the
cache-native PrefillBatch), softmax and get_attention_weights against the
oracle.

  * attention_prefill vs orc_attention_prefill (attention.cu:131-237),
    <= 1e-3 normwise per (b, h, token) row; its last row vs the product's
    attention_decode (test_transformer.cu:222-300, 5% there);
  * PrefillBatch over slot, permuted-block and block pools, GQA groups 1-8,
    prompts that start empty or continue a cached prefix: appended cache
    bytes bit-exact (gather vs the oracle pool), query token j of a sequence
    <= 1e-3 of the oracle's decode attention over its first p0 + j + 1 keys;
    one-shot prefill == the same prompt in chunks, bit for bit;
  * get_attention_weights bit-exact (same fmaf order); softmax within one
    fp16 rounding of the oracle, rows summing to 1 (test_kernels.cu:
    505-740)."""
import numpy as np
import pytest

from devutil import empty_dev, rel_err, stream, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[8, 4], ids=["8waves", "4waves"])
def pwaves(request, tl):
    """Forces the prefill workgroup size (tl_prefill_set_waves) for one test:
    both forms of the kernel run every parity case (head_dim 256 has the
    4-wave form only)."""
    old = tl.get_prefill_waves()
    tl.set_prefill_waves(request.param)
    yield request.param
    tl.set_prefill_waves(old)


def f16bits(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32).astype(np.float16).view(np.uint16)


def f32(bits):
    return bits.view(np.float16).astype(np.float32)


@pytest.mark.parametrize("B,H,S,D", [(1, 2, 8, 32), (2, 4, 100, 64), (1, 8, 300, 128),
                                     (1, 2, 70, 256), (3, 1, 1, 64), (1, 3, 129, 128)])
def test_attention_prefill_matches_oracle(tl, orc, pwaves, B, H, S, D):
    rng = np.random.default_rng(B * 1000 + S + D)
    q, k, v = (f16bits(rng, (B, H, S, D)) for _ in range(3))
    scale = 1.0 / np.sqrt(D)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    out = empty_dev((B, H, S, D))
    tl.attention_prefill(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), scale, B, H, S,
                         D, stream())
    got = f32(to_host(out))
    ref, _ = orc.attention_prefill(q, k, v, scale, B, H, S, D, nthreads=8)
    errs = [rel_err(got[b, h, i], ref[b, h, i]) for b in range(B) for h in range(H) for i in range(S)]
    assert max(errs) <= 1e-3, max(errs)
    # last row == decode attention over the whole sequence (the reference's
    # IncrementalDecodingEquivalence property)
    qd = to_dev(np.ascontiguousarray(q[:, :, S - 1]))
    od = empty_dev((B, H, D))
    tl.attention_decode(qd.data_ptr(), dk.data_ptr(), dv.data_ptr(), od.data_ptr(), scale, B, H, S, D,
                        stream())
    assert rel_err(f32(to_host(od)), got[:, :, S - 1]) <= 1e-3


def test_attention_prefill_nonpositive_dims_are_noop(tl):
    out = to_dev(np.full(64, 0x3C00, np.uint16))
    z = to_dev(np.zeros(64, np.uint16))
    tl.attention_prefill(z.data_ptr(), z.data_ptr(), z.data_ptr(), out.data_ptr(), 1.0, 0, 1, 8, 8,
                         stream())
    assert np.all(to_host(out) == 0x3C00)


def make_pool(tl, kind, L, H, D, M, B, rng):
    if kind == "blocks":
        return tl.KVCacheManager(L, H, D, M, B, block_tokens=16, num_blocks=B * M // 16)
    g = tl.KVCacheManager(L, H, D, M, B)
    if kind == "perm":
        assert g.setBlockMap(16, rng.permutation(B * M // 16).astype(np.int32)) is None
    return g


@pytest.mark.parametrize("kind", ["slots", "perm", "blocks"])
@pytest.mark.parametrize("D,G", [(128, 4), (64, 1), (128, 8), (32, 2), (256, 1)])
def test_prefill_batch_matches_oracle(tl, orc, pwaves, kind, D, G):
    rng = np.random.default_rng(D * 7 + G + len(kind))
    L, H, M, B = 2, 2, 512, 5
    Hq = H * G
    g = make_pool(tl, kind, L, H, D, M, B, rng)
    o = orc.KVCacheOracle(L, H, D, M, B)
    keep = []
    prefix = [0, 37, 0, 130, 64]
    new = [1, 17, 64, 200, 45]
    ids = []
    for p0 in prefix:
        sid, _ = g.allocateSequence(M)
        o.allocate(M)
        ids.append(sid)
        if p0:
            for layer in range(L):
                k, v = f16bits(rng, p0 * H * D), f16bits(rng, p0 * H * D)
                dk, dv = to_dev(k), to_dev(v)
                keep += [dk, dv]
                assert g.appendKV(sid, layer, dk.data_ptr(), dv.data_ptr(), p0, stream()) is None
                o.append(sid, layer, k, v, p0)
            g.advanceSeqLen(sid, p0)
            o.advance(sid, p0)
    T = sum(new)
    pb = tl.PrefillBatch(g, B, Hq)
    pb.prepare(ids, new, stream())
    assert pb.info() == {"n": B, "tokens": T}
    scale = 1.0 / np.sqrt(D)
    for layer in range(L):
        q = f16bits(rng, (T, Hq, D))
        nk, nv = f16bits(rng, (T, H * D)), f16bits(rng, (T, H * D))
        dq, dk, dv = to_dev(q), to_dev(nk), to_dev(nv)
        out = empty_dev((T, Hq, D))
        pb.run(layer, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), scale, stream())
        t0 = 0
        rows, lens = [], []
        for sid, p0, n in zip(ids, prefix, new):
            o.append(sid, layer, nk[t0:t0 + n].reshape(-1), nv[t0:t0 + n].reshape(-1), n)
            rows += [o.slot_of(sid)] * n
            lens += [p0 + j + 1 for j in range(n)]
            t0 += n
        view = orc.cache_view(o.pool(), L, H, D, M, layer, rows)
        ref, _ = orc.attn_decode_gqa(q, view, np.array(lens), Hq, H, D, scale, nthreads=8)
        got = f32(to_host(out))
        errs = [rel_err(got[t], ref[t]) for t in range(T)]
        assert max(errs) <= 1e-3, (layer, int(np.argmax(errs)), max(errs))
        # the appended bytes: gather every sequence through the product
        smax = max(p + n for p, n in zip(prefix, new))
        db = tl.DecodeBatch(g, B, Hq)
        lens_now = [p + n for p, n in zip(prefix, new)]
        db.prepare_lengths(ids, lens_now, stream())
        gk, gv = empty_dev((B, H, smax, D)), empty_dev((B, H, smax, D))
        db.gather(layer, gk.data_ptr(), gv.data_ptr(), smax, stream())
        cv = orc.cache_view(o.pool(), L, H, D, M, layer, [o.slot_of(s) for s in ids])
        assert np.array_equal(to_host(gk), orc.gather(cv, 0, lens_now, H, D, smax))
        assert np.array_equal(to_host(gv), orc.gather(cv, 1, lens_now, H, D, smax))
    pb.commit()
    assert [g.getSeqLen(s) for s in ids] == [p + n for p, n in zip(prefix, new)]


@pytest.mark.parametrize("D,G", [(128, 4), (64, 8)])
def test_chunked_prefill_equals_one_shot(tl, pwaves, D, G):
    """A prompt prefilled in one call and the same prompt in three chunks
    (each chunk attending to the cached earlier ones) give identical bits."""
    rng = np.random.default_rng(5 + D + G)
    H, M, S = 2, 1024, 333
    Hq = H * G
    q = f16bits(rng, (S, Hq, D))
    k, v = f16bits(rng, (S, H * D)), f16bits(rng, (S, H * D))
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    scale = 1.0 / np.sqrt(D)
    outs = []
    for chunks in ([S], [100, 64, 169]):
        g = tl.KVCacheManager(1, H, D, M, 1)
        sid, _ = g.allocateSequence(M)
        pb = tl.PrefillBatch(g, 1, Hq)
        out = empty_dev((S, Hq, D))
        t0 = 0
        for n in chunks:
            pb.prepare([sid], [n], stream())
            pb.run(0, dq[t0:].data_ptr(), dk[t0:].data_ptr(), dv[t0:].data_ptr(), out[t0:].data_ptr(),
                   scale, stream())
            pb.commit()
            t0 += n
        outs.append(to_host(out))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("kind", ["slots", "blocks"])
@pytest.mark.parametrize("D,G", [(128, 4), (64, 8), (32, 1), (256, 2)])
def test_fused_prefill_equals_append_then_attention(tl, pwaves, kind, D, G):
    """PrefillBatch.run (one launch: keys at or past the write position read
    from new_k/new_v, the rows written into the cache by the attention
    kernel) == append() followed by attention(): identical cache bytes and
    identical outputs, for prompts that start empty or continue a cached
    prefix."""
    rng = np.random.default_rng(D + 3 * G + len(kind))
    L, H, M, B = 2, 2, 512, 4
    Hq = H * G
    prefix, new = [0, 70, 0, 200], [33, 64, 150, 1]
    outs, pools = [], []
    q = f16bits(rng, (sum(new), Hq, D))
    nk, nv = f16bits(rng, (sum(new), H * D)), f16bits(rng, (sum(new), H * D))
    pre = [(f16bits(rng, p0 * H * D), f16bits(rng, p0 * H * D)) for p0 in prefix]
    keep = []
    for fused in (False, True):
        g = make_pool(tl, kind, L, H, D, M, B, np.random.default_rng(7))
        ids = []
        for p0, (k, v) in zip(prefix, pre):
            sid, _ = g.allocateSequence(M)
            ids.append(sid)
            if p0:
                dk, dv = to_dev(k), to_dev(v)
                keep += [dk, dv]
                assert g.appendKV(sid, 1, dk.data_ptr(), dv.data_ptr(), p0, stream()) is None
                g.advanceSeqLen(sid, p0)
        pb = tl.PrefillBatch(g, B, Hq)
        pb.prepare(ids, new, stream())
        dq, dk, dv = to_dev(q), to_dev(nk), to_dev(nv)
        out = empty_dev((sum(new), Hq, D))
        keep += [dq, dk, dv]
        if fused:
            pb.run(1, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), D ** -0.5, stream())
        else:
            pb.append(1, dk.data_ptr(), dv.data_ptr(), stream())
            pb.attention(1, dq.data_ptr(), out.data_ptr(), D ** -0.5, stream())
        outs.append(to_host(out))
        lens = [p + n for p, n in zip(prefix, new)]
        db = tl.DecodeBatch(g, B, Hq)
        db.prepare_lengths(ids, lens, stream())
        smax = max(lens)
        gk, gv = empty_dev((B, H, smax, D)), empty_dev((B, H, smax, D))
        db.gather(1, gk.data_ptr(), gv.data_ptr(), smax, stream())
        pools.append((to_host(gk), to_host(gv)))
        keep.append(g)
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(pools[0][0], pools[1][0]) and np.array_equal(pools[0][1], pools[1][1])


@pytest.mark.parametrize("D,G", [(128, 4), (64, 8), (32, 1), (128, 1)])
def test_prefill_waves_give_identical_bits(tl, D, G):
    """The 4- and 8-wave workgroups compute every query row with the same
    per-wave code and tile order (tiles past a row's last key, which only the
    longer query tile visits, add exact zeros), so both give the same output
    and cache bits: PrefillBatch.run over prompts with and without a cached
    prefix, and the compact attention_prefill."""
    rng = np.random.default_rng(31 + D + G)
    H, M, B = 2, 1024, 4
    Hq = H * G
    prefix, new = [0, 130, 0, 64], [333, 200, 64, 7]
    q = f16bits(rng, (sum(new), Hq, D))
    nk, nv = f16bits(rng, (sum(new), H * D)), f16bits(rng, (sum(new), H * D))
    pre = [(f16bits(rng, p0 * H * D), f16bits(rng, p0 * H * D)) for p0 in prefix]
    old = tl.get_prefill_waves()
    outs, pools, keep = [], [], []
    try:
        for waves in (8, 4):
            tl.set_prefill_waves(waves)
            g = tl.KVCacheManager(1, H, D, M, B)
            ids = []
            for p0, (k, v) in zip(prefix, pre):
                sid, _ = g.allocateSequence(M)
                ids.append(sid)
                if p0:
                    dk, dv = to_dev(k), to_dev(v)
                    keep += [dk, dv]
                    assert g.appendKV(sid, 0, dk.data_ptr(), dv.data_ptr(), p0, stream()) is None
                    g.advanceSeqLen(sid, p0)
            pb = tl.PrefillBatch(g, B, Hq)
            pb.prepare(ids, new, stream())
            dq, dk, dv = to_dev(q), to_dev(nk), to_dev(nv)
            out = empty_dev((sum(new), Hq, D))
            keep += [dq, dk, dv]
            pb.run(0, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), D ** -0.5, stream())
            outs.append(to_host(out))
            lens = [p + n for p, n in zip(prefix, new)]
            db = tl.DecodeBatch(g, B, Hq)
            db.prepare_lengths(ids, lens, stream())
            gk, gv = empty_dev((B, H, max(lens), D)), empty_dev((B, H, max(lens), D))
            db.gather(0, gk.data_ptr(), gv.data_ptr(), max(lens), stream())
            pools.append((to_host(gk), to_host(gv)))
            keep.append(g)
            cq, ck, cv = (to_dev(f16bits(np.random.default_rng(9), (2, Hq, 300, D))) for _ in range(3))
            co = empty_dev((2, Hq, 300, D))
            tl.attention_prefill(cq.data_ptr(), ck.data_ptr(), cv.data_ptr(), co.data_ptr(), D ** -0.5, 2, Hq,
                                 300, D, stream())
            outs.append(to_host(co))
            keep += [cq, ck, cv, co]
    finally:
        tl.set_prefill_waves(old)
    assert np.array_equal(outs[0], outs[2]) and np.array_equal(outs[1], outs[3])
    assert np.array_equal(pools[0][0], pools[1][0]) and np.array_equal(pools[0][1], pools[1][1])


def test_prefill_batch_errors(tl):
    g = tl.KVCacheManager(1, 2, 64, 64, 3)
    a, _ = g.allocateSequence(64)
    b, _ = g.allocateSequence(10)
    pb = tl.PrefillBatch(g, 3, 4)
    with pytest.raises(tl.TinyLLMError, match="overflow"):
        pb.prepare([a, b], [5, 11], stream())
    assert pb.info() == {"n": 0, "tokens": 0}
    with pytest.raises(tl.TinyLLMError, match="positive"):
        pb.prepare([a], [0], stream())
    with pytest.raises(tl.TinyLLMError, match="duplicate"):
        pb.prepare([a, a], [1, 1], stream())
    with pytest.raises(tl.TinyLLMError, match="not found"):
        pb.prepare([99], [1], stream())
    with pytest.raises(tl.TinyLLMError, match="multiple"):
        tl.PrefillBatch(g, 3, 3)
    gb = tl.KVCacheManager(1, 2, 64, 64, 3, block_tokens=16, num_blocks=3)
    c, _ = gb.allocateSequence(64)
    d, _ = gb.allocateSequence(64)
    pbb = tl.PrefillBatch(gb, 3, 2)
    with pytest.raises(tl.TinyLLMError, match="exhausted"):
        pbb.prepare([c, d], [33, 1], stream())  # 3 + 1 blocks
    assert gb.freeBlocks() == 3
    pbb.prepare([c, d], [32, 16], stream())
    assert gb.freeBlocks() == 0


@pytest.mark.parametrize("causal", [True, False])
def test_attention_weights_bit_exact(tl, orc, causal):
    rng = np.random.default_rng(21)
    B, H, Lq, Lk, D = 2, 3, 9, 300, 48
    q, k = f16bits(rng, (B, H, Lq, D)), f16bits(rng, (B, H, Lk, D))
    dq, dk = to_dev(q), to_dev(k)
    w = empty_dev((B, H, Lq, Lk))
    scale = 1.0 / np.sqrt(D)
    tl.get_attention_weights(dq.data_ptr(), dk.data_ptr(), w.data_ptr(), scale, B, H, Lq, Lk, D,
                             causal, stream())
    _, ref = orc.get_attention_weights(q, k, scale, B, H, Lq, Lk, D, causal)
    assert np.array_equal(to_host(w), ref)


@pytest.mark.parametrize("rows,S", [(4, 16), (16, 128), (3, 1000), (1, 1)])
def test_softmax_matches_oracle(tl, orc, rows, S):
    rng = np.random.default_rng(rows + S)
    x = f16bits(rng, (rows, S), 2.0)
    dx = to_dev(x)
    y = empty_dev((rows, S))
    tl.softmax(dx.data_ptr(), y.data_ptr(), rows, S, stream())
    got = f32(to_host(y)).astype(np.float64)
    ref32, _ = orc.softmax(x, rows, S)
    assert np.all(np.abs(got - ref32) <= np.abs(ref32) * 2.0 ** -10 + 2.0 ** -24)
    sums = got.sum(axis=1)
    assert np.all((sums > 0.98) & (sums < 1.02)) and np.all(got >= 0)


def test_failed_prepare_leaves_an_empty_batch(tl):
    """A prepare that fails (here: cache overflow) must not leave the
    previous step's plan armed: prefill/attention/append after it are
    no-ops, and the pool keeps the committed bytes."""
    from devutil import read_dev
    rng = np.random.default_rng(4242)
    H, D, M, Hq = 2, 64, 128, 4
    g = tl.KVCacheManager(1, H, D, M, 2)
    sid, _ = g.allocateSequence(M)
    k, v = f16bits(rng, (100, H * D)), f16bits(rng, (100, H * D))
    dk, dv = to_dev(k), to_dev(v)
    pb = tl.PrefillBatch(g, 2, Hq)
    pb.prepare([sid], [100], stream())
    q = to_dev(f16bits(rng, (100, Hq, D)))
    out = empty_dev((100, Hq, D))
    pb.run(0, q.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), D ** -0.5, stream())
    pb.commit()
    before = read_dev(g.pool(), g.slot_bytes() // 2)
    with pytest.raises(tl.TinyLLMError, match="cache overflow"):
        pb.prepare([sid], [100], stream())          # 100 + 100 > 128
    assert pb.info() == {"n": 0, "tokens": 0}
    other = to_dev(f16bits(rng, (100, H * D)))
    pb.run(0, q.data_ptr(), other.data_ptr(), other.data_ptr(), out.data_ptr(), D ** -0.5, stream())
    pb.append(0, other.data_ptr(), other.data_ptr(), stream())
    pb.commit()
    assert np.array_equal(read_dev(g.pool(), g.slot_bytes() // 2), before)
    assert g.getSeqLen(sid) == 100
