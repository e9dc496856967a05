"""GPU: the block-granular pool (tl_kv_create_paged) against the oracle and
the reference-layout pool.

The oracle restates the reference's slot pool (src/kv_cache.cpp); a block
pool must hold, for every live sequence, the same logical cache contents
(bit-exact), and its decode steps must give the same attention outputs as
the slot pool of the product (bit-identical: same plan, same arithmetic) and
the oracle (<= 1e-3 normwise), while memory follows the tokens held."""
import numpy as np
import pytest

from devutil import empty_dev, read_dev, rel_err, stream, to_dev, to_host

pytestmark = pytest.mark.gpu


def f16bits(rng, shape):
    return rng.standard_normal(shape).astype(np.float32).astype(np.float16).view(np.uint16)


def pool_elems(g, L, H, D, bt):
    return L * 2 * (g.numBlocks() + 1) * bt * H * D


def check_raw_layout(g, o, ids, L, H, D, bt):
    """Every token of every live sequence sits at
    [layer][K|V][block][t % bt][H][D] of the pool, block = blockTable[t // bt]."""
    raw = read_dev(g.pool(), pool_elems(g, L, H, D, bt))
    nb1, row = g.numBlocks() + 1, H * D
    opool, M = o.pool(), g.config.max_seq_len
    for sid in ids:
        table, err = g.blockTable(sid)
        assert err is None
        n = g.getSeqLen(sid)
        assert len(table) == -(-n // bt)
        slot = o.slot_of(sid)
        for layer in range(L):
            for kv in range(2):
                for t in range(n):
                    src = (((slot * L + layer) * 2 + kv) * M + t) * row
                    dst = (((layer * 2 + kv) * nb1 + table[t // bt]) * bt + t % bt) * row
                    assert np.array_equal(raw[dst:dst + row], opool[src:src + row]), (sid, layer, kv, t)


def gather_all(tl, g, ids, L, H, D):
    lens = [g.getSeqLen(s) for s in ids]
    smax = max(lens + [1])
    batch = tl.DecodeBatch(g, len(ids), H)
    batch.prepare_lengths(ids, lens, stream())
    out = []
    for layer in range(L):
        k, v = empty_dev((len(ids), H, smax, D)), empty_dev((len(ids), H, smax, D))
        batch.gather(layer, k.data_ptr(), v.data_ptr(), smax, stream())
        out.append((to_host(k), to_host(v)))
    return out, lens, smax


@pytest.mark.parametrize("bt", [16, 64])
@pytest.mark.parametrize("D,G", [(64, 1), (128, 4), (128, 8)])
def test_block_pool_churn_matches_slot_pool_and_oracle(tl, orc, D, G, bt):
    """Random allocate / prompt append / decode step / release sequences
    (seeded).  After each decode step: block-pool output == slot-pool output
    (bits) and <= 1e-3 of the oracle; at the end: gathered contents and the
    raw block placement equal the oracle's slot contents."""
    rng = np.random.default_rng(D * 10 + G + bt)
    L, H, M, B = 2, 2, 768, 6
    Hq = H * G
    nb = 3 * M // bt  # half of what B full slots would reserve
    gb = tl.KVCacheManager(L, H, D, M, B, block_tokens=bt, num_blocks=nb)
    gs = tl.KVCacheManager(L, H, D, M, B)
    o = orc.KVCacheOracle(L, H, D, M, B)
    bb, bs = tl.DecodeBatch(gb, B, Hq), tl.DecodeBatch(gs, B, Hq)
    live, keep, steps, cap = [], [], 0, {}
    scale = 1.0 / np.sqrt(D)
    for it in range(40):
        r = rng.random()
        if r < 0.3 and len(live) < B:
            max_len = int(rng.integers(64, M + 1))
            n = int(rng.integers(1, max_len // 2 + 1))
            if gb.freeBlocks() < -(-n // bt) + len(live) + 1:
                continue
            a, _ = gb.allocateSequence(max_len)
            b, _ = gs.allocateSequence(max_len)
            c, _ = o.allocate(max_len)
            assert a == b == c and gb.slot_of(a) == o.slot_of(a)
            for layer in range(L):
                k, v = f16bits(rng, n * H * D), f16bits(rng, n * H * D)
                dk, dv = to_dev(k), to_dev(v)
                keep += [dk, dv]
                assert gb.appendKV(a, layer, dk.data_ptr(), dv.data_ptr(), n, stream()) is None
                assert gs.appendKV(a, layer, dk.data_ptr(), dv.data_ptr(), n, stream()) is None
                o.append(a, layer, k, v, n)
            for m in (gb, gs):
                assert m.advanceSeqLen(a, n) is None
            o.advance(a, n)
            live.append(a)
            cap[a] = max_len
        elif r < 0.45 and live:
            s = live.pop(int(rng.integers(len(live))))
            assert gb.releaseSequence(s) is None and gs.releaseSequence(s) is None
            o.release(s)
        elif live:
            ids = [s for s in live if o.seq_len(s) < cap[s]]
            need = sum(max(0, -(-(o.seq_len(s) + 1) // bt) - len(gb.blockTable(s)[0])) for s in ids)
            if not ids or need > gb.freeBlocks():
                continue
            bb.prepare(ids, stream())
            bs.prepare(ids, stream())
            n = len(ids)
            q = f16bits(rng, (n, Hq, D))
            for layer in range(L):
                nk, nv = f16bits(rng, (n, H * D)), f16bits(rng, (n, H * D))
                dq, dnk, dnv = to_dev(q), to_dev(nk), to_dev(nv)
                ob, os_ = empty_dev((n, Hq, D)), empty_dev((n, Hq, D))
                bb.decode(layer, dq.data_ptr(), dnk.data_ptr(), dnv.data_ptr(), ob.data_ptr(), scale,
                          stream())
                bs.decode(layer, dq.data_ptr(), dnk.data_ptr(), dnv.data_ptr(), os_.data_ptr(), scale,
                          stream())
                keep += [dq, dnk, dnv]
                for i, s in enumerate(ids):
                    o.append(s, layer, nk[i], nv[i], 1)
                hb, hs = to_host(ob), to_host(os_)
                assert np.array_equal(hb, hs), (it, layer)
                lens = np.array([o.seq_len(s) + 1 for s in ids])
                view = orc.cache_view(o.pool(), L, H, D, M, layer, [o.slot_of(s) for s in ids])
                ref32, _ = orc.attn_decode_gqa(q, view, lens, Hq, H, D, scale, nthreads=8)
                got = hb.view(np.float16).astype(np.float32)
                assert max(rel_err(got[i], ref32[i]) for i in range(n)) <= 1e-3
            bb.commit(1)
            bs.commit(1)
            for s in ids:
                o.advance(s, 1)
            steps += 1
        used = sum(-(-gb.getSeqLen(s) // bt) for s in live)
        assert gb.getUsedMemory() == used * gb.blockBytes()
        assert gb.freeBlocks() == nb - used
    assert steps > 0 and live
    got, lens, smax = gather_all(tl, gb, live, L, H, D)
    for layer in range(L):
        view = orc.cache_view(o.pool(), L, H, D, M, layer, [o.slot_of(s) for s in live])
        assert np.array_equal(got[layer][0], orc.gather(view, 0, lens, H, D, smax))
        assert np.array_equal(got[layer][1], orc.gather(view, 1, lens, H, D, smax))
    check_raw_layout(gb, o, live, L, H, D, bt)


def test_block_pool_accounting_and_exhaustion(tl):
    L, H, D, M, B, bt, nb = 1, 2, 64, 256, 4, 16, 10
    g = tl.KVCacheManager(L, H, D, M, B, block_tokens=bt, num_blocks=nb)
    blk = bt * H * D * L * 2 * 2
    assert g.blockBytes() == blk and g.numBlocks() == nb
    assert g.getTotalMemory() == nb * blk and g.getUsedMemory() == 0
    rng = np.random.default_rng(5)
    src = to_dev(f16bits(rng, M * H * D))
    p = src.data_ptr()
    a, _ = g.allocateSequence(M)
    b, _ = g.allocateSequence(M)
    assert g.getUsedMemory() == 0  # allocation alone holds no blocks
    assert g.appendKV(a, 0, p, p, 100, stream()) is None  # 7 blocks
    assert g.freeBlocks() == 3 and g.getUsedMemory() == 7 * blk
    assert g.getFreeMemory() == 3 * blk
    err = g.appendKV(b, 0, p, p, 64, stream())  # needs 4
    assert err is not None and "exhausted" in err
    assert g.freeBlocks() == 3 and g.blockTable(b)[0] == [] and g.getSeqLen(b) == 0
    assert g.appendKV(b, 0, p, p, 48, stream()) is None
    assert g.freeBlocks() == 0
    assert g.advanceSeqLen(a, 100) is None and g.getSeqLen(a) == 100
    err = g.advanceSeqLen(a, 20)  # would need an 8th block
    assert err is not None and "exhausted" in err and g.getSeqLen(a) == 100
    assert g.advanceSeqLen(a, 12) is None and g.getSeqLen(a) == 112
    batch = tl.DecodeBatch(g, B, H)
    with pytest.raises(tl.TinyLLMError, match="exhausted"):
        batch.prepare([a, b], stream())  # a needs block 8 for position 112
    assert batch.info()["n"] == 0
    assert g.releaseSequence(a) is None
    assert g.freeBlocks() == 7 and g.getUsedMemory() == 3 * blk
    assert g.advanceSeqLen(b, 48) is None
    batch.prepare([b], stream())  # position 48 opens block 4
    assert g.freeBlocks() == 6 and len(g.blockTable(b)[0]) == 4
    assert "block" in g.getCacheChecked(b, 0)[1]
    assert "block pool" in g.setBlockMap(16, np.arange(B * M // 16, dtype=np.int32))
    ids = [g.allocateSequence(16)[0] for _ in range(3)]
    assert None not in ids
    sid, err = g.allocateSequence(16)
    assert sid is None and "exhausted" in err  # max_batch_size live sequences
    for s in ids + [b]:
        assert g.releaseSequence(s) is None
    assert g.freeBlocks() == nb and g.getUsedMemory() == 0


def test_create_paged_rejects_bad_geometry(tl):
    for bt, nb in [(8, 10), (24, 10), (0, 10), (16, 0), (16, -1)]:
        m, err = tl.KVCacheManager.create(num_layers=1, num_heads=2, head_dim=64, max_seq_len=256,
                                          max_batch_size=2, block_tokens=bt or -16, num_blocks=nb)
        assert m is None and err


def test_block_pool_batched_append_and_projection(tl, orc):
    """DecodeBatch.append over several layers and the fused projection
    epilogue write the same cache contents into a block pool as into the
    slot pool."""
    rng = np.random.default_rng(9)
    L, H, D, M, B, bt = 3, 2, 64, 256, 4, 16
    gb = tl.KVCacheManager(L, H, D, M, B, block_tokens=bt, num_blocks=40)
    gs = tl.KVCacheManager(L, H, D, M, B)
    keep, ids = [], []
    for n in (15, 16, 33, 70):
        a, _ = gb.allocateSequence(M)
        gs.allocateSequence(M)
        for layer in range(L):
            k, v = to_dev(f16bits(rng, n * H * D)), to_dev(f16bits(rng, n * H * D))
            keep += [k, v]
            for m in (gb, gs):
                assert m.appendKV(a, layer, k.data_ptr(), v.data_ptr(), n, stream()) is None
        for m in (gb, gs):
            m.advanceSeqLen(a, n)
        ids.append(a)
    nk, nv = to_dev(f16bits(rng, L * B * H * D)), to_dev(f16bits(rng, L * B * H * D))
    hidden, gsz = 128, 32
    x = to_dev(f16bits(rng, (B, hidden)))
    w = [rng.integers(-128, 128, size=(hidden, H * D), dtype=np.int64).astype(np.int8) for _ in range(2)]
    sc = [orc.f2h((np.abs(rng.standard_normal((hidden // gsz, H * D))) * 0.02 + 1e-3).astype(np.float32))
          for _ in range(2)]
    import devutil
    dw = [devutil.to_dev_raw(a) for a in w]
    ds = [to_dev(a) for a in sc]
    for m in (gb, gs):
        batch = tl.DecodeBatch(m, B, H)
        batch.prepare(ids, stream())
        batch.append(0, L, nk.data_ptr(), nv.data_ptr(), stream())
        batch.commit(1)
        batch.prepare(ids, stream())
        batch.project(1, x.data_ptr(), hidden, gsz, dw[0].data_ptr(), ds[0].data_ptr(),
                      dw[1].data_ptr(), ds[1].data_ptr(), 0, 0, 0, stream())
        batch.commit(1)
    got_b, lens, smax = gather_all(tl, gb, ids, L, H, D)
    got_s, lens_s, _ = gather_all(tl, gs, ids, L, H, D)
    assert lens == lens_s == [17, 18, 35, 72]
    for layer in range(L):
        for kv in range(2):
            assert np.array_equal(got_b[layer][kv], got_s[layer][kv]), (layer, kv)
