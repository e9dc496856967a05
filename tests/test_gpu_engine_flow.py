"""GPU: every row of the path in one engine-shaped flow, against the oracle.

A two-layer GQA model's attention side runs the way InferenceEngine drives
TransformerLayer::attention (src/inference_engine.cpp:233-291,
src/transformer.cpp:200-247), on a block pool:

  * prompts are prefilled in chunks through PrefillBatch (append + causal
    attention over the cache, each chunk continuing the cached ones);
  * decode steps run DecodeBatch.project (Q/K/V projections with the K/V
    rows written straight into the cache), DecodeBatch.attention and the
    o_proj + residual (w8a16_matmul_residual).

The oracle mirrors the cache contents and checks every stage: prefill and
decode attention <= 1e-3 normwise per row, projections and o_proj + residual
<= 1e-3 per row against the reference-order W8A16 product, and at the end
the gathered cache equal to the oracle's contents bit for bit."""
import numpy as np
import pytest

from devutil import empty_dev, rel_err, stream, to_dev, to_dev_raw, to_host

pytestmark = pytest.mark.gpu
TOL = 1e-3


def f16bits(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32).astype(np.float16).view(np.uint16)


def f32(bits):
    return np.asarray(bits).view(np.float16).astype(np.float32)


def rows_ok(got_bits, ref32):
    got = f32(got_bits).reshape(ref32.shape[0], -1)
    ref = ref32.reshape(ref32.shape[0], -1)
    return max(rel_err(got[i], ref[i]) for i in range(ref.shape[0]))


def test_prefill_chunks_then_decode_with_projections(tl, orc):
    rng = np.random.default_rng(2026)
    L, Hkv, G, D, hidden, gs = 2, 2, 4, 64, 256, 64
    Hq, M, slots = Hkv * G, 512, 4
    row, qrow = Hkv * D, Hq * D
    scale = 1.0 / np.sqrt(D)
    g = tl.KVCacheManager(L, Hkv, D, M, slots, block_tokens=16, num_blocks=slots * M // 32)
    o = orc.KVCacheOracle(L, Hkv, D, M, slots)
    keep = []

    # ---- prompts, prefilled in chunks (round r takes every prompt's r-th chunk)
    chunks = {37: [37], 130: [64, 66], 300: [128, 100, 72]}
    ids = []
    for _ in chunks:
        sid, err = g.allocateSequence(M)
        assert err is None
        o.allocate(M)
        ids.append(sid)
    pb = tl.PrefillBatch(g, slots, Hq)
    for r in range(3):
        part = [(sid, c[r]) for sid, c in zip(ids, chunks.values()) if r < len(c)]
        sids, counts = [p[0] for p in part], [p[1] for p in part]
        pb.prepare(sids, counts, stream())
        T = sum(counts)
        for layer in range(L):
            q, k, v = f16bits(rng, (T, Hq, D)), f16bits(rng, (T, row)), f16bits(rng, (T, row))
            dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
            out = empty_dev((T, Hq, D))
            keep += [dq, dk, dv]
            pb.run(layer, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), scale, stream())
            t0, rows, lens = 0, [], []
            for sid, n in part:
                p0 = o.seq_len(sid)
                o.append(sid, layer, k[t0:t0 + n].reshape(-1), v[t0:t0 + n].reshape(-1), n)
                rows += [o.slot_of(sid)] * n
                lens += [p0 + j + 1 for j in range(n)]
                t0 += n
            view = orc.cache_view(o.pool(), L, Hkv, D, M, layer, rows)
            ref, _ = orc.attn_decode_gqa(q, view, np.array(lens), Hq, Hkv, D, scale, nthreads=8)
            assert rows_ok(to_host(out), ref) <= TOL, (r, layer)
        pb.commit()
        for sid, n in part:
            o.advance(sid, n)
    assert [g.getSeqLen(s) for s in ids] == [37, 130, 300]

    # ---- decode steps: projections into the cache, attention, o_proj + residual
    def weights(k_in, n_out):
        w = rng.integers(-128, 128, size=(k_in, n_out), dtype=np.int64).astype(np.int8)
        s = orc.f2h((np.abs(rng.standard_normal((k_in // gs, n_out))) * 0.01 + 1e-3).astype(np.float32))
        return w, s
    # W_q/W_k/W_v: [hidden][heads * D]; W_o: [Hq * D][hidden] (transformer.cpp:208-247)
    W = [{"q": weights(hidden, qrow), "k": weights(hidden, row), "v": weights(hidden, row),
          "o": weights(qrow, hidden)} for _ in range(L)]
    for lw in W:
        assert lw["o"][0].shape == (qrow, hidden) and lw["q"][0].shape == (hidden, qrow)
    dW = [{k: (to_dev_raw(w), to_dev(s)) for k, (w, s) in lw.items()} for lw in W]
    n = len(ids)
    state = f16bits(rng, (n, hidden))  # the residual stream
    dstate = to_dev(state)
    batch = tl.DecodeBatch(g, slots, Hq)
    for step in range(4):
        batch.prepare(ids, stream())
        lens = [o.seq_len(s) + 1 for s in ids]
        for layer in range(L):
            x = f16bits(rng, (n, hidden))  # stands for rms_norm(state)
            dx = to_dev(x)
            q_out = empty_dev((n, qrow))
            keep.append(dx)
            (wq, sq), (wk, sk), (wv, sv), (wo, so) = (dW[layer][k] for k in "qkvo")
            batch.project(layer, dx.data_ptr(), hidden, gs, wk.data_ptr(), sk.data_ptr(), wv.data_ptr(),
                          sv.data_ptr(), wq.data_ptr(), sq.data_ptr(), q_out.data_ptr(), stream())
            # the projected rows, read back from the cache at each write position
            smax = max(lens)
            gk, gv = empty_dev((n, Hkv, smax, D)), empty_dev((n, Hkv, smax, D))
            batch.gather(layer, gk.data_ptr(), gv.data_ptr(), smax, stream())
            hk, hv = to_host(gk), to_host(gv)
            new_k = np.stack([hk[i, :, lens[i] - 1, :].reshape(-1) for i in range(n)])
            new_v = np.stack([hv[i, :, lens[i] - 1, :].reshape(-1) for i in range(n)])
            for name, got in (("k", new_k), ("v", new_v), ("q", to_host(q_out))):
                w, s = W[layer][name]
                ref32, _ = orc.w8a16_matmul(x, w, s, n, w.shape[1], hidden, gs)
                assert rows_ok(got, ref32) <= TOL, (step, layer, name)
            for i, sid in enumerate(ids):
                o.append(sid, layer, new_k[i], new_v[i], 1)
            out = empty_dev((n, Hq, D))
            batch.attention(layer, q_out.data_ptr(), out.data_ptr(), scale, stream())
            view = orc.cache_view(o.pool(), L, Hkv, D, M, layer, [o.slot_of(s) for s in ids])
            qh = to_host(q_out).reshape(n, Hq, D)
            ref, _ = orc.attn_decode_gqa(qh, view, np.array(lens), Hq, Hkv, D, scale, nthreads=8)
            attn = to_host(out)
            assert rows_ok(attn, ref) <= TOL, (step, layer, "attention")
            # o_proj + residual: state = fp16(state + fp16(attn @ W_o))
            before = to_host(dstate).copy()
            tl.w8a16_matmul_residual(out.data_ptr(), wo.data_ptr(), so.data_ptr(), dstate.data_ptr(), n,
                                     hidden, qrow, gs, stream())
            o32, _ = orc.w8a16_matmul(attn.reshape(n, qrow), W[layer]["o"][0], W[layer]["o"][1], n,
                                      hidden, qrow, gs)
            assert rows_ok(to_host(dstate), f32(before) + o32) <= TOL, (step, layer, "o_proj")
        batch.commit(1)
        for s in ids:
            o.advance(s, 1)

    # ---- the whole cache, gathered, equals the oracle's contents
    final = [o.seq_len(s) for s in ids]
    assert final == [g.getSeqLen(s) for s in ids] == [41, 134, 304]
    smax = max(final)
    db = tl.DecodeBatch(g, slots, Hq)
    db.prepare_lengths(ids, final, stream())
    for layer in range(L):
        gk, gv = empty_dev((n, Hkv, smax, D)), empty_dev((n, Hkv, smax, D))
        db.gather(layer, gk.data_ptr(), gv.data_ptr(), smax, stream())
        view = orc.cache_view(o.pool(), L, Hkv, D, M, layer, [o.slot_of(s) for s in ids])
        assert np.array_equal(to_host(gk), orc.gather(view, 0, final, Hkv, D, smax))
        assert np.array_equal(to_host(gv), orc.gather(view, 1, final, Hkv, D, smax))
    used = sum(-(-L_ // 16) for L_ in final)
    assert g.getUsedMemory() == used * g.blockBytes()
