"""GPU: the benchmark's own pool geometries and step logic, against the
oracle.

  * config 2 at its real 32 layers on the bench's slot pool (16 slots of
    2 x 32 x M x 32 x 128 fp16, about 35 GB: most slot and layer offsets lie
    past 2^32 bytes; the reference computes them in size_t,
    kv_cache.cpp:69-80);
  * config 5 on the bench's 1280-slot pool (26.8 GB) for the first steps of
    the bench's seeded event sequence, replayed through the bench's own step
    logic (workloads.ChurnDriver): range-appended prompts, fused token
    appends, commits, releases and slot reuse over stale bytes
    (kv_cache.cpp:82-137);
  * PrefillBatch appends that cross the range launch's limits (64 ranges,
    32768 tokens per launch; a range continues in the next launch), the
    bytes of appendKV(n) (kv_cache.cpp:226-233).

Cache bytes are compared bit for bit, attention rows within 1e-3 normwise
relative error of the oracle's fp32 output (metric of
tests/test_transformer.cu:80-92).  Set TL_PARITY_REPORT=<file> to append each
check's worst error as a JSON line."""
import numpy as np
import pytest
import torch

import workloads
from devutil import empty_dev, read_dev, stream, to_dev, to_host
from test_gpu_configs import cus, elem_err, host_bits, randn, report, row_errors

pytestmark = pytest.mark.gpu


def test_cfg2_32_layers_slot_pool_over_4gib(tl, orc):
    """Config 2: B=16, MHA 32/32 heads, D=128, contexts U{512..4096} (the
    bench's seeded draw), KV ~ 0.5 N(0,1), all 32 layers filled through
    appendKV, one decode step with the bench's call sequence (prepare, decode
    of every layer, commit).  Every layer: the appended rows bit-exact.
    Layers 0 and 31: the whole context, the appended row and the zero bytes
    past it bit-exact, and every attention row against the oracle."""
    cfg = workloads.config(2)
    B, Hq, Hkv, D, L = cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim, cfg.num_layers
    ctx = cfg.contexts.astype(np.int64)
    M = workloads.fixed_pool_len(cfg, 100)
    g = tl.KVCacheManager(L, Hkv, D, M, B)
    assert g.slot_bytes() * B >= 32 << 30 and L == 32
    gen = torch.Generator(device="cuda")
    gen.manual_seed(workloads.seed(2, 1))
    check_layers = (0, L - 1)
    host, ids = {}, []
    for b in range(B):
        sid, err = g.allocateSequence(M)
        assert err is None, err
        c = int(ctx[b])
        for layer in range(L):
            k = randn(gen, (c, Hkv * D), cfg.kv_std)
            v = randn(gen, (c, Hkv * D), cfg.kv_std)
            assert g.appendKV(sid, layer, k.data_ptr(), v.data_ptr(), c, stream()) is None
            if layer in check_layers:
                host[b, layer] = (host_bits(k), host_bits(v))
        g.advanceSeqLen(sid, c)
        ids.append(sid)
    batch = tl.DecodeBatch(g, B, Hq)
    batch.prepare(ids, stream())
    info = batch.info()
    plan = tl.attn_plan((ctx + 1).astype(np.int32), Hkv, num_cus=cus(), head_fuse="current")
    assert (info["chunk_tokens"], info["work_items"]) == (plan["chunk_tokens"], plan["work_items"])
    q = randn(gen, (L, B, Hq, D), cfg.q_std)
    nk = randn(gen, (L, B, Hkv * D), cfg.kv_std)
    nv = randn(gen, (L, B, Hkv * D), cfg.kv_std)
    outs = {}
    for layer in range(L):
        out = empty_dev((B, Hq, D))
        batch.decode(layer, q[layer].data_ptr(), nk[layer].data_ptr(), nv[layer].data_ptr(),
                     out.data_ptr(), cfg.scale, stream())
        if layer in check_layers:
            outs[layer] = out
    batch.commit(1)
    assert [g.getSeqLen(s) for s in ids] == (ctx + 1).tolist()
    row = Hkv * D
    slot_elems = g.slot_bytes() // 2
    layer_elems = 2 * M * row
    nkh, nvh = host_bits(nk), host_bits(nv)
    slots = [g.slot_of(s) for s in ids]
    assert max(slots) * slot_elems * 2 > 4 << 30
    for b, s in enumerate(slots):
        c = int(ctx[b])
        for layer in range(L):
            base = s * slot_elems + layer * layer_elems + c * row
            assert np.array_equal(read_dev(g.pool() + 2 * base, row), nkh[layer, b]), (b, layer)
            assert np.array_equal(read_dev(g.pool() + 2 * (base + M * row), row), nvh[layer, b]), \
                (b, layer)
    for layer in check_layers:
        lp = np.empty((B, 2, M, row), dtype=np.uint16)
        for b, s in enumerate(slots):
            c = int(ctx[b])
            lp[b] = read_dev(g.pool() + 2 * (s * slot_elems + layer * layer_elems),
                             layer_elems).reshape(2, M, row)
            k, v = host[b, layer]
            assert np.array_equal(lp[b, 0, :c], k), f"K context, entry {b}, layer {layer}"
            assert np.array_equal(lp[b, 1, :c], v), f"V context, entry {b}, layer {layer}"
            assert np.array_equal(lp[b, 0, c], nkh[layer, b])
            assert np.array_equal(lp[b, 1, c], nvh[layer, b])
            assert not lp[b, :, c + 1:].any(), f"bytes past the tail, entry {b}, layer {layer}"
        view = orc.cache_view(lp.reshape(-1), 1, Hkv, D, M, 0, list(range(B)))
        ref32, _ = orc.attn_decode_gqa(host_bits(q[layer]), view, ctx + 1, Hq, Hkv, D, cfg.scale,
                                       nthreads=16)
        bits = host_bits(outs[layer])
        errs = row_errors(bits, ref32)
        report(f"cfg2_32L_layer{layer}", errs, {"chunk": info["chunk_tokens"],
                                                "pool_gib": round(g.slot_bytes() * B / (1 << 30), 1),
                                                "worst_elem_err": elem_err(bits, ref32)})
        assert errs.max() <= 1e-3, (layer, float(errs.max()))
    del g, batch, q, nk, nv, outs
    torch.cuda.empty_cache()


def test_cfg5_churn_bench_events_on_the_slot_pool(tl, orc):
    """Config 5 on the bench's pool: 1280 slots of 5120 tokens (26.8 GB), 64 q
    / 8 kv heads, D=128, the first 120 steps of the bench's seeded event
    sequence through the bench's step logic (workloads.ChurnDriver), with
    fresh token rows every step.  The oracle replays the same allocations,
    prompt appends (the same source rows), token appends, commits and
    releases on the reference's slot allocator.  Every 10th step: every
    attention row within 1e-3 of the oracle.  At the end: the used slots of
    the pool (live sequences, the stale bytes of released ones, reused slots)
    bit-exact against the oracle's pool, and every live sequence gathered
    through a batch bit-exact."""
    Hq, Hkv, D, M, slots, steps, src_rows = 64, 8, 128, 5120, 1280, 120, 32768
    g = tl.KVCacheManager(1, Hkv, D, M, slots)
    o = orc.KVCacheOracle(1, Hkv, D, M, slots)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(workloads.seed(5, 1))
    src_k, src_v = randn(gen, (src_rows, Hkv * D)), randn(gen, (src_rows, Hkv * D))
    sk, sv = host_bits(src_k), host_bits(src_v)
    q = randn(gen, (slots, Hq, D))
    nk, nv = randn(gen, (slots, Hkv * D)), randn(gen, (slots, Hkv * D))
    out = empty_dev((slots, Hq, D))
    batch = tl.DecodeBatch(g, slots, Hq)
    drv = workloads.ChurnDriver(g, batch, tl.PrefillBatch(g, slots, Hq), slots=slots,
                                max_seq_len=M, hq=Hq, hkv=Hkv, head_dim=D, src_rows=src_rows)
    sim = workloads.ChurnSim(steps=steps, hq=Hq, hkv=Hkv, head_dim=D, max_seq_len=M, slots=slots)
    scale = 1.0 / np.sqrt(D)
    bufs = dict(q=q.data_ptr(), nk=nk.data_ptr(), nv=nv.data_ptr(), out=out.data_ptr(),
                scale=scale, src_k=src_k.data_ptr(), src_v=src_v.data_ptr())
    freed, reused, top_slot, checks, worst, worst_elem = set(), 0, 0, 0, 0.0, 0.0
    for ev in sim.events():
        nk.copy_(randn(gen, nk.shape))
        nv.copy_(randn(gen, nv.shape))
        check = ev.step % 10 == 9
        if check:
            q.copy_(randn(gen, q.shape))
        rec = drv.step(ev, stream(), record=True, **bufs)
        assert rec.rejected == 0 and not rec.preempted
        for sid, prompt, r0 in rec.admitted:
            oid, err = o.allocate(M)
            assert err is None and oid == sid, (sid, oid, err)
            slot = o.slot_of(sid)
            reused += slot in freed
            freed.discard(slot)
            top_slot = max(top_slot, slot)
            assert o.append(sid, 0, sk[r0:r0 + prompt], sv[r0:r0 + prompt], prompt) is None
            assert o.advance(sid, prompt) is None
        if rec.decoded_ids is None:  # nothing live this step
            assert not rec.released
            continue
        ids, lens = rec.decoded_ids, rec.decoded_lens
        n = len(ids)
        nkh, nvh = host_bits(nk[:n]), host_bits(nv[:n])
        for i, sid in enumerate(ids):
            assert o.append(int(sid), 0, nkh[i], nvh[i], 1) is None
        if check:
            view = orc.cache_view(o.pool(), 1, Hkv, D, M, 0, [o.slot_of(int(s)) for s in ids])
            ref32, _ = orc.attn_decode_gqa(host_bits(q[:n]), view, lens + 1, Hq, Hkv, D, scale,
                                           nthreads=16)
            bits = host_bits(out[:n])
            errs = row_errors(bits, ref32)
            worst = max(worst, float(errs.max()))
            worst_elem = max(worst_elem, elem_err(bits, ref32))
            checks += 1
            assert errs.max() <= 1e-3, (ev.step, float(errs.max()))
        for sid in ids:
            assert o.advance(int(sid), 1) is None
        for sid in rec.released:
            freed.add(o.slot_of(sid))
            assert o.release(sid) is None
    live, lens = drv.live()
    info = batch.info()
    report("cfg5_churn_slot_pool_120_steps", np.array([worst]),
           {"checks": checks, "live": int(len(live)), "reused_slots": reused,
            "chunk": info["chunk_tokens"], "work_items": info["work_items"],
            "worst_elem_err": worst_elem})
    assert checks >= steps // 10 - 1 and len(live) > 100 and reused > 0
    # the plan of the last steps: one chunk per sequence in the compact
    # kernel-argument encoding (head-fused chunk items on 256 CUs)
    plan = tl.attn_plan((lens).astype(np.int32), Hkv, num_cus=cus(), head_fuse="current")
    assert plan["inline_compact"] == 1
    assert plan["head_fused"] == 2 or cus() != 256
    # every slot ever used: live, stale and reused bytes
    slot_elems = g.slot_bytes() // 2
    used = (top_slot + 1) * slot_elems
    assert np.array_equal(read_dev(g.pool(), used), o.pool()[:used]), "pool bytes differ"
    # every live sequence through the batch gather, 32 at a time
    gb = tl.DecodeBatch(g, 32, Hkv)
    for i in range(0, len(live), 32):
        sub, sl = live[i:i + 32], lens[i:i + 32]
        smax = int(sl.max())
        gb.prepare_lengths(sub, sl, stream())
        view = orc.cache_view(o.pool(), 1, Hkv, D, M, 0, [o.slot_of(int(s)) for s in sub])
        for which in (0, 1):
            got = empty_dev((len(sub), Hkv, smax, D))
            gb.gather(0, got.data_ptr() if which == 0 else 0, got.data_ptr() if which else 0,
                      smax, stream())
            assert np.array_equal(to_host(got), orc.gather(view, which, sl, Hkv, D, smax)), \
                ("gather", i, which)
    drv.release_all()
    del g, batch, drv, gb
    torch.cuda.empty_cache()


@pytest.mark.parametrize("kind", ["slots", "blocks"])
def test_prefill_append_crosses_the_range_launch_limits(tl, orc, kind):
    """PrefillBatch.append of 72 sequences (more than the 64 ranges one
    launch carries) with one prompt of 33000 tokens (more than the 32768
    tokens of one launch: it continues in the next launch at a source-row
    offset) and one of exactly 32768, several on top of a cached prefix, on
    two layers: the bytes equal appendKV per sequence in the oracle -- the
    whole pool for the slot pool, every sequence gathered for the block
    pool."""
    rng = np.random.default_rng(20261206 + len(kind))
    L, Hkv, D, M, B = 2, 1, 32, 33792, 72
    row = Hkv * D
    counts = rng.integers(1, 300, B)
    counts[3], counts[10] = 33000, 32768
    prefix = np.where(rng.random(B) < 0.3, rng.integers(1, 600, B), 0)
    prefix[3], prefix[10] = 500, 0
    assert (prefix + counts <= M).all()
    if kind == "blocks":
        nblocks = int(((prefix + counts + 15) // 16).sum()) + 8
        g = tl.KVCacheManager(L, Hkv, D, M, B, block_tokens=16, num_blocks=nblocks)
    else:
        g = tl.KVCacheManager(L, Hkv, D, M, B)
    o = orc.KVCacheOracle(L, Hkv, D, M, B)
    ids, keep = [], []
    for b in range(B):
        sid, err = g.allocateSequence(M)
        assert err is None, err
        assert o.allocate(M)[0] == sid
        ids.append(sid)
        p0 = int(prefix[b])
        if p0:
            for layer in range(L):
                k = rng.integers(0, 1 << 16, p0 * row, dtype=np.uint16)
                v = rng.integers(0, 1 << 16, p0 * row, dtype=np.uint16)
                dk, dv = to_dev(k), to_dev(v)
                keep += [dk, dv]
                assert g.appendKV(sid, layer, dk.data_ptr(), dv.data_ptr(), p0, stream()) is None
                assert o.append(sid, layer, k, v, p0) is None
            g.advanceSeqLen(sid, p0)
            o.advance(sid, p0)
    T = int(counts.sum())
    assert T > 2 * 32768
    pb = tl.PrefillBatch(g, B, Hkv)
    pb.prepare(ids, counts.tolist(), stream())
    assert pb.info() == {"n": B, "tokens": T}
    for layer in range(L):
        nk = rng.integers(0, 1 << 16, T * row, dtype=np.uint16)  # every bit pattern
        nv = rng.integers(0, 1 << 16, T * row, dtype=np.uint16)
        dk, dv = to_dev(nk), to_dev(nv)
        pb.append(layer, dk.data_ptr(), dv.data_ptr(), stream())
        t0 = 0
        for b, sid in enumerate(ids):
            n = int(counts[b])
            assert o.append(sid, layer, nk[t0 * row:(t0 + n) * row], nv[t0 * row:(t0 + n) * row],
                            n) is None
            t0 += n
        torch.cuda.synchronize()
    pb.commit()
    for b, sid in enumerate(ids):
        o.advance(sid, int(counts[b]))
        assert g.getSeqLen(sid) == o.seq_len(sid) == int(prefix[b] + counts[b])
    if kind == "slots":
        assert np.array_equal(read_dev(g.pool(), o.pool().size), o.pool())
        return
    lens = [o.seq_len(s) for s in ids]
    gb = tl.DecodeBatch(g, 8, Hkv)
    for i in range(0, B, 8):
        sub, sl = ids[i:i + 8], lens[i:i + 8]
        smax = max(sl)
        gb.prepare_lengths(sub, sl, stream())
        for layer in range(L):
            view = orc.cache_view(o.pool(), L, Hkv, D, M, layer, [o.slot_of(s) for s in sub])
            k, v = empty_dev((len(sub), Hkv, smax, D)), empty_dev((len(sub), Hkv, smax, D))
            gb.gather(layer, k.data_ptr(), v.data_ptr(), smax, stream())
            assert np.array_equal(to_host(k), orc.gather(view, 0, sl, Hkv, D, smax)), (i, layer)
            assert np.array_equal(to_host(v), orc.gather(view, 1, sl, Hkv, D, smax)), (i, layer)
