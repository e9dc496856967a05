"""GPU: the benchmark configurations at their real sizes and launch plans,
against the oracle.

The bench times the decode kernel on plans that small tests do not reach:
cfg3's head-fused plan (an 8-wave workgroup per sequence and kv head pair,
each wave a quarter of the sequence's tiles of one head), cfg4's 5120-token chunks (two kv heads per 8-wave
workgroup; 3/2 of the per-head plan's 3328) over a permuted 16-token block
map of a pool larger than 4 GiB, cfg5's ~4600-token chunks over a block pool
with hundreds of group-8 sequences and the compact metadata encoding.  Each
test builds that state through appendKV, asserts the plan the bench reports
(DecodeBatch.info and tl_attn_plan), runs the decode step (fused append +
attention, the bench's call), and checks

  * the appended K/V rows and the rest of the cache bit-exact (whole pool
    where it is a slot pool; gathered through the batch for paged layouts),
  * every output row (sequence, query head) within 1e-3 normwise relative
    error of the oracle (oracle/kv_oracle.c, the fp32 restatement of
    kernels/attention.cu:11-112 over the cache layout of kv_cache.cpp:69-80;
    metric of tests/test_transformer.cu:80-92).

Inputs are drawn on the device (torch, seeded) and copied to the host for the
oracle.  Set TL_PARITY_REPORT=<file> to append each test's worst error as a
JSON line.  Config 2 at its 32 layers and config 5's churn on the bench's
slot pool are in test_gpu_bench_geometry.py."""
import json
import os

import numpy as np
import pytest
import torch

import workloads
from devutil import empty_dev, read_dev, rel_err, stream, to_dev, to_host

pytestmark = pytest.mark.gpu


def cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def host_bits(t):
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def randn(gen, shape, std=1.0):
    t = torch.randn(shape, generator=gen, device="cuda", dtype=torch.float16)
    return t * std if std != 1.0 else t


def report(name, errs, extra=None):
    path = os.environ.get("TL_PARITY_REPORT")
    line = {"test": name, "rows": int(np.size(errs)), "worst_rel_err": float(np.max(errs))}
    line.update(extra or {})
    print(json.dumps(line), flush=True)
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(line) + "\n")


def row_errors(got_bits, ref32):
    got = got_bits.view(np.float16).astype(np.float32)
    B, H = ref32.shape[:2]
    return np.array([[rel_err(got[b, h], ref32[b, h]) for h in range(H)] for b in range(B)])


def elem_err(got_bits, ref32):
    """Worst elementwise |a - b| / max(|b|, 1e-2 max|b|) over every (sequence,
    head) row, max|b| taken per row: the second, reported-only metric beside
    the normwise gate (small elements are compared against 1% of their row's
    largest, so one fp16 rounding of the output stays far below it)."""
    got = got_bits.view(np.float16).astype(np.float64)
    ref = np.asarray(ref32, dtype=np.float64)
    floor = 1e-2 * np.abs(ref).max(axis=-1, keepdims=True)
    den = np.maximum(np.abs(ref), floor)
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.where(den > 0, np.abs(got - ref) / den, np.where(got == ref, 0.0, np.inf))
    return float(e.max(initial=0.0))


def compact_view(orc, k_parts, v_parts, hkv, d):
    """Oracle view over the logical contents of each sequence: sequence b's
    tokens (k_parts[b] [S_b][Hkv*D]) start at a 16-token aligned offset of
    one host array (K region, then V region); the block table names those
    16-token blocks in order."""
    starts, off = [], 0
    for k in k_parts:
        starts.append(off)
        off += -(-k.shape[0] // 16) * 16
    row = hkv * d
    pool = np.zeros(2 * off * row, dtype=np.uint16)
    nblk = max(-(-k.shape[0] // 16) for k in k_parts)
    bt = np.zeros((len(k_parts), nblk), dtype=np.int32)
    for b, (k, v) in enumerate(zip(k_parts, v_parts)):
        s = k.shape[0]
        pool[starts[b] * row:(starts[b] + s) * row] = k.reshape(-1)
        pool[(off + starts[b]) * row:(off + starts[b] + s) * row] = v.reshape(-1)
        nb = -(-s // 16)
        bt[b, :nb] = starts[b] // 16 + np.arange(nb)
    return orc.View(pool, 0, off * row, bt, 4, 16 * row, row, d)


def test_cfg3_full_size(tl, orc):
    """Config 3 (headline): B=64, 32 q / 8 kv heads, D=128, context 8192, the
    bench's pool (max_seq_len 8448, the slot stride the bench times) and two
    consecutive decode steps."""
    cfg = workloads.config(3)
    B, Hq, Hkv, D = cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim
    ctx = int(cfg.contexts[0])
    M = workloads.fixed_pool_len(cfg, 100)
    assert M == 8448
    gen = torch.Generator(device="cuda")
    gen.manual_seed(workloads.seed(3, 1))
    g = tl.KVCacheManager(1, Hkv, D, M, B)
    k_all = randn(gen, (B, ctx, Hkv * D))
    v_all = randn(gen, (B, ctx, Hkv * D))
    ids = []
    for b in range(B):
        sid, err = g.allocateSequence(M)
        assert err is None, err
        assert g.appendKV(sid, 0, k_all[b].data_ptr(), v_all[b].data_ptr(), ctx, stream()) is None
        g.advanceSeqLen(sid, ctx)
        ids.append(sid)
    kh, vh = host_bits(k_all), host_bits(v_all)
    del k_all, v_all
    batch = tl.DecodeBatch(g, B, Hq)
    scale = cfg.scale
    slot_elems = g.slot_bytes() // 2
    for step in range(2):
        S = ctx + 1  # attended: the context plus the token this step appends
        batch.prepare(ids, stream())
        info = batch.info()
        # head-fused: one 8-wave workgroup per (sequence, kv head pair), 256
        # in all, one per CU; the whole sequence per workgroup, no merge
        assert info["chunk_tokens"] == 8448 and info["work_items"] == 64
        plan = tl.attn_plan(np.full(B, S, np.int32), Hkv, num_cus=cus(), head_fuse="auto")
        assert (plan["chunk_tokens"], plan["work_items"], plan["waves"], plan["head_fused"],
                plan["any_multi"]) == (8448, 64, 8, 2, 0)
        q = randn(gen, (B, Hq, D))
        nk = randn(gen, (B, Hkv * D))
        nv = randn(gen, (B, Hkv * D))
        out = empty_dev((B, Hq, D))
        batch.decode(0, q.data_ptr(), nk.data_ptr(), nv.data_ptr(), out.data_ptr(), scale, stream())
        batch.commit(1)
        pool = read_dev(g.pool(), B * slot_elems).reshape(B, 2, M, Hkv * D)
        slots = [g.slot_of(s) for s in ids]
        nkh, nvh = host_bits(nk), host_bits(nv)
        for b, s in enumerate(slots):
            assert np.array_equal(pool[s, 0, :ctx], kh[b]), f"K context, entry {b}"
            assert np.array_equal(pool[s, 1, :ctx], vh[b]), f"V context, entry {b}"
            assert np.array_equal(pool[s, 0, S - 1], nkh[b]), f"appended K, entry {b}"
            assert np.array_equal(pool[s, 1, S - 1], nvh[b]), f"appended V, entry {b}"
            assert not pool[s, :, S:].any(), f"bytes past the tail, entry {b}"
        view = orc.cache_view(pool.reshape(-1), 1, Hkv, D, M, 0, slots)
        ref32, _ = orc.attn_decode_gqa(host_bits(q), view, np.full(B, S), Hq, Hkv, D, scale,
                                       nthreads=16)
        bits = host_bits(out)
        errs = row_errors(bits, ref32)
        report(f"cfg3_full_size_step{step}", errs, {"attended": S, "chunk": info["chunk_tokens"],
                                                    "worst_elem_err": elem_err(bits, ref32)})
        assert errs.max() <= 1e-3, (step, float(errs.max()))
        # the next step's expected context: this step's (verified) tokens
        kh = np.stack([pool[s, 0, :S] for s in slots])
        vh = np.stack([pool[s, 1, :S] for s in slots])
        ctx = S
        del pool


def _check_gathered(tl, g, ids, subset, k_parts, v_parts, hkv, d):
    """Gather the attended tokens of `subset` entries through a batch and
    compare them bit for bit with the logical contents."""
    lens = [k_parts[b].shape[0] for b in subset]
    smax = max(lens)
    gb = tl.DecodeBatch(g, len(subset), hkv)
    gb.prepare_lengths([ids[b] for b in subset], lens, stream())
    gk = empty_dev((len(subset), hkv, smax, d))
    gv = empty_dev((len(subset), hkv, smax, d))
    gb.gather(0, gk.data_ptr(), gv.data_ptr(), smax, stream())
    hk, hv = to_host(gk), to_host(gv)
    for i, b in enumerate(subset):
        s = lens[i]
        exp_k = k_parts[b].reshape(s, hkv, d).transpose(1, 0, 2)
        exp_v = v_parts[b].reshape(s, hkv, d).transpose(1, 0, 2)
        assert np.array_equal(hk[i, :, :s], exp_k), f"K of entry {b}"
        assert np.array_equal(hv[i, :, :s], exp_v), f"V of entry {b}"
        assert not hk[i, :, s:].any() and not hv[i, :, s:].any()


def test_cfg4_ragged_permuted_blocks_over_4gib(tl, orc):
    """Config 4: B=128, lognormal contexts (median 2048, sigma 1, clipped to
    32768), 32 q / 8 kv heads, D=128, 16-token blocks behind the bench's
    seeded random permutation of a pool larger than 4 GiB, so most reads and
    appends land past byte offset 2^32."""
    cfg = workloads.config(4)
    B, Hq, Hkv, D, bt = cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim, cfg.block_tokens
    ctx = cfg.contexts.astype(np.int64)
    M = int((ctx.max() + 100 + 1 + 63) // 64 * 64)
    g = tl.KVCacheManager(1, Hkv, D, M, B)
    assert g.slot_bytes() * B > 4 << 30
    perm = workloads.block_permutation(B * M // bt, workloads.seed(4, 4))
    assert g.setBlockMap(bt, perm) is None
    gen = torch.Generator(device="cuda")
    gen.manual_seed(workloads.seed(4, 1))
    k_parts, v_parts, ids = [], [], []
    for b in range(B):
        sid, err = g.allocateSequence(M)
        assert err is None, err
        c = int(ctx[b])
        k, v = randn(gen, (c, Hkv * D)), randn(gen, (c, Hkv * D))
        assert g.appendKV(sid, 0, k.data_ptr(), v.data_ptr(), c, stream()) is None
        g.advanceSeqLen(sid, c)
        k_parts.append(host_bits(k))
        v_parts.append(host_bits(v))
        ids.append(sid)
    batch = tl.DecodeBatch(g, B, Hq)
    batch.prepare(ids, stream())
    info = batch.info()
    assert info["chunk_tokens"] == 5120 and info["work_items"] == 163
    plan = tl.attn_plan((ctx + 1).astype(np.int32), Hkv, num_cus=cus(), head_fuse="off")  # per head
    assert (plan["chunk_tokens"], plan["work_items"]) == (3328, 195)
    assert (plan["waves"], plan["any_multi"]) == (4, 1) and plan["inline_words"] > 0
    q, nk, nv = randn(gen, (B, Hq, D)), randn(gen, (B, Hkv * D)), randn(gen, (B, Hkv * D))
    out = empty_dev((B, Hq, D))
    batch.decode(0, q.data_ptr(), nk.data_ptr(), nv.data_ptr(), out.data_ptr(), cfg.scale, stream())
    nkh, nvh = host_bits(nk), host_bits(nv)
    for b in range(B):
        k_parts[b] = np.concatenate([k_parts[b], nkh[b][None]])
        v_parts[b] = np.concatenate([v_parts[b], nvh[b][None]])
    view = compact_view(orc, k_parts, v_parts, Hkv, D)
    ref32, _ = orc.attn_decode_gqa(host_bits(q), view, ctx + 1, Hq, Hkv, D, cfg.scale, nthreads=16)
    bits = host_bits(out)
    errs = row_errors(bits, ref32)
    report("cfg4_full_size", errs, {"chunk": info["chunk_tokens"],
                                    "pool_gib": round(g.slot_bytes() * B / (1 << 30), 2),
                                    "worst_elem_err": elem_err(bits, ref32)})
    assert errs.max() <= 1e-3, float(errs.max())
    # cache bytes: the longest sequences and the entries whose blocks sit
    # highest in the pool, read back through the batch gather
    order = np.argsort(-ctx)
    subset = sorted(set(order[:6].tolist()) | set(range(B - 6, B)))
    _check_gathered(tl, g, ids, subset, k_parts, v_parts, Hkv, D)


def test_cfg5_block_pool_500_live_group8(tl, orc):
    """Config 5's attention step: 520 live sequences of 64 q / 8 kv heads
    (group 8), D=128, prompts U{256..4096} plus up to 600 decoded tokens, on a
    16-token block pool whose blocks interleave across sequences (prompts
    appended in 512-token rounds), max_seq_len 5120; the step's metadata
    travels in the kernel arguments in the compact encoding (one word per
    sequence, 16 bits per work item)."""
    Hq, Hkv, D, M, bt, n = 64, 8, 128, 5120, 16, 520
    rng = np.random.default_rng(workloads.seed(5, 3))
    ctx = rng.integers(256, 4097, n) + rng.integers(0, 601, n)
    nblocks = int(((ctx + 1 + bt - 1) // bt).sum()) + 64
    g = tl.KVCacheManager(1, Hkv, D, M, n, block_tokens=bt, num_blocks=nblocks)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(workloads.seed(5, 1))
    ids = []
    for _ in range(n):
        sid, err = g.allocateSequence(M)
        assert err is None, err
        ids.append(sid)
    k_parts = [[] for _ in range(n)]
    v_parts = [[] for _ in range(n)]
    done = np.zeros(n, dtype=np.int64)
    while (done < ctx).any():
        for b in range(n):
            c = int(min(512, ctx[b] - done[b]))
            if c <= 0:
                continue
            k, v = randn(gen, (c, Hkv * D)), randn(gen, (c, Hkv * D))
            assert g.appendKV(ids[b], 0, k.data_ptr(), v.data_ptr(), c, stream()) is None
            g.advanceSeqLen(ids[b], c)
            k_parts[b].append(host_bits(k))
            v_parts[b].append(host_bits(v))
            done[b] += c
    k_parts = [np.concatenate(p) for p in k_parts]
    v_parts = [np.concatenate(p) for p in v_parts]
    batch = tl.DecodeBatch(g, n, Hq)
    batch.prepare(ids, stream())
    info = batch.info()
    plan = tl.attn_plan((ctx + 1).astype(np.int32), Hkv, num_cus=cus(), head_fuse="off")
    assert info["chunk_tokens"] == plan["chunk_tokens"] and info["work_items"] == plan["work_items"]
    # 520 entries of one chunk each: the compact kernel-argument metadata
    assert plan["waves"] == 4 and plan["inline_compact"] == 1 and plan["inline_words"] == 780
    assert plan["chunk_tokens"] >= 4096  # the long-chunk plan of the benchmark
    q, nk, nv = randn(gen, (n, Hq, D)), randn(gen, (n, Hkv * D)), randn(gen, (n, Hkv * D))
    out = empty_dev((n, Hq, D))
    scale = 1.0 / np.sqrt(D)
    batch.decode(0, q.data_ptr(), nk.data_ptr(), nv.data_ptr(), out.data_ptr(), scale, stream())
    batch.commit(1)
    nkh, nvh = host_bits(nk), host_bits(nv)
    for b in range(n):
        k_parts[b] = np.concatenate([k_parts[b], nkh[b][None]])
        v_parts[b] = np.concatenate([v_parts[b], nvh[b][None]])
    view = compact_view(orc, k_parts, v_parts, Hkv, D)
    ref32, _ = orc.attn_decode_gqa(host_bits(q), view, ctx + 1, Hq, Hkv, D, scale, nthreads=16)
    bits = host_bits(out)
    errs = row_errors(bits, ref32)
    report("cfg5_block_pool_520_live", errs, {"chunk": info["chunk_tokens"],
                                              "work_items": info["work_items"],
                                              "worst_elem_err": elem_err(bits, ref32)})
    assert errs.max() <= 1e-3, float(errs.max())
    order = np.argsort(-ctx)
    subset = sorted(set(order[:8].tolist()) | set(range(0, n, 65)))
    _check_gathered(tl, g, ids, subset, k_parts, v_parts, Hkv, D)
