"""GPU: tl_attn_decode_gqa_noalloc, the decode attention entry point that
allocates nothing (split-K partials and spilled plan metadata in the
library's static device scratch), against tl_attn_decode_gqa on the same
inputs: bit-identical outputs on two calls in a row, the second smaller than
the first, and the oracle's 1e-3 gate.  A call that needs more scratch than
the array holds is rejected before any launch."""
import ctypes as C

import numpy as np
import pytest
import torch

from devutil import rel_err, stream, to_host

pytestmark = pytest.mark.gpu


def paged_cache(tl, rng, lens, Hkv, D, blk=16):
    """K/V in 16-token blocks at seeded random physical positions; returns
    (keep-alive tensors, tl view, host pool bits, oracle block table)."""
    nblk = [max(1, -(-int(s) // blk)) for s in lens]
    total = sum(nblk)
    phys = rng.permutation(total).astype(np.int32)
    width = max(nblk)
    bt = np.zeros((len(lens), width), dtype=np.int32)
    o = 0
    for b, n in enumerate(nblk):
        bt[b, :n] = phys[o:o + n]
        o += n
    row = Hkv * D
    pool = (rng.standard_normal(2 * total * blk * row) * 1.0).astype(np.float16).view(np.uint16)
    dpool = torch.from_numpy(pool.view(np.int16).copy()).cuda()
    dbt = torch.from_numpy(bt.copy()).cuda()
    base = dpool.data_ptr()
    view = tl.KVView(base, base + 2 * total * blk * row, dbt.data_ptr(), width, 4, blk * row, row, D)
    return (dpool, dbt), view, pool, bt, total * blk * row


def run_pair(tl, orc, rng, lens, Hq, Hkv, D):
    keep, view, pool, bt, v_off = paged_cache(tl, rng, lens, Hkv, D)
    B = len(lens)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16).view(np.uint16)
    dq = torch.from_numpy(q.view(np.int16).copy()).cuda()
    ref_out = torch.empty((B, Hq, D), dtype=torch.float16, device="cuda")
    got_out = torch.full((B, Hq, D), float("nan"), dtype=torch.float16, device="cuda")
    scale = 1.0 / np.sqrt(D)
    tl.attn_decode_gqa(dq.data_ptr(), view, lens, Hq, Hkv, D, scale, ref_out.data_ptr(), stream())
    tl.attn_decode_gqa_noalloc(dq.data_ptr(), view, lens, Hq, Hkv, D, scale, got_out.data_ptr(),
                               stream())
    got, ref = to_host(got_out), to_host(ref_out)
    assert np.array_equal(got, ref), "noalloc output differs from tl_attn_decode_gqa"
    oview = orc.View(pool, 0, v_off, bt, 4, 16 * Hkv * D, Hkv * D, D)
    ref32, _ = orc.attn_decode_gqa(q, oview, np.asarray(lens), Hq, Hkv, D, scale, nthreads=8)
    g32 = got.view(np.float16).astype(np.float32)
    errs = [rel_err(g32[b], ref32[b]) for b in range(B)]
    assert max(errs) <= 1e-3, max(errs)
    return keep


def test_noalloc_matches_decode_gqa_twice_then_smaller(tl, orc):
    rng = np.random.default_rng(20261202)
    Hq, Hkv, D = 16, 2, 128
    # call 1: 300 sequences, one of 30000 tokens split into many chunks
    # (partials in the scratch), metadata beyond the kernel arguments (filled
    # into the scratch by the metadata kernel), empty sequences included
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    lens1 = np.concatenate([[30000, 0], rng.integers(1, 1000, 298)]).astype(np.int32)
    # the plan the entry point runs: ragged lengths, the chunk plan's items
    # with 2 kv heads per 8-wave workgroup
    p1 = tl.attn_plan(lens1, Hkv, num_cus=ncu, with_rows=False, head_fuse="current")
    assert p1["any_multi"] == 1 and p1["any_empty"] == 1 and p1["inline_words"] == -1
    assert (p1["head_fused"], p1["fused_chunked"]) == (2, 1) or ncu != 256
    run_pair(tl, orc, rng, lens1, Hq, Hkv, D)
    # call 2: five sequences, metadata in the kernel arguments, partials in
    # the scratch the first call left behind
    lens2 = np.array([5000, 100, 0, 3000, 1], dtype=np.int32)
    p2 = tl.attn_plan(lens2, Hkv, num_cus=ncu, with_rows=False, head_fuse="current")
    assert p2["any_multi"] == 1 and p2["inline_words"] > 0
    assert p2["head_fused"] == 0 or ncu != 256  # 8-wave per-head workgroups
    run_pair(tl, orc, rng, lens2, Hq, Hkv, D)


def test_noalloc_head_fused_twice_then_smaller(tl, orc):
    """Head-fused plans (several kv heads per workgroup): two items per
    sequence interleaving its tiles (partials in the scratch), then a smaller
    call with one item per sequence."""
    rng = np.random.default_rng(20261203)
    Hq, Hkv, D = 32, 8, 128
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    for B, lo, hi, nch in ((32, 4200, 4400, 2), (64, 2048, 2100, 1)):
        lens = rng.integers(lo, hi + 1, B).astype(np.int32)
        p = tl.attn_plan(lens, Hkv, num_cus=ncu, with_rows=False, head_fuse="current")
        assert p["head_fused"] == 2 or ncu != 256
        assert p["work_items"] == B * nch or ncu != 256
        run_pair(tl, orc, rng, lens, Hq, Hkv, D)


def test_noalloc_balanced_split_then_smaller(tl, orc):
    """Ragged MHA lengths whose whole sequences would run in per-head 8-wave
    workgroups two per CU take the planner's balanced split (head pairs in
    chunks, partials in the scratch, the merge launch); then a smaller call
    whose sequences stay whole."""
    rng = np.random.default_rng(20261205)
    Hq, Hkv, D = 16, 16, 128
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    lens1 = rng.integers(300, 2000, 32).astype(np.int32)
    p1 = tl.attn_plan(lens1, Hkv, num_cus=ncu, with_rows=False, head_fuse="current")
    assert (p1["chunk_tokens"], p1["head_fused"], p1["fused_chunked"], p1["any_multi"]) == (1280, 2, 1, 1) \
        or ncu != 256
    run_pair(tl, orc, rng, lens1, Hq, Hkv, D)
    lens2 = np.array([700, 650, 600, 500], dtype=np.int32)
    p2 = tl.attn_plan(lens2, Hkv, num_cus=ncu, with_rows=False, head_fuse="current")
    assert p2["any_multi"] == 0
    run_pair(tl, orc, rng, lens2, Hq, Hkv, D)


def test_noalloc_rejects_calls_beyond_the_scratch(tl, monkeypatch):
    """400 split items of 64 heads x (256 + 2) fp32 need 26 MB of partials,
    more than the 16 MiB array: rejected with a clear error, nothing runs."""
    assert tl.attn_noalloc_scratch_bytes() == 16 << 20
    monkeypatch.setenv("TL_ATTN_CHUNK", "256")
    B, Hq, Hkv, D = 100, 64, 8, 256
    buf = torch.zeros(1 << 16, dtype=torch.float16, device="cuda")
    bt = torch.zeros((B, 64), dtype=torch.int32, device="cuda")
    out = torch.zeros((B, Hq, D), dtype=torch.float16, device="cuda")
    view = tl.KVView(buf.data_ptr(), buf.data_ptr(), bt.data_ptr(), 64, 4, 16 * Hkv * D, Hkv * D, D)
    lens = np.full(B, 1000, dtype=np.int32)
    with pytest.raises(tl.TinyLLMError, match="bytes of scratch"):
        tl.attn_decode_gqa_noalloc(buf.data_ptr(), view, lens, Hq, Hkv, D, 0.0625, out.data_ptr(),
                                   stream())
    torch.cuda.synchronize()
    assert not out.any().item()


def test_noalloc_allocates_nothing_on_a_first_large_call(tl, orc):
    """After one small call (code objects loaded, the scratch address looked
    up), a first call with a much larger split plan leaves the device's free
    memory unchanged to the byte."""
    rng = np.random.default_rng(20261204)
    Hq, Hkv, D = 32, 8, 128
    keep = run_pair(tl, orc, rng, np.array([300, 17], dtype=np.int32), Hq, Hkv, D)
    lens = np.concatenate([[24000, 0], rng.integers(1, 3000, 250)]).astype(np.int32)
    keep2, view, _, _, _ = paged_cache(tl, rng, lens, Hkv, D)
    q = torch.randn((len(lens), Hq, D), dtype=torch.float16, device="cuda")
    out = torch.empty((len(lens), Hq, D), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    tl.attn_decode_gqa_noalloc(q.data_ptr(), view, lens, Hq, Hkv, D, 0.0884, out.data_ptr(),
                               stream())
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.isfinite(out.float()).all().item()
    del keep, keep2


def test_noalloc_replays_under_hip_graph_capture(tl, orc):
    """A call captured in a HIP graph (torch.cuda.CUDAGraph; the split-K
    partials and the plan metadata in the static scratch, the metadata
    written by a kernel) and replayed on new cache and query values, with
    eager calls between the replays: every replay equals tl_attn_decode_gqa
    on the same inputs, bit for bit."""
    rng = np.random.default_rng(20261205)
    Hq, Hkv, D = 32, 8, 128
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    lens = np.concatenate([[20000, 0], rng.integers(1, 2000, 298)]).astype(np.int32)
    p = tl.attn_plan(lens, Hkv, num_cus=ncu, with_rows=False, head_fuse="current")
    assert p["any_multi"] == 1 and p["inline_words"] == -1  # partials and metadata in scratch
    (dpool, dbt), view, _, _, _ = paged_cache(tl, rng, lens, Hkv, D)
    B = len(lens)
    dq = torch.randn((B, Hq, D), dtype=torch.float16, device="cuda")
    got = torch.empty((B, Hq, D), dtype=torch.float16, device="cuda")
    ref = torch.empty((B, Hq, D), dtype=torch.float16, device="cuda")
    scale = 1.0 / np.sqrt(D)
    # warm-up outside the capture: per-device set-up happens on a first call
    tl.attn_decode_gqa_noalloc(dq.data_ptr(), view, lens, Hq, Hkv, D, scale, got.data_ptr(),
                               stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tl.attn_decode_gqa_noalloc(dq.data_ptr(), view, lens, Hq, Hkv, D, scale, got.data_ptr(),
                                   stream())
    torch.cuda.synchronize()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(20261205)
    for rep in range(3):
        dq.copy_(torch.randn(dq.shape, generator=gen, device="cuda", dtype=torch.float16))
        dpool.copy_(torch.randn(dpool.shape, generator=gen, device="cuda",
                                dtype=torch.float16).view(torch.int16))
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        tl.attn_decode_gqa(dq.data_ptr(), view, lens, Hq, Hkv, D, scale, ref.data_ptr(), stream())
        torch.cuda.synchronize()
        assert np.array_equal(to_host(got), to_host(ref)), f"replay {rep} differs"
        assert torch.isfinite(got.float()).all().item()
    del graph
