"""GPU: the W8A16 product (tl_w8a16_matmul), o_proj + residual
(tl_w8a16_matmul_residual) and the decode projection with the append fused
into its epilogue (DecodeBatch.project), against the oracle's restatement of
kernels/w8a16_matmul.cu:71-98.  Bars: <= 1e-3 normwise per output row for the
MFMA path; bit-exact fp16 for the reference-order kernel; bit-exact cache
bytes between the fused projection and w8a16_matmul + appendKV(n=1)."""
import numpy as np
import pytest

from devutil import empty_dev, read_dev, rel_err, stream, to_dev, to_dev_raw, to_host

pytestmark = pytest.mark.gpu
TOL = 1e-3


def operands(orc, rng, M, N, K, gs):
    x = orc.f2h(rng.standard_normal((M, K)).astype(np.float32))
    w = rng.integers(-128, 128, size=(K, N), dtype=np.int64).astype(np.int8)
    s = orc.f2h((np.abs(rng.standard_normal(((K + gs - 1) // gs, N))) * 0.02 + 1e-3).astype(np.float32))
    return x, w, s


@pytest.fixture
def generic(tl):
    yield tl.w8a16_set_path
    tl.w8a16_set_path(0)


def rows_close(got16, ref32):
    got = got16.view(np.float16).astype(np.float32)
    return max(rel_err(got[i], ref32[i]) for i in range(got.shape[0]))


SHAPES = [  # (M, N, K, gs, mfma-eligible)
    (64, 1024, 4096, 128, True),   # cfg3 K projection
    (64, 256, 4096, 128, True),
    (1, 64, 128, 32, True),
    (17, 48, 96, 32, True),        # partial row tile, 16-column tail, K % 64 == 32
    (100, 80, 256, 64, True),      # two row tiles
    (300, 32, 512, 128, True),     # M > 256: no split-K
    (17, 48, 96, 64, True),        # K % 64 == 32 with a partial last scale group
    (5, 32, 160, 128, True),
    (9, 64, 1056, 256, True),      # several batches, the last one short
    # the decode kernel (M <= 64, K % 128 == 0, K <= 4096): row halves, waves
    # without a chunk (K = 384: 3 chunks for 8 waves), every fold width
    (33, 112, 384, 64, True),      # two row halves, M past the first by one
    (48, 4096, 4096, 32, True),    # a fold per k step
    (64, 6144, 4096, 256, True),   # a group over two chunks, three-block tiles
    (20, 3072, 2048, 512, True),   # one row half
    (64, 16, 128, 128, True),      # one block, one chunk
    (4, 8, 16, 8, False),          # the reference's test shapes (reference-order kernel)
    (17, 33, 65, 32, False),
    (64, 1, 128, 32, False),
]


@pytest.mark.parametrize("M,N,K,gs,mfma", SHAPES)
def test_w8a16_matches_oracle(tl, orc, M, N, K, gs, mfma):
    rng = np.random.default_rng(M * 131 + N * 7 + K)
    x, w, s = operands(orc, rng, M, N, K, gs)
    ref32, ref16 = orc.w8a16_matmul(x, w, s, M, N, K, gs)
    dx, dw, ds = to_dev(x), to_dev_raw(w), to_dev(s)
    out = empty_dev((M, N))
    tl.w8a16_matmul(dx.data_ptr(), dw.data_ptr(), ds.data_ptr(), out.data_ptr(), M, N, K, gs, stream())
    got = to_host(out)
    if mfma:
        assert rows_close(got, ref32) <= TOL
    else:  # reference-order kernel: same operations in the same order
        assert np.array_equal(got, ref16)


@pytest.mark.parametrize("M,N,K,gs", [(64, 1024, 4096, 128), (17, 48, 96, 32)])
def test_w8a16_reference_order_kernel_is_bit_exact(tl, orc, generic, M, N, K, gs):
    generic(1)
    rng = np.random.default_rng(5)
    x, w, s = operands(orc, rng, M, N, K, gs)
    _, ref16 = orc.w8a16_matmul(x, w, s, M, N, K, gs)
    dx, dw, ds = to_dev(x), to_dev_raw(w), to_dev(s)
    out = empty_dev((M, N))
    tl.w8a16_matmul(dx.data_ptr(), dw.data_ptr(), ds.data_ptr(), out.data_ptr(), M, N, K, gs, stream())
    assert np.array_equal(to_host(out), ref16)


def pack_np(w):
    """The packed layout, restated in numpy.  The B fragment of column block
    nb and k step ks is 64 lanes x 8 bytes, lane l holding rows 32ks +
    8(l/16) .. +7 of column 16nb + l%16 as offset-binary bytes (w + 128, the
    bits of w ^ 0x80).  Column block nb takes K*16 bytes from nb*K*16; in it
    steps 2p and 2p+1 share 1024 bytes, lane l's 16 bytes at 16l (step 2p
    first); a last unpaired step takes 8 bytes per lane."""
    K, N = w.shape
    ks_n = K // 32
    frag = np.empty((N // 16, ks_n, 64, 8), np.uint8)
    lanes = np.arange(64)
    wu = w.view(np.uint8) ^ 0x80
    for nb in range(N // 16):
        for ks in range(ks_n):
            rows = 32 * ks + 8 * (lanes // 16)[:, None] + np.arange(8)[None, :]
            frag[nb, ks] = wu[rows, 16 * nb + (lanes % 16)[:, None]]
    out = np.empty((N // 16, K * 16), np.uint8)
    pairs = ks_n // 2
    for nb in range(N // 16):
        paired = frag[nb, :2 * pairs].reshape(pairs, 2, 64, 8).transpose(0, 2, 1, 3)
        out[nb, :pairs * 1024] = paired.reshape(-1)
        if ks_n % 2:
            out[nb, pairs * 1024:] = frag[nb, ks_n - 1].reshape(-1)
    return out.view(np.int8).reshape(-1)


def test_w8a16_pack_layout(tl, orc):
    rng = np.random.default_rng(3)
    import torch
    for K, N in ((128, 48), (96, 32)):  # paired steps only; a last unpaired step
        w = rng.integers(-128, 128, size=(K, N), dtype=np.int64).astype(np.int8)
        dw = to_dev_raw(w)
        out = to_dev_raw(np.zeros(K * N, np.int8))
        tl.w8a16_pack(dw.data_ptr(), K, N, out.data_ptr(), stream())
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), pack_np(w))
    with pytest.raises(tl.TinyLLMError, match="multiple"):
        tl.w8a16_pack(dw.data_ptr(), 100, N, out.data_ptr(), stream())


def packed_dev(tl, w):
    K, N = w.shape
    dw = to_dev_raw(w)
    out = to_dev_raw(np.zeros(K * N, np.int8))
    tl.w8a16_pack(dw.data_ptr(), K, N, out.data_ptr(), stream())
    return out


@pytest.mark.parametrize("path", [0, 1, 2])
def test_w8a16_residual(tl, orc, generic, path):
    """hidden = fp16(hidden + fp16(x @ W)) (transformer.cpp:149-151, 246-247);
    path 0: MFMA on the reference layout, 1: reference-order kernel, 2: MFMA
    on packed weights."""
    generic(1 if path == 1 else 0)
    M, N, K, gs = 64, 512, 4096, 128
    rng = np.random.default_rng(11)
    x, w, s = operands(orc, rng, M, N, K, gs)
    hidden = orc.f2h(rng.standard_normal((M, N)).astype(np.float32))
    o32, o16 = orc.w8a16_matmul(x, w, s, M, N, K, gs)
    ref = hidden.copy()
    orc.add_inplace(ref, o16)
    dx, dw, ds, dh = to_dev(x), to_dev_raw(w), to_dev(s), to_dev(hidden)
    tl.w8a16_matmul_residual(dx.data_ptr(), dw.data_ptr(), ds.data_ptr(), dh.data_ptr(), M, N, K, gs,
                             stream())
    got = to_host(dh)
    if path == 1:
        assert np.array_equal(got, ref)
    else:
        ref32 = orc.h2f(hidden) + o32
        assert rows_close(got, ref32) <= TOL
    if path == 2:
        dp, dh2 = packed_dev(tl, w), to_dev(hidden)
        tl.w8a16_matmul_residual(dx.data_ptr(), dp.data_ptr(), ds.data_ptr(), dh2.data_ptr(), M, N, K,
                                 gs, stream(), packed=True)
        assert rows_close(to_host(dh2), ref32) <= TOL


PACKED_SHAPES = [sh[:4] for sh in SHAPES if sh[4]] + [
    (130, 96, 1056, 64),    # three row tiles, K % 512 == 32
    (64, 208, 4096, 256),   # a 16-column block tail in the last 64-column tile
    (64, 112, 2048, 512),
    (257, 48, 640, 32),     # M > 256: one split, epilogue in the GEMM kernel
]


@pytest.mark.parametrize("M,N,K,gs", PACKED_SHAPES)
def test_w8a16_packed_matches_oracle(tl, orc, M, N, K, gs):
    """The MFMA kernel on the reference layout (o_proj + residual onto a zero
    residual, i.e. fp16(acc)) stays within 1e-3 of the oracle, and on packed
    weights gives the same bits (same fragments, same summation order), again
    on a second call."""
    rng = np.random.default_rng(M * 3 + N + K * 5 + gs)
    x, w, s = operands(orc, rng, M, N, K, gs)
    ref32, _ = orc.w8a16_matmul(x, w, s, M, N, K, gs)
    zero = np.zeros((M, N), np.uint16)
    dx, dw, ds = to_dev(x), to_dev_raw(w), to_dev(s)
    dh, dh2 = to_dev(zero), to_dev(zero)
    tl.w8a16_matmul_residual(dx.data_ptr(), dw.data_ptr(), ds.data_ptr(), dh.data_ptr(), M, N, K, gs,
                             stream())
    dp = packed_dev(tl, w)
    tl.w8a16_matmul_residual(dx.data_ptr(), dp.data_ptr(), ds.data_ptr(), dh2.data_ptr(), M, N, K, gs,
                             stream(), packed=True)
    got, got_p = to_host(dh), to_host(dh2)
    assert rows_close(got, ref32) <= TOL
    assert np.array_equal(got, got_p)
    dh3 = to_dev(zero)
    tl.w8a16_matmul_residual(dx.data_ptr(), dp.data_ptr(), ds.data_ptr(), dh3.data_ptr(), M, N, K, gs,
                             stream(), packed=True)
    assert np.array_equal(to_host(dh3), got_p)


def test_w8a16_packed_interleaved_shapes_repeat_bits(tl, orc):
    """Interleaved packed calls of shapes with different row-tile, column-tile
    and split counts (sharing the library's split-K workspace) each give their
    first call's bits again."""
    rng = np.random.default_rng(77)
    runs = []
    for M, N, K, gs in [(64, 512, 4096, 128), (130, 96, 1056, 64), (200, 320, 2048, 32)]:
        x, w, s = operands(orc, rng, M, N, K, gs)
        dx, dp, ds = to_dev(x), packed_dev(tl, w), to_dev(s)
        runs.append((M, N, K, gs, dx, dp, ds))

    def call(M, N, K, gs, dx, dp, ds):
        dh = to_dev(np.zeros((M, N), np.uint16))
        tl.w8a16_matmul_residual(dx.data_ptr(), dp.data_ptr(), ds.data_ptr(), dh.data_ptr(), M, N, K,
                                 gs, stream(), packed=True)
        return to_host(dh)
    first = [call(*r) for r in runs]
    for _ in range(2):
        for r, f in zip(reversed(runs), reversed(first)):
            assert np.array_equal(call(*r), f)


def test_w8a16_nonpositive_dims_noop(tl):
    out = to_dev(np.full((2, 16), 0x3C00, np.uint16))
    tl.w8a16_matmul(0, 0, 0, out.data_ptr(), 0, 16, 32, 32, stream())  # M = 0
    assert np.all(to_host(out) == 0x3C00)


def _cache(tl, orc, rng, L, Hkv, D, M, lens, paged):
    slots = len(lens) + 1
    g = tl.KVCacheManager(L, Hkv, D, M, slots)
    o = orc.KVCacheOracle(L, Hkv, D, M, slots)
    if paged:
        perm = rng.permutation(slots * (M // 16)).astype(np.int32)
        assert g.setBlockMap(16, perm) is None
    ids, keep = [], []
    for S in lens:
        sid, _ = g.allocateSequence(M)
        o.allocate(M)
        for layer in range(L):
            k = orc.f2h(rng.standard_normal(S * Hkv * D).astype(np.float32))
            v = orc.f2h(rng.standard_normal(S * Hkv * D).astype(np.float32))
            dk, dv = to_dev(k), to_dev(v)
            keep += [dk, dv]
            assert g.appendKV(sid, layer, dk.data_ptr(), dv.data_ptr(), S, stream()) is None
            o.append(sid, layer, k, v, S)
        g.advanceSeqLen(sid, S)
        o.advance(sid, S)
        ids.append(sid)
    return g, o, ids, keep


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("paged", [False, True])
def test_project_fused_append(tl, orc, paged, packed):
    """Fused projection: cache bytes == w8a16_matmul + appendKV(n=1) (bit-exact,
    whole pool), K/V rows within 1e-3 of the oracle, q_out == w8a16_matmul of
    wq (bit-exact), and attention afterwards == decode() with the same rows.
    With packed weights the unfused products are the packed kernel's own
    (o_proj + residual onto zeros, i.e. fp16(acc))."""
    rng = np.random.default_rng(21 + paged)
    L, Hkv, G, D, hidden, gs = 2, 4, 4, 64, 512, 128
    Hq, row = Hkv * G, Hkv * D
    lens = [5, 300, 64, 1000]
    M = 1024 + 16
    g, o, ids, keep = _cache(tl, orc, rng, L, Hkv, D, M, lens, paged)
    g2, _, ids2, keep2 = _cache(tl, orc, np.random.default_rng(21 + paged), L, Hkv, D, M, lens, paged)
    B = len(ids)
    x = orc.f2h(rng.standard_normal((B, hidden)).astype(np.float32))
    _, wk, sk = operands(orc, rng, 1, row, hidden, gs)
    _, wv, sv = operands(orc, rng, 1, row, hidden, gs)
    _, wq, sq = operands(orc, rng, 1, Hq * D, hidden, gs)
    dx, dwk, dsk, dwv, dsv, dwq, dsq = (to_dev(x), to_dev_raw(wk), to_dev(sk), to_dev_raw(wv),
                                        to_dev(sv), to_dev_raw(wq), to_dev(sq))
    layer = 1
    # fused
    batch = tl.DecodeBatch(g, B, Hq)
    batch.prepare(ids, stream())
    q_out = empty_dev((B, Hq * D))
    if packed:
        pk, pv, pq = packed_dev(tl, wk), packed_dev(tl, wv), packed_dev(tl, wq)
        batch.project(layer, dx.data_ptr(), hidden, gs, pk.data_ptr(), dsk.data_ptr(), pv.data_ptr(),
                      dsv.data_ptr(), pq.data_ptr(), dsq.data_ptr(), q_out.data_ptr(), stream(),
                      packed=True)
    else:
        batch.project(layer, dx.data_ptr(), hidden, gs, dwk.data_ptr(), dsk.data_ptr(), dwv.data_ptr(),
                      dsv.data_ptr(), dwq.data_ptr(), dsq.data_ptr(), q_out.data_ptr(), stream())
    # unfused: w8a16_matmul into buffers, then batched appendKV(n=1) of layer 1
    kb, vb, qb = empty_dev((B, row)), empty_dev((B, row)), empty_dev((B, Hq * D))
    if packed:
        for w_, s_, out_, n_ in ((pk, dsk, kb, row), (pv, dsv, vb, row), (pq, dsq, qb, Hq * D)):
            out_.zero_()
            tl.w8a16_matmul_residual(dx.data_ptr(), w_.data_ptr(), s_.data_ptr(), out_.data_ptr(), B, n_,
                                     hidden, gs, stream(), packed=True)
    else:
        for w_, s_, out_, n_ in ((dwk, dsk, kb, row), (dwv, dsv, vb, row), (dwq, dsq, qb, Hq * D)):
            tl.w8a16_matmul(dx.data_ptr(), w_.data_ptr(), s_.data_ptr(), out_.data_ptr(), B, n_, hidden,
                            gs, stream())
    batch2 = tl.DecodeBatch(g2, B, Hq)
    batch2.prepare(ids2, stream())
    batch2.append(layer, 1, kb.data_ptr(), vb.data_ptr(), stream())
    pool_elems = g.slot_bytes() // 2 * (B + 1)
    assert np.array_equal(read_dev(g.pool(), pool_elems), read_dev(g2.pool(), pool_elems))
    assert np.array_equal(to_host(q_out), to_host(qb))
    # the appended rows against the oracle's product
    k32, _ = orc.w8a16_matmul(x, wk, sk, B, row, hidden, gs)
    v32, _ = orc.w8a16_matmul(x, wv, sv, B, row, hidden, gs)
    assert rows_close(to_host(kb), k32) <= TOL and rows_close(to_host(vb), v32) <= TOL
    # attention over the projected token == decode() fusing the same rows
    out1, out2 = empty_dev((B, Hq, D)), empty_dev((B, Hq, D))
    batch.attention(layer, q_out.data_ptr(), out1.data_ptr(), D ** -0.5, stream())
    g3, _, ids3, keep3 = _cache(tl, orc, np.random.default_rng(21 + paged), L, Hkv, D, M, lens, paged)
    batch3 = tl.DecodeBatch(g3, B, Hq)
    batch3.prepare(ids3, stream())
    batch3.decode(layer, qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), out2.data_ptr(), D ** -0.5, stream())
    assert np.array_equal(to_host(out1), to_host(out2))


def test_project_rejects_bad_calls(tl):
    g = tl.KVCacheManager(1, 2, 64, 64, 2)
    sid, _ = g.allocateSequence(64)
    batch = tl.DecodeBatch(g, 2, 2)
    batch.prepare_lengths([sid], [1], stream())
    with pytest.raises(tl.TinyLLMError, match="prepare"):
        batch.project(0, 16, 64, 32, 16, 16, 16, 16)
    batch.prepare([sid], stream())
    with pytest.raises(tl.TinyLLMError, match="all set or all null"):
        batch.project(0, 16, 64, 32, 16, 16, 16, 16, wq=16)
    with pytest.raises(tl.TinyLLMError, match="layer"):
        batch.project(3, 16, 64, 32, 16, 16, 16, 16)


@pytest.mark.parametrize("packed", [False, True])
def test_project_fused_append_llama_layer(tl, orc, packed):
    """The benchmarked shape: a Llama-3-8B layer (hidden 4096, 8 KV heads and
    32 query heads of 128, group 128) for a decode batch of 64.  The fused
    projection's column tiles span the K|V and V|Q segment boundaries; cache
    bytes and q_out equal w8a16_matmul + appendKV(n=1) bit for bit (both
    weight layouts), and the K, V and Q rows stay within 1e-3 of the oracle."""
    rng = np.random.default_rng(4096 + packed)
    L, Hkv, G, D, hidden, gs = 1, 8, 4, 128, 4096, 128
    Hq, row = Hkv * G, Hkv * D
    lens = [int(v) for v in np.random.default_rng(77).integers(1, 48, size=64)]
    M = 64
    g, o, ids, keep = _cache(tl, orc, rng, L, Hkv, D, M, lens, False)
    g2, _, ids2, keep2 = _cache(tl, orc, np.random.default_rng(4096 + packed), L, Hkv, D, M, lens, False)
    B = len(ids)
    x = orc.f2h(rng.standard_normal((B, hidden)).astype(np.float32))
    _, wk, sk = operands(orc, rng, 1, row, hidden, gs)
    _, wv, sv = operands(orc, rng, 1, row, hidden, gs)
    _, wq, sq = operands(orc, rng, 1, Hq * D, hidden, gs)
    dx, dsk, dsv, dsq = to_dev(x), to_dev(sk), to_dev(sv), to_dev(sq)
    if packed:
        dwk, dwv, dwq = packed_dev(tl, wk), packed_dev(tl, wv), packed_dev(tl, wq)
    else:
        dwk, dwv, dwq = to_dev_raw(wk), to_dev_raw(wv), to_dev_raw(wq)
    batch = tl.DecodeBatch(g, B, Hq)
    batch.prepare(ids, stream())
    q_out = empty_dev((B, Hq * D))
    batch.project(0, dx.data_ptr(), hidden, gs, dwk.data_ptr(), dsk.data_ptr(), dwv.data_ptr(),
                  dsv.data_ptr(), dwq.data_ptr(), dsq.data_ptr(), q_out.data_ptr(), stream(), packed=packed)
    kb, vb, qb = empty_dev((B, row)), empty_dev((B, row)), empty_dev((B, Hq * D))
    for w_, s_, out_, n_ in ((dwk, dsk, kb, row), (dwv, dsv, vb, row), (dwq, dsq, qb, Hq * D)):
        out_.zero_()
        tl.w8a16_matmul_residual(dx.data_ptr(), w_.data_ptr(), s_.data_ptr(), out_.data_ptr(), B, n_,
                                 hidden, gs, stream(), packed=packed)
    batch2 = tl.DecodeBatch(g2, B, Hq)
    batch2.prepare(ids2, stream())
    batch2.append(0, 1, kb.data_ptr(), vb.data_ptr(), stream())
    pool_elems = g.slot_bytes() // 2 * (B + 1)
    assert np.array_equal(read_dev(g.pool(), pool_elems), read_dev(g2.pool(), pool_elems))
    assert np.array_equal(to_host(q_out), to_host(qb))
    for got, (w, s, n) in ((kb, (wk, sk, row)), (vb, (wv, sv, row)), (qb, (wq, sq, Hq * D))):
        ref32, _ = orc.w8a16_matmul(x, w, s, B, n, hidden, gs)
        assert rows_close(to_host(got), ref32) <= TOL
