"""Pins the oracle's decode attention (restating kernels/attention.cu:11-112
over cache views).

Independent checks:
  * float64 textbook softmax(q K^T * scale) V in numpy, on dense K/V that the
    test holds itself (not read back through the oracle's addressing), for the
    compact, cache and paged views and GQA groups 1..8;
  * closed forms: S = 1, q = 0, identical keys, one dominant score;
  * invariances: permutation of positions, heads of one GQA group;
  * decode == last row of causal full attention (test_transformer.cu:222-300).
"""
import numpy as np
import pytest

RTOL = 2e-5  # fp32 accumulation vs float64, normwise


def f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def bits(x16):
    return np.ascontiguousarray(x16).view(np.uint16)


def ref64(q, K, V, scale, G):
    """q [Hq][D], K/V [Hkv][S][D] (float16 values) -> float64 [Hq][D]."""
    q = q.astype(np.float64)
    K = np.repeat(K.astype(np.float64), G, axis=0)
    V = np.repeat(V.astype(np.float64), G, axis=0)
    s = np.einsum("hd,hsd->hs", q, K) * scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return np.einsum("hs,hsd->hd", p, V) / (p.sum(axis=1, keepdims=True) + 1e-6)


def normwise(a, b):
    mx = max(np.abs(a).max(), np.abs(b).max())
    return np.abs(a - b).max() / mx if mx > 0 else 0.0


@pytest.mark.parametrize("B,Hkv,G,D,S", [(1, 2, 1, 32, 8), (2, 4, 1, 64, 100), (3, 2, 4, 128, 257),
                                         (2, 1, 8, 64, 33), (1, 3, 2, 256, 5)])
def test_compact_view_vs_float64(orc, B, Hkv, G, D, S):
    rng = np.random.default_rng(B * 1000 + S)
    Hq = Hkv * G
    q = f16(rng.standard_normal((B, Hq, D)))
    K = f16(rng.standard_normal((B, Hkv, S, D)))
    V = f16(rng.standard_normal((B, Hkv, S, D)))
    view = orc.compact_view(bits(K), bits(V), B, Hkv, S, D)
    scale = 1.0 / np.sqrt(D)
    o32, o16 = orc.attn_decode_gqa(bits(q), view, np.full(B, S), Hq, Hkv, D, scale)
    for b in range(B):
        r = ref64(q[b], K[b], V[b], scale, G)
        assert normwise(o32[b], r) < RTOL
        assert np.array_equal(o16[b], bits(f16(o32[b])))


def test_legacy_contract_equals_gqa_with_g1(orc):
    rng = np.random.default_rng(1)
    B, H, S, D = 2, 4, 19, 32
    q = bits(f16(rng.standard_normal((B, H, D))))
    k = bits(f16(rng.standard_normal((B, H, S, D))))
    v = bits(f16(rng.standard_normal((B, H, S, D))))
    a32, a16 = orc.attention_decode(q, k, v, 0.25, B, H, S, D)
    b32, b16 = orc.attn_decode_gqa(q, orc.compact_view(k, v, B, H, S, D), np.full(B, S), H, H, D, 0.25)
    assert np.array_equal(a32, b32) and np.array_equal(a16, b16)
    z32, _ = orc.attention_decode(q, k, v, 0.25, B, H, 0, D)  # non-positive dim: no-op
    assert not z32.any()


def _cache_with_data(orc, rng, L, Hkv, D, M, slots, ctx, layer, kv_std=1.0):
    """Fill a KVCacheOracle through appendKV; return it with the dense K/V."""
    c = orc.KVCacheOracle(L, Hkv, D, M, slots)
    ids, Ks, Vs = [], [], []
    # occupy slots out of order so slot != batch index
    dummy = [c.allocate(M)[0] for _ in range(slots)]
    for s in dummy[::2]:
        c.release(s)
    for S in ctx:
        sid, err = c.allocate(M)
        assert err is None
        K = f16(rng.standard_normal((S, Hkv, D)) * kv_std)
        V = f16(rng.standard_normal((S, Hkv, D)) * kv_std)
        for lay in range(L):
            kk, vv = (K, V) if lay == layer else (f16(-K), f16(-V))
            assert c.append(sid, lay, bits(kk), bits(vv), S) is None
        c.advance(sid, S)
        ids.append(sid)
        Ks.append(K.transpose(1, 0, 2))
        Vs.append(V.transpose(1, 0, 2))
    return c, ids, Ks, Vs


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_cache_view_vs_float64(orc, G):
    rng = np.random.default_rng(40 + G)
    L, Hkv, D, M = 3, 2, 64, 96
    ctx = [1, 17, 64, 95]
    c, ids, Ks, Vs = _cache_with_data(orc, rng, L, Hkv, D, M, 8, ctx, layer=1)
    slots = [c.slot_of(i) for i in ids]
    view = orc.cache_view(c.pool(), L, Hkv, D, M, 1, slots)
    Hq = Hkv * G
    q = f16(rng.standard_normal((len(ctx), Hq, D)))
    o32, _ = orc.attn_decode_gqa(bits(q), view, np.array(ctx), Hq, Hkv, D, 0.125)
    for b in range(len(ctx)):
        assert normwise(o32[b], ref64(q[b], Ks[b], Vs[b], 0.125, G)) < RTOL


def test_paged_view_vs_float64(orc):
    rng = np.random.default_rng(9)
    Hkv, D, M, slots, G = 2, 32, 64, 6, 4
    c = orc.KVCacheOracle(1, Hkv, D, M, slots)
    pool = c.pool()
    per_slot = M // 16
    perm = rng.permutation(slots * per_slot)
    # physical block ids in units of 16*Hkv*D from the layer base (K region of
    # each slot spans per_slot blocks, then its V region)
    phys = (perm // per_slot) * (2 * per_slot) + perm % per_slot
    ctx = [5, 16, 33, 64]
    B = len(ctx)
    table = np.zeros((B, per_slot), np.int32)
    Ks, Vs = [], []
    for b, S in enumerate(ctx):
        K = f16(rng.standard_normal((S, Hkv, D)))
        V = f16(rng.standard_normal((S, Hkv, D)))
        table[b] = phys[b * per_slot:(b + 1) * per_slot]
        for t in range(S):
            p = table[b, t // 16]
            off = p * 16 * Hkv * D + (t % 16) * Hkv * D
            pool[off:off + Hkv * D] = bits(K[t]).reshape(-1)
            pool[M * Hkv * D + off:M * Hkv * D + off + Hkv * D] = bits(V[t]).reshape(-1)
        Ks.append(K.transpose(1, 0, 2))
        Vs.append(V.transpose(1, 0, 2))
    view = orc.paged_view(pool, 1, Hkv, D, M, 0, table)
    Hq = Hkv * G
    q = f16(rng.standard_normal((B, Hq, D)))
    o32, _ = orc.attn_decode_gqa(bits(q), view, np.array(ctx), Hq, Hkv, D, 0.3)
    for b in range(B):
        assert normwise(o32[b], ref64(q[b], Ks[b], Vs[b], 0.3, G)) < RTOL


def _one(orc, q, K, V, scale=0.2):
    """Single entry, Hkv = 1, G = q.shape[0]."""
    S, D = K.shape
    view = orc.compact_view(bits(f16(K)[None]), bits(f16(V)[None]), 1, 1, S, D)
    o32, _ = orc.attn_decode_gqa(bits(f16(q))[None], view, np.array([S]), q.shape[0], 1, D, scale)
    return o32[0]


def test_closed_form_single_token(orc):
    rng = np.random.default_rng(2)
    v = f16(rng.standard_normal((1, 64)))
    o = _one(orc, rng.standard_normal((1, 64)), rng.standard_normal((1, 64)), v)
    assert np.allclose(o[0], v[0].astype(np.float64) / (1 + 1e-6), rtol=1e-6, atol=0)


def test_closed_form_zero_query_is_mean(orc):
    rng = np.random.default_rng(3)
    V = f16(rng.standard_normal((50, 32)))
    o = _one(orc, np.zeros((1, 32)), rng.standard_normal((50, 32)), V)
    assert normwise(o[0], V.astype(np.float64).mean(0)) < 1e-5


def test_closed_form_identical_keys_is_mean(orc):
    rng = np.random.default_rng(4)
    k = rng.standard_normal(32)
    V = f16(rng.standard_normal((40, 32)))
    o = _one(orc, rng.standard_normal((1, 32)), np.tile(k, (40, 1)), V)
    assert normwise(o[0], V.astype(np.float64).mean(0)) < 1e-5


def test_closed_form_dominant_score_selects_row(orc):
    rng = np.random.default_rng(5)
    K = rng.standard_normal((30, 32)) * 0.01
    K[17] = 4.0
    V = f16(rng.standard_normal((30, 32)))
    o = _one(orc, np.full((1, 32), 4.0), K, V, scale=1.0)
    assert normwise(o[0], V[17].astype(np.float64)) < 1e-6


def test_permutation_invariance(orc):
    rng = np.random.default_rng(6)
    K, V = rng.standard_normal((77, 64)), rng.standard_normal((77, 64))
    q = rng.standard_normal((2, 64))
    perm = rng.permutation(77)
    assert normwise(_one(orc, q, K, V), _one(orc, q, K[perm], V[perm])) < 1e-6


def test_gqa_heads_with_equal_queries_agree(orc):
    rng = np.random.default_rng(7)
    K, V = rng.standard_normal((60, 64)), rng.standard_normal((60, 64))
    q = np.tile(rng.standard_normal(64), (8, 1))
    o = _one(orc, q, K, V)
    assert all(np.array_equal(o[0], o[h]) for h in range(8))


@pytest.mark.parametrize("S", [4, 17, 32])
def test_decode_equals_last_row_of_causal_attention(orc, S):
    # Property 5 (test_transformer.cu:222-300): decode over the full cache
    # equals the last query row of causal full attention.
    rng = np.random.default_rng(S)
    D = 48
    Q = f16(rng.standard_normal((S, D)))
    K = f16(rng.standard_normal((S, D)))
    V = f16(rng.standard_normal((S, D)))
    scale = 1 / np.sqrt(D)
    s = (Q.astype(np.float64) @ K.astype(np.float64).T) * scale
    s[np.triu_indices(S, 1)] = -np.inf
    p = np.exp(s - s.max(1, keepdims=True))
    full = (p @ V.astype(np.float64)) / p.sum(1, keepdims=True)
    o = _one(orc, Q[-1:].astype(np.float64), K, V, scale=scale)
    assert normwise(o[0], full[-1]) < RTOL


def test_zero_length_gives_zero_row(orc):
    rng = np.random.default_rng(8)
    K = bits(f16(rng.standard_normal((2, 1, 8, 32))))
    view = orc.compact_view(K, K, 2, 1, 8, 32)
    q = bits(f16(rng.standard_normal((2, 1, 32))))
    o32, o16 = orc.attn_decode_gqa(q, view, np.array([0, 8]), 1, 1, 32, 0.1)
    assert not o32[0].any() and not o16[0].any() and o32[1].any()


def test_gather_matches_dense(orc):
    rng = np.random.default_rng(10)
    L, Hkv, D, M = 2, 3, 32, 48
    ctx = [3, 48, 20]
    c, ids, Ks, Vs = _cache_with_data(orc, rng, L, Hkv, D, M, 5, ctx, layer=0)
    view = orc.cache_view(c.pool(), L, Hkv, D, M, 0, [c.slot_of(i) for i in ids])
    smax = 50
    gk = orc.gather(view, 0, np.array(ctx), Hkv, D, smax)
    gv = orc.gather(view, 1, np.array(ctx), Hkv, D, smax)
    for b, S in enumerate(ctx):
        assert np.array_equal(gk[b, :, :S], bits(Ks[b])) and not gk[b, :, S:].any()
        assert np.array_equal(gv[b, :, :S], bits(Vs[b])) and not gv[b, :, S:].any()


@pytest.mark.parametrize("G,D,lens,paged", [
    (1, 32, [8, 1, 0, 13], False), (4, 128, [257, 64, 9, 1000], False),
    (8, 128, [1, 7, 300, 4100], True), (2, 64, [95, 0, 33], True), (1, 256, [40, 41], False),
    (4, 40, [21, 9], False)])
def test_fast_timing_form_is_bit_identical(orc, G, D, lens, paged):
    """orc_attn_decode_gqa_fast (the CPU baseline's vectorised form) gives the
    checker's bits on slot and paged views, ragged and empty lengths,
    lengths that are not multiples of its 8-token blocks, and a head_dim it
    does not vectorise (40: the fallback)."""
    rng = np.random.default_rng(G * 1000 + D + len(lens))
    Hkv, B = 2, len(lens)
    Hq = Hkv * G
    M = max(16, -(-max(lens) // 16) * 16)
    row = Hkv * D
    pool = bits(f16(rng.standard_normal(2 * B * M * row)))
    if paged:
        nblk = M // 16
        table = rng.permutation(B * nblk).astype(np.int32).reshape(B, nblk)
        view = orc.View(pool, 0, B * M * row, table, 4, 16 * row, row, D)
    else:
        view = orc.View(pool, 0, B * M * row, np.arange(B, dtype=np.int32).reshape(B, 1), 30,
                        M * row, row, D)
    q = bits(f16(rng.standard_normal((B, Hq, D)) * 2))
    a32, a16 = orc.attn_decode_gqa(q, view, np.array(lens), Hq, Hkv, D, D ** -0.5, nthreads=3)
    b32, b16 = orc.attn_decode_gqa(q, view, np.array(lens), Hq, Hkv, D, D ** -0.5, nthreads=3,
                                   fast=True)
    assert np.array_equal(a32.view(np.uint32), b32.view(np.uint32))
    assert np.array_equal(a16, b16)
