"""Pins the oracle's prefill attention, softmax and attention weights
(restating kernels/attention.cu:131-354).

Independent checks:
  * prefill row i == the pinned decode oracle over the first i + 1 keys, bit
    for bit: the reference's masked keys contribute exact zeros
    (test_transformer.cu:222-300 asks the last row to match within 5%);
  * float64 causal softmax(Q K^T * scale) V by numpy;
  * closed form: row 0 attends to key 0 alone, out = v_0 / (1 + 1e-6);
  * softmax: float64 by numpy, rows sum to 1, order kept
    (test_kernels.cu:505-530, :664-740);
  * attention weights: float64 scale * q.k within one fp16 rounding, exact
    zeros above the diagonal (test_kernels.cu:558-662).
"""
import numpy as np
import pytest


def f16bits(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32).astype(np.float16).view(np.uint16)


def h(bits):
    return bits.view(np.float16).astype(np.float64)


@pytest.mark.parametrize("B,H,S,D", [(1, 2, 8, 32), (2, 3, 17, 64), (1, 1, 40, 128)])
def test_prefill_rows_equal_decode_over_prefix(orc, B, H, S, D):
    rng = np.random.default_rng(S * D + H)
    q, k, v = (f16bits(rng, (B, H, S, D)) for _ in range(3))
    scale = 1.0 / np.sqrt(D)
    o32, o16 = orc.attention_prefill(q, k, v, scale, B, H, S, D)
    for i in range(S):
        d32, d16 = orc.attention_decode(np.ascontiguousarray(q[:, :, i]),
                                        np.ascontiguousarray(k[:, :, :i + 1]),
                                        np.ascontiguousarray(v[:, :, :i + 1]), scale, B, H, i + 1, D)
        assert np.array_equal(o32[:, :, i], d32), i
        assert np.array_equal(o16[:, :, i], d16), i


@pytest.mark.parametrize("B,H,S,D", [(1, 2, 8, 32), (2, 2, 33, 64)])
def test_prefill_matches_float64_causal_attention(orc, B, H, S, D):
    rng = np.random.default_rng(7 + S)
    q, k, v = (f16bits(rng, (B, H, S, D)) for _ in range(3))
    scale = 1.0 / np.sqrt(D)
    o32, _ = orc.attention_prefill(q, k, v, scale, B, H, S, D)
    s = np.einsum("bhid,bhpd->bhip", h(q), h(k)) * scale
    s[:, :, np.triu_indices(S, 1)[0], np.triu_indices(S, 1)[1]] = -np.inf
    s -= s.max(axis=3, keepdims=True)
    p = np.exp(s)
    ref = np.einsum("bhip,bhpd->bhid", p, h(v)) / (p.sum(axis=3, keepdims=True) + 1e-6)
    err = np.abs(o32 - ref).max() / np.abs(ref).max()
    assert err < 2e-5, err


def test_prefill_first_row_is_first_value(orc):
    rng = np.random.default_rng(3)
    B, H, S, D = 2, 2, 5, 32
    q, k, v = (f16bits(rng, (B, H, S, D)) for _ in range(3))
    o32, _ = orc.attention_prefill(q, k, v, 0.125, B, H, S, D)
    expect = h(v)[:, :, 0] * np.float32(1.0 / (1.0 + 1e-6))
    assert np.abs(o32[:, :, 0] - expect).max() <= 2e-7 * np.abs(expect).max()


def test_prefill_nonpositive_dims_are_noop(orc):
    z = np.zeros(64, np.uint16)
    o32 = np.full(64, 5.0, np.float32)
    o16 = np.full(64, 9, np.uint16)
    orc.lib().orc_attention_prefill(z.ctypes.data, z.ctypes.data, z.ctypes.data, o32.ctypes.data,
                                    o16.ctypes.data, 1.0, 0, 1, 8, 8, 1)
    assert np.all(o16 == 9) and np.all(o32 == 5.0)


@pytest.mark.parametrize("rows,S", [(4, 16), (3, 100), (1, 1)])
def test_softmax_float64_sum_and_order(orc, rows, S):
    rng = np.random.default_rng(rows * S)
    x = f16bits(rng, (rows, S), 2.0)
    o32, o16 = orc.softmax(x, rows, S)
    xf = h(x)
    e = np.exp(xf - xf.max(axis=1, keepdims=True))
    ref = e / (e.sum(axis=1, keepdims=True) + 1e-6)
    assert np.abs(o32 - ref).max() < 1e-6
    assert np.array_equal(o16, o32.astype(np.float16).view(np.uint16))
    sums = h(o16).sum(axis=1)
    assert np.all((sums > 0.98) & (sums < 1.02))
    for r in range(rows):
        hi = xf[r][:, None] > xf[r][None, :] + 0.1
        assert np.all(h(o16)[r][:, None][hi.any(axis=1)] >= 0)
        ii, jj = np.nonzero(hi)
        assert np.all(h(o16)[r][ii] >= h(o16)[r][jj])


@pytest.mark.parametrize("causal", [True, False])
def test_attention_weights_float64_and_mask(orc, causal):
    rng = np.random.default_rng(11)
    B, H, Lq, Lk, D = 2, 3, 9, 12, 48
    q = f16bits(rng, (B, H, Lq, D))
    k = f16bits(rng, (B, H, Lk, D))
    scale = 1.0 / np.sqrt(D)
    o32, o16 = orc.get_attention_weights(q, k, scale, B, H, Lq, Lk, D, causal)
    ref = np.einsum("bhid,bhpd->bhip", h(q), h(k)) * scale
    mask = np.triu(np.ones((Lq, Lk), bool), 1)
    if causal:
        ref[:, :, mask] = 0.0
        assert np.all(o16[:, :, mask] == 0)
    assert np.abs(o32 - ref).max() <= 1e-5 * np.abs(ref).max()
    got = h(o16)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 2.0 ** -24 + 1e-5 * np.abs(ref).max())
