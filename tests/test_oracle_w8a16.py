"""Pins the oracle's W8A16 product (orc_w8a16_matmul, restating
kernels/w8a16_matmul.cu:71-98) and add_inplace (kernels/elementwise.cu:7-14)
with checks that do not restate the formula: a float64 product of the
dequantized weights, closed forms that fix the group indexing, exact scaling,
and the reference's own test shapes with its 1% bound against an fp16 matmul
of dequantized weights (tests/test_w8a16_matmul.cu:94-222, 247-342)."""
import numpy as np
import pytest

SHAPES = [  # (M, N, K, group_size): the reference's test shapes first
    (4, 8, 16, 8), (1, 64, 128, 32), (64, 1, 128, 32), (17, 33, 65, 32),
    (13, 40, 300, 64), (5, 48, 256, 128),
]


def operands(orc, rng, M, N, K, gs):
    x = orc.f2h(rng.standard_normal((M, K)).astype(np.float32))
    w = rng.integers(-128, 128, size=(K, N), dtype=np.int64).astype(np.int8)
    s = orc.f2h((np.abs(rng.standard_normal(((K + gs - 1) // gs, N))) * 0.02 + 1e-3).astype(np.float32))
    return x, w, s


def dequant64(orc, w, s, gs):
    K = w.shape[0]
    sc = orc.h2f(s).astype(np.float64)[np.arange(K) // gs]
    return w.astype(np.float64) * sc


@pytest.mark.parametrize("M,N,K,gs", SHAPES)
def test_matches_float64_product(orc, M, N, K, gs):
    rng = np.random.default_rng(M * 1000 + N * 10 + K)
    x, w, s = operands(orc, rng, M, N, K, gs)
    o32, o16 = orc.w8a16_matmul(x, w, s, M, N, K, gs)
    ref = orc.h2f(x).astype(np.float64) @ dequant64(orc, w, s, gs)
    assert np.abs(o32 - ref).max() <= 1e-5 * np.abs(ref).max()
    assert np.array_equal(o16, orc.f2h(o32))


def test_identity_weights_return_x(orc):
    rng = np.random.default_rng(1)
    K = 64
    x = orc.f2h(rng.standard_normal((3, K)).astype(np.float32))
    w = np.eye(K, dtype=np.int8)
    s = orc.f2h(np.ones((2, K), np.float32))
    _, o16 = orc.w8a16_matmul(x, w, s, 3, K, K, 32)
    assert np.array_equal(o16, x)


def test_group_index_closed_form(orc):
    """x = 1, w = 1, s[g][n] = g + 1: out = sum_g (g + 1) * |group g|, with a
    partial last group (K = 100, gs = 32: groups of 32, 32, 32, 4)."""
    M, N, K, gs = 2, 5, 100, 32
    x = orc.f2h(np.ones((M, K), np.float32))
    w = np.ones((K, N), np.int8)
    s = orc.f2h(np.repeat(np.arange(1, 5, dtype=np.float32)[:, None], N, axis=1))
    o32, _ = orc.w8a16_matmul(x, w, s, M, N, K, gs)
    assert np.all(o32 == 1 * 32 + 2 * 32 + 3 * 32 + 4 * 4)


def test_doubled_scales_double_exactly(orc):
    rng = np.random.default_rng(2)
    M, N, K, gs = 6, 24, 192, 64
    x, w, s = operands(orc, rng, M, N, K, gs)
    s2 = orc.f2h(orc.h2f(s) * 2.0)
    a, _ = orc.w8a16_matmul(x, w, s, M, N, K, gs)
    b, _ = orc.w8a16_matmul(x, w, s2, M, N, K, gs)
    assert np.array_equal(b, a * 2.0)


@pytest.mark.parametrize("M,N,K,gs", SHAPES)
def test_reference_bound_vs_fp16_dequantized_matmul(orc, M, N, K, gs):
    """The reference tests' check: w8a16 vs fp16_matmul_reference over
    dequantize_weights (fp16(w * s)), computeRelativeError < 1%."""
    rng = np.random.default_rng(K * 7 + gs)
    x, w, s = operands(orc, rng, M, N, K, gs)
    _, o16 = orc.w8a16_matmul(x, w, s, M, N, K, gs)
    w16 = orc.h2f(orc.f2h((w.astype(np.float32) * orc.h2f(s)[np.arange(K) // gs]).astype(np.float32)))
    ref = orc.h2f(x).astype(np.float64) @ w16.astype(np.float64)
    ref16 = orc.h2f(orc.f2h(ref.astype(np.float32)))
    got = orc.h2f(o16)
    rel = np.abs(got - ref16).max() / max(np.abs(got).max(), np.abs(ref16).max())
    assert rel < 0.01


def test_nonpositive_dims_are_noop(orc):
    x = np.zeros((1, 32), np.uint16)
    w = np.zeros((32, 16), np.int8)
    s = np.zeros((1, 16), np.uint16)
    o32 = np.full((1, 16), 7.0, np.float32)
    o16 = np.full((1, 16), 7, np.uint16)
    orc.lib().orc_w8a16_matmul(x.ctypes.data, w.ctypes.data, s.ctypes.data, o32.ctypes.data,
                               o16.ctypes.data, 0, 16, 32, 32)
    assert np.all(o16 == 7) and np.all(o32 == 7.0)


def test_add_inplace_rounding(orc):
    data = orc.f2h(np.array([1.0, 5.0, 2048.0, 2050.0, -3.0], np.float32))
    add = orc.f2h(np.array([2.0, 0.0, 1.0, 1.0, 3.0], np.float32))
    orc.add_inplace(data, add)
    # 2048 + 1 ties between 2048 and 2050 -> even mantissa 2048; 2050 + 1 -> 2052
    assert list(orc.h2f(data)) == [3.0, 5.0, 2048.0, 2052.0, 0.0]
