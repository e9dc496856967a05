"""Config-1 golden fixture (tests/golden/cfg1_decode.*, written by
tests/golden/make_cfg1.py).

CPU: the seeded inputs regenerate to the recorded digests; the oracle
reproduces the recorded cache pool and outputs bit for bit; and the recorded
fp32 output agrees with an independent float64 evaluation of
softmax(q K^T / 8) V (the math of kernels/attention.cu:11-112) -- so the
fixture does not merely restate the oracle.
GPU: one decode step through the HIP library (DecodeBatch.decode: fused
append + GQA attention) gives the recorded pool bytes exactly and the
recorded output within 1e-3 normwise per row."""
import hashlib
import json
import os

import numpy as np
import pytest

from golden.make_cfg1 import B, CTX, D, HKV, HQ, L, M, inputs, run_oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-3


@pytest.fixture(scope="module")
def fixture():
    with open(os.path.join(HERE, "cfg1_decode.json")) as f:
        meta = json.load(f)
    arr = dict(np.load(os.path.join(HERE, "cfg1_decode.npz")))
    return meta, arr


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_inputs_regenerate(orc, fixture):
    meta, arr = fixture
    q, k, v = inputs(orc)
    assert sha(q) == meta["sha256"]["q"]
    assert sha(k) == meta["sha256"]["k_stream"]
    assert sha(v) == meta["sha256"]["v_stream"]
    off = sum(CTX)
    assert np.array_equal(arr["q"], q)
    assert np.array_equal(arr["new_k"], k[off:]) and np.array_equal(arr["new_v"], v[off:])


def test_oracle_reproduces_fixture(orc, fixture):
    meta, arr = fixture
    pool, lens, o32, o16 = run_oracle(orc, *inputs(orc))
    assert sha(pool) == meta["sha256"]["pool_after_step"]
    assert np.array_equal(lens, arr["lens"])
    assert np.array_equal(o32, arr["out_f32"])
    assert np.array_equal(o16, arr["out_f16"])


def test_fixture_matches_float64_math(orc, fixture):
    _, arr = fixture
    q, k, v = inputs(orc)
    f = lambda x: x.view(np.float16).astype(np.float64)
    qf, kf, vf = f(q), f(k).reshape(-1, HKV, D), f(v).reshape(-1, HKV, D)
    off, new = 0, sum(CTX)
    for b, c in enumerate(CTX):
        K = np.concatenate([kf[off:off + c], kf[new + b:new + b + 1]])  # [S][H][D]
        V = np.concatenate([vf[off:off + c], vf[new + b:new + b + 1]])
        off += c
        for h in range(HQ):
            s = K[:, h, :] @ qf[b, h] * 0.125
            p = np.exp(s - s.max())
            o = (p @ V[:, h, :]) / p.sum()
            got = arr["out_f32"][b, h].astype(np.float64)
            assert np.abs(got - o).max() / np.abs(o).max() < 2e-5, (b, h)


@pytest.mark.gpu
def test_gpu_decode_step_matches_fixture(tl, orc, fixture):
    from devutil import empty_dev, read_dev, rel_err, stream, to_dev, to_host
    meta, arr = fixture
    q, k, v = inputs(orc)
    g = tl.KVCacheManager(L, HKV, D, M, B)
    ids, keep, off = [], [], 0
    for c in CTX:
        sid, err = g.allocateSequence(M)
        assert err is None, err
        dk, dv = to_dev(k[off:off + c]), to_dev(v[off:off + c])
        keep += [dk, dv]
        assert g.appendKV(sid, 0, dk.data_ptr(), dv.data_ptr(), c, stream()) is None
        g.advanceSeqLen(sid, c)
        off += c
        ids.append(sid)
    batch = tl.DecodeBatch(g, B, HQ)
    batch.prepare(ids, stream())
    dq, dnk, dnv = to_dev(arr["q"]), to_dev(arr["new_k"]), to_dev(arr["new_v"])
    out = empty_dev((B, HQ, D))
    batch.decode(0, dq.data_ptr(), dnk.data_ptr(), dnv.data_ptr(), out.data_ptr(), meta["scale"],
                 stream())
    pool = read_dev(g.pool(), B * g.slot_bytes() // 2)
    assert sha(pool) == meta["sha256"]["pool_after_step"]
    got = to_host(out).view(np.float16).astype(np.float32)
    errs = [rel_err(got[b, h], arr["out_f32"][b, h]) for b in range(B) for h in range(HQ)]
    assert max(errs) <= TOL, max(errs)
