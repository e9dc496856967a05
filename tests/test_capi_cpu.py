"""CPU: the C-ABI library loads, exports every symbol include/tinyllm_kv.h
declares, and rejects bad arguments before touching a GPU."""
import ctypes as C

import numpy as np
import pytest


@pytest.fixture(scope="module")
def tlc():
    import tinyllm_kv
    tinyllm_kv.load()
    return tinyllm_kv


def _has_gpu():
    try:
        import torch
        return torch.cuda.device_count() > 0
    except Exception:
        return False


def test_exports_every_declared_symbol(tlc):
    lib = tlc.load()
    syms = tlc.header_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_version_names_gfx950(tlc):
    assert "gfx950" in tlc.load().tl_version().decode()


def test_invalid_config_rejected_before_device_work(tlc):
    obj, err = tlc.KVCacheManager.create(num_layers=2, num_heads=0, head_dim=64, max_seq_len=16,
                                         max_batch_size=1)
    assert obj is None and err == "KVCacheManager: invalid configuration parameters"


@pytest.mark.skipif(_has_gpu(), reason="checks the no-GPU failure path")
def test_create_without_gpu_fails_loudly(tlc):
    obj, err = tlc.KVCacheManager.create(num_layers=1, num_heads=1, head_dim=64, max_seq_len=16,
                                         max_batch_size=1)
    assert obj is None and err.startswith("KVCacheManager: hip")


def test_gqa_argument_validation(tlc):
    v = tlc.KVView(16, 16, None, 0, 30, 1024, 128, 128)
    lens = np.array([4], np.int32)
    lib = tlc.load()
    rc = lib.tl_attn_decode_gqa(16, C.byref(v), lens.ctypes.data, 1, 6, 4, 128, 1.0, 16, None)
    assert rc == tlc.TL_ERR_INVALID and "multiple" in tlc.last_error()
    rc = lib.tl_attn_decode_gqa(16, C.byref(v), lens.ctypes.data, 1, 4, 4, 96, 1.0, 16, None)
    assert rc == tlc.TL_ERR_INVALID and "unsupported" in tlc.last_error()
    rc = lib.tl_attn_decode_gqa(16, C.byref(v), lens.ctypes.data, 1, 64, 4, 128, 1.0, 16, None)
    assert rc == tlc.TL_ERR_INVALID  # group 16 is not instantiated
    bad = np.array([-1], np.int32)
    rc = lib.tl_attn_decode_gqa(16, C.byref(v), bad.ctypes.data, 1, 4, 4, 128, 1.0, 16, None)
    assert rc == tlc.TL_ERR_INVALID and "negative" in tlc.last_error()
    rc = lib.tl_attn_decode_gqa(18, C.byref(v), lens.ctypes.data, 1, 4, 4, 128, 1.0, 16, None)
    assert rc == tlc.TL_ERR_INVALID and "aligned" in tlc.last_error()


def test_null_handles_are_rejected(tlc):
    lib = tlc.load()
    assert lib.tl_kv_release_sequence(None, 0) == tlc.TL_ERR_INVALID
    assert lib.tl_kv_seq_len(None, 0) == 0
    assert lib.tl_kv_batch_prepare(None, None, 0, None) == tlc.TL_ERR_INVALID
    assert lib.tl_profile_query(b"nope", C.byref(C.c_double()), C.byref(C.c_longlong())) \
        == tlc.TL_ERR_INVALID


def test_destructors_survive_interpreter_shutdown(tlc, monkeypatch):
    """At interpreter shutdown module globals (load() among them) may already
    be None when a manager or batch is collected: the destructors use the
    handle taken at construction, so they still release the object and raise
    nothing."""
    freed = []
    monkeypatch.setattr(tlc, "load", None)
    for cls in (tlc.KVCacheManager, tlc.DecodeBatch, tlc.PrefillBatch):
        obj = object.__new__(cls)
        obj._h = C.c_void_p(0x1000 + len(freed))
        obj._destroy = lambda h, name=cls.__name__: freed.append((name, h.value))
        obj.__del__()
        obj.__del__()  # a second close is a no-op
        assert obj._h is None
    assert [n for n, _ in freed] == ["KVCacheManager", "DecodeBatch", "PrefillBatch"]
