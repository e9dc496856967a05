"""ctypes binding of the CPU oracle (oracle/kv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, where it is the checker.  The product
(tiny-llm_amd/) never imports it.

All fp16 data crosses as numpy uint16 arrays holding binary16 bit patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libkv_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, no GPU); make rebuilds it
    when a source is newer than the library."""
    if force and os.path.exists(_LIB_PATH):
        os.remove(_LIB_PATH)
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def use_native_build() -> str:
    """The CPU baseline's timing build: compile kv_oracle.c with -O3
    -march=native on this machine (make native) and route every later call of
    this module through it.  Returns a description of the build used; falls
    back to the portable build when the compile fails."""
    global _lib
    path = os.path.join(_HERE, "_build", "libkv_oracle_native.so")
    if os.path.exists(path):
        os.remove(path)  # -march=native belongs to the machine it runs on
    try:
        subprocess.run(["make", "-s", "-C", _HERE, "native"], check=True, capture_output=True,
                       timeout=300)
        native = C.CDLL(path)
    except (subprocess.SubprocessError, OSError) as e:
        lib()
        return f"portable build (-O3 -march=x86-64-v3; native build failed: {e})"
    _declare(native)
    _lib = native
    return "gcc -O3 -march=native -fopenmp, built on this host"


class _Config(C.Structure):
    _fields_ = [("num_layers", C.c_int), ("num_heads", C.c_int), ("head_dim", C.c_int),
                ("max_seq_len", C.c_int), ("max_batch_size", C.c_int)]


class _View(C.Structure):
    _fields_ = [("k_base", C.c_void_p), ("v_base", C.c_void_p), ("block_table", C.c_void_p),
                ("bt_stride", C.c_int), ("log2_blk", C.c_int), ("blk_stride", C.c_int64),
                ("tok_stride", C.c_int64), ("head_stride", C.c_int64)]


def _declare(L: C.CDLL) -> None:
    vp, i, sz, cp = C.c_void_p, C.c_int, C.c_size_t, C.c_char_p
    L.orc_h2f.restype, L.orc_h2f.argtypes = C.c_float, [C.c_uint16]
    L.orc_f2h.restype, L.orc_f2h.argtypes = C.c_uint16, [C.c_float]
    L.orc_h2f_n.argtypes = [vp, vp, sz]
    L.orc_f2h_n.argtypes = [vp, vp, sz]
    L.orc_fill_normal_f16.argtypes = [C.c_uint64, C.c_float, vp, sz]
    L.orc_kv_create.restype, L.orc_kv_create.argtypes = i, [C.POINTER(_Config), C.POINTER(vp), cp, i]
    L.orc_kv_destroy.argtypes = [vp]
    L.orc_kv_allocate.restype, L.orc_kv_allocate.argtypes = i, [vp, i, C.POINTER(i), cp, i]
    L.orc_kv_release.restype, L.orc_kv_release.argtypes = i, [vp, i, cp, i]
    L.orc_kv_get_cache.restype = i
    L.orc_kv_get_cache.argtypes = [vp, i, i, C.POINTER(sz), C.POINTER(sz), cp, i]
    L.orc_kv_append.restype, L.orc_kv_append.argtypes = i, [vp, i, i, vp, vp, i, cp, i]
    L.orc_kv_advance.restype, L.orc_kv_advance.argtypes = i, [vp, i, i, cp, i]
    for name in ("orc_kv_seq_len", "orc_kv_has", "orc_kv_slot_of"):
        getattr(L, name).restype, getattr(L, name).argtypes = i, [vp, i]
    for name in ("orc_kv_used", "orc_kv_total", "orc_kv_free", "orc_kv_slot_bytes",
                 "orc_kv_pool_elems"):
        getattr(L, name).restype, getattr(L, name).argtypes = sz, [vp]
    L.orc_kv_active.restype, L.orc_kv_active.argtypes = i, [vp]
    L.orc_kv_pool.restype, L.orc_kv_pool.argtypes = vp, [vp]
    L.orc_attn_decode_gqa.argtypes = [vp, C.POINTER(_View), vp, i, i, i, i, C.c_float, vp, vp, i]
    L.orc_attn_decode_gqa_fast.argtypes = L.orc_attn_decode_gqa.argtypes
    L.orc_attention_decode.argtypes = [vp, vp, vp, vp, vp, C.c_float, i, i, i, i]
    L.orc_kv_gather.argtypes = [C.POINTER(_View), i, vp, i, i, i, i, vp]
    L.orc_attention_prefill.argtypes = [vp, vp, vp, vp, vp, C.c_float, i, i, i, i, i]
    L.orc_attention_prefill.restype = None
    L.orc_softmax.argtypes = [vp, vp, vp, i, i]
    L.orc_softmax.restype = None
    L.orc_get_attention_weights.argtypes = [vp, vp, vp, vp, C.c_float, i, i, i, i, i, i]
    L.orc_get_attention_weights.restype = None
    L.orc_w8a16_matmul.argtypes = [vp, vp, vp, vp, vp, i, i, i, i]
    L.orc_w8a16_matmul.restype = None
    L.orc_add_inplace.argtypes = [vp, vp, C.c_size_t]
    L.orc_add_inplace.restype = None


def _ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------- fp16 helpers
def h2f(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().orc_h2f_n(_ptr(bits), _ptr(out), bits.size)
    return out


def f2h(vals: np.ndarray) -> np.ndarray:
    vals = np.ascontiguousarray(vals, dtype=np.float32)
    out = np.empty(vals.shape, dtype=np.uint16)
    lib().orc_f2h_n(_ptr(vals), _ptr(out), vals.size)
    return out


def normal_f16(seed: int, shape, stddev: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().orc_fill_normal_f16(C.c_uint64(seed), stddev, _ptr(out), out.size)
    return out


# ----------------------------------------------------------------- KV manager
class OracleError(RuntimeError):
    pass


class KVCacheOracle:
    """Host-memory restatement of tiny_llm::KVCacheManager (kv_cache.cpp)."""

    def __init__(self, num_layers, num_heads, head_dim, max_seq_len, max_batch_size):
        self.cfg = _Config(num_layers, num_heads, head_dim, max_seq_len, max_batch_size)
        self._h = C.c_void_p()
        err = C.create_string_buffer(512)
        if lib().orc_kv_create(C.byref(self.cfg), C.byref(self._h), err, 512) != 0:
            raise OracleError(err.value.decode())

    @classmethod
    def try_create(cls, *args):
        try:
            return cls(*args), None
        except OracleError as e:
            return None, str(e)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_kv_destroy(self._h)
            self._h = None

    def _call(self, fn, *args):
        err = C.create_string_buffer(512)
        rc = fn(self._h, *args, err, 512)
        return rc, err.value.decode()

    def allocate(self, max_len):
        out = C.c_int(-1)
        rc, msg = self._call(lib().orc_kv_allocate, max_len, C.byref(out))
        return (out.value, None) if rc == 0 else (None, msg)

    def release(self, seq_id):
        rc, msg = self._call(lib().orc_kv_release, seq_id)
        return None if rc == 0 else msg

    def get_cache(self, seq_id, layer):
        k, v = C.c_size_t(), C.c_size_t()
        rc, msg = self._call(lib().orc_kv_get_cache, seq_id, layer, C.byref(k), C.byref(v))
        return ((k.value, v.value), None) if rc == 0 else (None, msg)

    def append(self, seq_id, layer, new_k, new_v, num_tokens):
        nk = None if new_k is None else np.ascontiguousarray(new_k, dtype=np.uint16)
        nv = None if new_v is None else np.ascontiguousarray(new_v, dtype=np.uint16)
        rc, msg = self._call(lib().orc_kv_append, seq_id, layer, _ptr(nk), _ptr(nv), num_tokens)
        return None if rc == 0 else msg

    def advance(self, seq_id, n):
        rc, msg = self._call(lib().orc_kv_advance, seq_id, n)
        return None if rc == 0 else msg

    def seq_len(self, seq_id):
        return lib().orc_kv_seq_len(self._h, seq_id)

    def has(self, seq_id):
        return bool(lib().orc_kv_has(self._h, seq_id))

    def slot_of(self, seq_id):
        return lib().orc_kv_slot_of(self._h, seq_id)

    def used(self):
        return lib().orc_kv_used(self._h)

    def total(self):
        return lib().orc_kv_total(self._h)

    def free(self):
        return lib().orc_kv_free(self._h)

    def active(self):
        return lib().orc_kv_active(self._h)

    def slot_bytes(self):
        return lib().orc_kv_slot_bytes(self._h)

    def pool(self) -> np.ndarray:
        """Live numpy view of the host pool (uint16)."""
        n = lib().orc_kv_pool_elems(self._h)
        addr = lib().orc_kv_pool(self._h)
        return np.ctypeslib.as_array(C.cast(addr, C.POINTER(C.c_uint16)), shape=(n,))


# -------------------------------------------------------------- views / math
@dataclass
class View:
    """Addressing of (sequence b, kv head g, token t) -> element offset.

    elem = blk(b, t >> log2_blk) * blk_stride + (t & mask) * tok_stride + g * head_stride
    blk(b, j) = block_table[b, j] if block_table is not None else b.
    k_off / v_off are element offsets of the K and V bases inside `pool`.
    """
    pool: np.ndarray
    k_off: int
    v_off: int
    block_table: np.ndarray | None
    log2_blk: int
    blk_stride: int
    tok_stride: int
    head_stride: int

    def c_view(self) -> _View:
        base = self.pool.ctypes.data
        bt = None
        if self.block_table is not None:
            self._bt = np.ascontiguousarray(self.block_table, dtype=np.int32)
            bt = self._bt.ctypes.data
        stride = 0 if self.block_table is None else self._bt.shape[1]
        return _View(base + 2 * self.k_off, base + 2 * self.v_off, bt, stride, self.log2_blk,
                     self.blk_stride, self.tok_stride, self.head_stride)


def cache_view(pool, num_layers, hkv, d, max_seq_len, layer, slots):
    """The reference pool layout (kv_cache.cpp:69-80, 226-233) as a view whose
    block table holds the slot index of each batch entry."""
    kv_per_layer = hkv * max_seq_len * d
    bt = np.asarray(slots, dtype=np.int32).reshape(-1, 1)
    return View(pool, layer * 2 * kv_per_layer, layer * 2 * kv_per_layer + kv_per_layer, bt, 30,
                2 * num_layers * kv_per_layer, hkv * d, d)


def paged_view(pool, num_layers, hkv, d, max_seq_len, layer, block_table, log2_blk=4):
    """16-token paged view over the same pool: physical block p of a layer's K
    region starts at element layer*2*M*Hkv*D + p*16*Hkv*D; V is M*Hkv*D later."""
    kv_per_layer = hkv * max_seq_len * d
    return View(pool, layer * 2 * kv_per_layer, layer * 2 * kv_per_layer + kv_per_layer,
                np.asarray(block_table, dtype=np.int32), log2_blk, (1 << log2_blk) * hkv * d,
                hkv * d, d)


def compact_view(k, v, B, H, S, D):
    """attention.cu:12-14 layout: [B][H][S][D] for K and V (separate arrays
    concatenated into one pool so the view has a single base)."""
    pool = np.concatenate([np.ascontiguousarray(k).reshape(-1), np.ascontiguousarray(v).reshape(-1)])
    return View(pool, 0, k.size, None, 30, H * S * D, D, S * D)


def attn_decode_gqa(q, view: View, seq_lens, Hq, Hkv, D, scale, nthreads=1, fast=False):
    """Returns (out_f32, out_f16_bits), each [B][Hq][D].  fast: the
    vectorised timing form (orc_attn_decode_gqa_fast, the same bits)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    B = lens.shape[0]
    o32 = np.zeros((B, Hq, D), dtype=np.float32)
    o16 = np.zeros((B, Hq, D), dtype=np.uint16)
    cv = view.c_view()
    fn = lib().orc_attn_decode_gqa_fast if fast else lib().orc_attn_decode_gqa
    fn(_ptr(q), C.byref(cv), _ptr(lens), B, Hq, Hkv, D, scale, _ptr(o32), _ptr(o16), nthreads)
    return o32, o16


def attention_decode(q, k, v, scale, B, H, S, D):
    """Literal attention_decode contract (compact layout, MHA)."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, k, v))
    o32 = np.zeros((B, H, D), dtype=np.float32)
    o16 = np.zeros((B, H, D), dtype=np.uint16)
    lib().orc_attention_decode(_ptr(q), _ptr(k), _ptr(v), _ptr(o32), _ptr(o16), scale, B, H, S, D)
    return o32, o16


def attention_prefill(q, k, v, scale, B, H, S, D, nthreads=1):
    """Literal attention_prefill contract: compact [B][H][S][D], causal, MHA.
    Returns (out_f32, out_f16 bits), each [B][H][S][D]."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, k, v))
    o32 = np.zeros((B, H, S, D), dtype=np.float32)
    o16 = np.zeros((B, H, S, D), dtype=np.uint16)
    lib().orc_attention_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(o32), _ptr(o16), scale, B, H, S, D,
                                nthreads)
    return o32, o16


def softmax(x, rows, S):
    """softmax over rows of S fp16 bit patterns -> (f32, f16 bits)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    o32 = np.zeros((rows, S), dtype=np.float32)
    o16 = np.zeros((rows, S), dtype=np.uint16)
    lib().orc_softmax(_ptr(x), _ptr(o32), _ptr(o16), rows, S)
    return o32, o16


def get_attention_weights(q, k, scale, B, H, Lq, Lk, D, causal):
    """Scaled scores [B][H][Lq][Lk] (no softmax), zero above the diagonal when
    causal -> (f32, f16 bits)."""
    q, k = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, k))
    o32 = np.zeros((B, H, Lq, Lk), dtype=np.float32)
    o16 = np.zeros((B, H, Lq, Lk), dtype=np.uint16)
    lib().orc_get_attention_weights(_ptr(q), _ptr(k), _ptr(o32), _ptr(o16), scale, B, H, Lq, Lk, D,
                                    int(causal))
    return o32, o16


def gather(view: View, which, seq_lens, Hkv, D, S_max):
    lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    B = lens.shape[0]
    out = np.empty((B, Hkv, S_max, D), dtype=np.uint16)
    cv = view.c_view()
    lib().orc_kv_gather(C.byref(cv), which, _ptr(lens), B, Hkv, D, S_max, _ptr(out))
    return out


def w8a16_matmul(x, w, s, M, N, K, group_size):
    """Reference-order W8A16 product: x [M][K] fp16 bits, w [K][N] int8,
    s [ceil(K/gs)][N] fp16 bits -> (out_f32 [M][N], out_f16 bits [M][N])."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    o32 = np.zeros((M, N), dtype=np.float32)
    o16 = np.zeros((M, N), dtype=np.uint16)
    lib().orc_w8a16_matmul(_ptr(x), _ptr(w), _ptr(s), _ptr(o32), _ptr(o16), M, N, K, group_size)
    return o32, o16


def add_inplace(data, add):
    """data (fp16 bits, modified in place) += add, rounded like add_inplace."""
    a = np.ascontiguousarray(add, dtype=np.uint16)
    assert data.flags.c_contiguous and data.dtype == np.uint16 and data.size == a.size
    lib().orc_add_inplace(_ptr(data), _ptr(a), data.size)
    return data

