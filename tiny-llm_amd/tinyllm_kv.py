"""ctypes binding of libtinyllm_kv.so (the C ABI of include/tinyllm_kv.h).

This is the host-side mirror used by tests/, bench.py and __graft_entry__:
the same names and argument meaning as the reference's KVCacheManager
(include/tiny_llm/kv_cache.h) and attention_decode (kernels/attention.cuh),
plus the batched decode surface.  Device memory is passed as integer device
addresses (e.g. torch tensor .data_ptr()); streams as integer hipStream_t
handles (0 = default stream).

There is no fallback: if the library is missing, load() raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
_REPO = os.path.dirname(_HERE)
# Always the in-tree build: no environment override, so a test, the smoke
# check or the bench can never pick up some other copy of the library.
LIB_PATH = os.path.join(_HERE, "_build", "libtinyllm_kv.so")
HEADER_PATH = os.path.join(_REPO, "include", "tinyllm_kv.h")

TL_OK = 0
TL_ERR_INVALID = -1
TL_ERR_HIP = -2

_lib = None


class TinyLLMError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code
        self.msg = msg


def build(jobs: int = 8) -> str:
    """Compile the HIP library for gfx950 (always runs make; make skips
    up-to-date objects)."""
    subprocess.run(["make", "-s", "-C", _HERE, f"-j{jobs}"], check=True)
    return LIB_PATH


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if os.environ.get("TINYLLM_KV_LIB"):
            raise RuntimeError("TINYLLM_KV_LIB is set; this binding loads only the in-tree "
                               f"library {LIB_PATH}")
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (or make -C tiny-llm_amd)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
        mapped = loaded_path()
        if mapped is None or os.path.realpath(mapped) != os.path.realpath(LIB_PATH):
            raise RuntimeError(f"libtinyllm_kv.so mapped from {mapped}, expected {LIB_PATH}")
    return _lib


def version() -> str:
    """tl_version(): names the build (and a comparison build's switch)."""
    return load().tl_version().decode()


def loaded_path() -> str | None:
    """Path of the libtinyllm_kv.so this process has mapped (from
    /proc/self/maps), or None when none is mapped."""
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                if line.rstrip().endswith("libtinyllm_kv.so"):
                    return line.split(None, 5)[5].strip()
    except OSError:
        pass
    return None


class KVConfig(C.Structure):
    _fields_ = [("num_layers", C.c_int), ("num_heads", C.c_int), ("head_dim", C.c_int),
                ("max_seq_len", C.c_int), ("max_batch_size", C.c_int)]


class KVView(C.Structure):
    _fields_ = [("k_base", C.c_void_p), ("v_base", C.c_void_p), ("block_table", C.c_void_p),
                ("bt_stride", C.c_int), ("log2_blk", C.c_int), ("blk_stride", C.c_int64),
                ("tok_stride", C.c_int64), ("head_stride", C.c_int64)]


class AttnPlanInfo(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("chunk_tokens", "work_items", "waves", "any_multi",
                                       "any_empty", "max_len", "inline_words", "inline_compact",
                                       "head_fused", "fused_chunked")]


def _declare(L: C.CDLL) -> None:
    vp, i, sz, f = C.c_void_p, C.c_int, C.c_size_t, C.c_float
    ip = C.POINTER(C.c_int)
    sig = {
        "tl_last_error": (C.c_char_p, []),
        "tl_version": (C.c_char_p, []),
        "tl_kv_create": (i, [C.POINTER(KVConfig), C.POINTER(vp)]),
        "tl_kv_destroy": (None, [vp]),
        "tl_kv_allocate_sequence": (i, [vp, i, ip]),
        "tl_kv_release_sequence": (i, [vp, i]),
        "tl_kv_get_cache": (i, [vp, i, i, C.POINTER(vp), C.POINTER(vp)]),
        "tl_kv_append": (i, [vp, i, i, vp, vp, i, vp]),
        "tl_kv_advance": (i, [vp, i, i]),
        "tl_kv_seq_len": (i, [vp, i]),
        "tl_kv_has_sequence": (i, [vp, i]),
        "tl_kv_used_memory": (sz, [vp]),
        "tl_kv_total_memory": (sz, [vp]),
        "tl_kv_free_memory": (sz, [vp]),
        "tl_kv_active_count": (i, [vp]),
        "tl_kv_get_config": (i, [vp, C.POINTER(KVConfig)]),
        "tl_kv_pool": (vp, [vp]),
        "tl_kv_slot_bytes": (sz, [vp]),
        "tl_kv_slot_of": (i, [vp, i]),
        "tl_kv_set_block_map": (i, [vp, i, vp, sz]),
        "tl_kv_create_paged": (i, [C.POINTER(KVConfig), i, i, C.POINTER(vp)]),
        "tl_kv_num_blocks": (i, [vp]),
        "tl_kv_free_blocks": (i, [vp]),
        "tl_kv_block_bytes": (sz, [vp]),
        "tl_kv_block_table": (i, [vp, i, vp, ip]),
        "tl_kv_batch_create": (i, [vp, i, i, C.POINTER(vp)]),
        "tl_kv_batch_destroy": (None, [vp]),
        "tl_kv_batch_prepare": (i, [vp, vp, i, vp]),
        "tl_kv_batch_prepare_lengths": (i, [vp, vp, vp, i, vp]),
        "tl_kv_batch_info": (i, [vp, ip, ip, ip]),
        "tl_kv_batch_append": (i, [vp, i, i, vp, vp, vp]),
        "tl_kv_batch_attention": (i, [vp, i, vp, vp, f, vp]),
        "tl_kv_batch_decode": (i, [vp, i, vp, vp, vp, vp, f, vp]),
        "tl_kv_batch_gather": (i, [vp, i, vp, vp, i, vp]),
        "tl_kv_batch_commit": (i, [vp, i]),
        "tl_kv_batch_project": (i, [vp, i, vp, i, i, vp, vp, vp, vp, vp, vp, vp, i, vp]),
        "tl_w8a16_pack": (i, [vp, i, i, vp, vp]),
        "tl_w8a16_matmul": (i, [vp, vp, vp, vp, i, i, i, i, vp]),
        "tl_w8a16_matmul_residual": (i, [vp, vp, vp, vp, i, i, i, i, i, vp]),
        "tl_w8a16_set_path": (i, [i]),
        "tl_attn_decode_gqa": (i, [vp, C.POINTER(KVView), vp, i, i, i, i, f, vp, vp]),
        "tl_attn_decode_gqa_noalloc": (i, [vp, C.POINTER(KVView), vp, i, i, i, i, f, vp, vp]),
        "tl_attn_noalloc_scratch_bytes": (sz, []),
        "tl_attention_decode": (None, [vp, vp, vp, vp, f, i, i, i, i, vp]),
        "tl_attention_prefill": (None, [vp, vp, vp, vp, f, i, i, i, i, vp]),
        "tl_softmax": (None, [vp, vp, i, i, vp]),
        "tl_get_attention_weights": (None, [vp, vp, vp, f, i, i, i, i, i, i, vp]),
        "tl_kv_prefill_create": (i, [vp, i, i, C.POINTER(vp)]),
        "tl_kv_prefill_destroy": (None, [vp]),
        "tl_kv_prefill_prepare": (i, [vp, vp, vp, i, vp]),
        "tl_kv_prefill_info": (i, [vp, ip, ip]),
        "tl_kv_prefill_append": (i, [vp, i, vp, vp, vp]),
        "tl_kv_prefill_attention": (i, [vp, i, vp, vp, f, vp]),
        "tl_kv_prefill_run": (i, [vp, i, vp, vp, vp, vp, f, vp]),
        "tl_kv_prefill_commit": (i, [vp]),
        "tl_prefill_set_waves": (i, [i]),
        "tl_prefill_get_waves": (i, []),
        "tl_prefill_plan_waves": (i, [vp, vp, i, i, i, i, i, ip]),
        "tl_attn_set_score_path": (i, [i]),
        "tl_attn_get_score_path": (i, []),
        "tl_attn_set_waves": (i, [i]),
        "tl_attn_get_waves": (i, []),
        "tl_attn_set_head_fuse": (i, [i]),
        "tl_attn_get_head_fuse": (i, []),
        "tl_attn_set_fused_merge": (i, [i]),
        "tl_attn_get_fused_merge": (i, []),
        "tl_fill_normal_f16": (i, [C.c_uint64, C.c_uint64, C.c_float, vp, sz, vp]),
        "tl_attn_plan": (i, [vp, i, i, i, i, i, i, i, i, C.POINTER(AttnPlanInfo), vp, vp]),
        "tl_profile_enable": (None, [i]),
        "tl_profile_reset": (None, []),
        "tl_profile_query": (i, [C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_longlong)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Every function the public header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tl_[a-z0-9_]+)\s*\(", text)))


def last_error() -> str:
    return load().tl_last_error().decode()


def _check(rc: int) -> None:
    if rc != TL_OK:
        raise TinyLLMError(rc, last_error())


def _int_array(vals):
    """A C int array for the C ABI: a C-contiguous int32 numpy array is
    passed by address (no copy); anything else is copied."""
    if type(vals).__name__ == "ndarray" and vals.dtype.str == "<i4" and vals.flags.c_contiguous:
        return (vals.ctypes.data if vals.size else None), int(vals.size)
    vals = list(vals)
    return (C.c_int * max(1, len(vals)))(*vals), len(vals)


class KVCacheManager:
    """tiny_llm::KVCacheManager over HIP (same method names as the reference)."""

    def __init__(self, num_layers=32, num_heads=32, head_dim=128, max_seq_len=2048,
                 max_batch_size=1, block_tokens=0, num_blocks=0):
        """block_tokens > 0: a block-granular pool of num_blocks blocks
        (tl_kv_create_paged); otherwise the reference's slot pool."""
        L = load()
        # the destructor's handle: module globals may already be None when a
        # manager is collected at interpreter shutdown
        self._destroy = L.tl_kv_destroy
        self.config = KVConfig(num_layers, num_heads, head_dim, max_seq_len, max_batch_size)
        self._h = C.c_void_p()
        if block_tokens:
            _check(L.tl_kv_create_paged(C.byref(self.config), block_tokens, num_blocks,
                                        C.byref(self._h)))
        else:
            _check(L.tl_kv_create(C.byref(self.config), C.byref(self._h)))

    @classmethod
    def create(cls, **cfg):
        """Result-style factory: (manager, None) or (None, error message)."""
        try:
            return cls(**cfg), None
        except TinyLLMError as e:
            return None, e.msg

    def close(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    # Result<T>-like methods return (value, error) with error None on success.
    def allocateSequence(self, max_len):
        out = C.c_int(-1)
        rc = load().tl_kv_allocate_sequence(self._h, max_len, C.byref(out))
        return (out.value, None) if rc == TL_OK else (None, last_error())

    def releaseSequence(self, seq_id):
        rc = load().tl_kv_release_sequence(self._h, seq_id)
        return None if rc == TL_OK else last_error()

    def getCacheChecked(self, seq_id, layer_idx):
        k, v = C.c_void_p(), C.c_void_p()
        rc = load().tl_kv_get_cache(self._h, seq_id, layer_idx, C.byref(k), C.byref(v))
        return ((k.value or 0, v.value or 0), None) if rc == TL_OK else (None, last_error())

    def getCache(self, seq_id, layer_idx):
        r, _ = self.getCacheChecked(seq_id, layer_idx)
        return r if r is not None else (0, 0)

    def numBlocks(self):
        return load().tl_kv_num_blocks(self._h)

    def freeBlocks(self):
        return load().tl_kv_free_blocks(self._h)

    def blockBytes(self):
        return load().tl_kv_block_bytes(self._h)

    def blockTable(self, seq_id):
        """(physical block ids in token order, None) or (None, error)."""
        n = C.c_int(0)
        rc = load().tl_kv_block_table(self._h, seq_id, None, C.byref(n))
        if rc != TL_OK:
            return None, last_error()
        out = (C.c_int32 * max(1, n.value))()
        rc = load().tl_kv_block_table(self._h, seq_id, out, C.byref(n))
        return (list(out)[:n.value], None) if rc == TL_OK else (None, last_error())

    def appendKV(self, seq_id, layer_idx, new_k, new_v, num_tokens, stream=0):
        rc = load().tl_kv_append(self._h, seq_id, layer_idx, new_k, new_v, num_tokens, stream)
        if rc == TL_ERR_HIP:
            raise TinyLLMError(rc, last_error())
        return None if rc == TL_OK else last_error()

    def advanceSeqLen(self, seq_id, num_tokens):
        rc = load().tl_kv_advance(self._h, seq_id, num_tokens)
        return None if rc == TL_OK else last_error()

    def getSeqLen(self, seq_id):
        return load().tl_kv_seq_len(self._h, seq_id)

    def hasSequence(self, seq_id):
        return bool(load().tl_kv_has_sequence(self._h, seq_id))

    def getUsedMemory(self):
        return load().tl_kv_used_memory(self._h)

    def getTotalMemory(self):
        return load().tl_kv_total_memory(self._h)

    def getFreeMemory(self):
        return load().tl_kv_free_memory(self._h)

    def getActiveSequenceCount(self):
        return load().tl_kv_active_count(self._h)

    def getConfig(self):
        c = KVConfig()
        _check(load().tl_kv_get_config(self._h, C.byref(c)))
        return c

    def pool(self) -> int:
        return load().tl_kv_pool(self._h) or 0

    def slot_bytes(self) -> int:
        return load().tl_kv_slot_bytes(self._h)

    def slot_of(self, seq_id) -> int:
        return load().tl_kv_slot_of(self._h, seq_id)

    def setBlockMap(self, block_tokens, perm):
        if perm is None:
            rc = load().tl_kv_set_block_map(self._h, block_tokens, None, 0)
        else:
            import numpy as np
            p = np.ascontiguousarray(perm, dtype=np.int32)
            rc = load().tl_kv_set_block_map(self._h, block_tokens, p.ctypes.data, p.size)
        return None if rc == TL_OK else last_error()


class DecodeBatch:
    """Batched decode step over a KVCacheManager (tl_kv_batch_*)."""

    def __init__(self, mgr: KVCacheManager, max_seqs: int, num_q_heads: int):
        self._mgr = mgr
        self._h = C.c_void_p()
        self._destroy = load().tl_kv_batch_destroy  # usable at interpreter shutdown
        _check(load().tl_kv_batch_create(mgr._h, max_seqs, num_q_heads, C.byref(self._h)))

    def close(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def prepare(self, seq_ids, stream=0):
        arr, n = _int_array(seq_ids)
        _check(load().tl_kv_batch_prepare(self._h, arr, n, stream))

    def prepare_lengths(self, seq_ids, attended, stream=0):
        ids, n = _int_array(seq_ids)
        att, m = _int_array(attended)
        assert n == m
        _check(load().tl_kv_batch_prepare_lengths(self._h, ids, att, n, stream))

    def info(self):
        n, chunk, work = C.c_int(), C.c_int(), C.c_int()
        _check(load().tl_kv_batch_info(self._h, C.byref(n), C.byref(chunk), C.byref(work)))
        return {"n": n.value, "chunk_tokens": chunk.value, "work_items": work.value}

    def append(self, layer_begin, num_layers, new_k, new_v, stream=0):
        _check(load().tl_kv_batch_append(self._h, layer_begin, num_layers, new_k, new_v, stream))

    def attention(self, layer, q, out, scale, stream=0):
        _check(load().tl_kv_batch_attention(self._h, layer, q, out, scale, stream))

    def decode(self, layer, q, new_k, new_v, out, scale, stream=0):
        _check(load().tl_kv_batch_decode(self._h, layer, q, new_k, new_v, out, scale, stream))

    def gather(self, layer, k_out, v_out, s_max, stream=0):
        _check(load().tl_kv_batch_gather(self._h, layer, k_out or None, v_out or None, s_max, stream))

    def project(self, layer, x, hidden, group_size, wk, sk, wv, sv, wq=None, sq=None, q_out=None,
                stream=0, packed=False):
        """K/V projections with the append fused (tl_kv_batch_project)."""
        _check(load().tl_kv_batch_project(self._h, layer, x, hidden, group_size, wk, sk, wv, sv,
                                          wq or None, sq or None, q_out or None, int(packed), stream))

    def commit(self, num_tokens=1):
        """advanceSeqLen(seq, num_tokens) for every sequence of the last prepare."""
        _check(load().tl_kv_batch_commit(self._h, num_tokens))


class PrefillBatch:
    """tiny_llm::PrefillBatch: new tokens of several sequences appended and
    attended causally over the cache (tl_kv_prefill_*)."""

    def __init__(self, mgr: KVCacheManager, max_seqs: int, num_q_heads: int):
        self.mgr = mgr
        self._h = C.c_void_p()
        self._destroy = load().tl_kv_prefill_destroy  # usable at interpreter shutdown
        _check(load().tl_kv_prefill_create(mgr._h, max_seqs, num_q_heads, C.byref(self._h)))

    def close(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def prepare(self, seq_ids, num_tokens, stream=0):
        n = len(seq_ids)
        ids = (C.c_int * max(1, n))(*seq_ids)
        cnt = (C.c_int * max(1, n))(*num_tokens)
        _check(load().tl_kv_prefill_prepare(self._h, ids, cnt, n, stream))

    def info(self):
        n, t = C.c_int(), C.c_int()
        _check(load().tl_kv_prefill_info(self._h, C.byref(n), C.byref(t)))
        return {"n": n.value, "tokens": t.value}

    def append(self, layer, new_k, new_v, stream=0):
        _check(load().tl_kv_prefill_append(self._h, layer, new_k, new_v, stream))

    def attention(self, layer, q, out, scale, stream=0):
        _check(load().tl_kv_prefill_attention(self._h, layer, q, out, scale, stream))

    def run(self, layer, q, new_k, new_v, out, scale, stream=0):
        _check(load().tl_kv_prefill_run(self._h, layer, q, new_k, new_v, out, scale, stream))

    def commit(self):
        _check(load().tl_kv_prefill_commit(self._h))


def attention_prefill(q, k, v, out, scale, batch, num_heads, seq_len, head_dim, stream=0):
    """kernels::attention_prefill: compact [B][H][S][D], causal."""
    load().tl_attention_prefill(q, k, v, out, scale, batch, num_heads, seq_len, head_dim, stream)


def softmax(inp, out, batch, seq_len, stream=0):
    load().tl_softmax(inp, out, batch, seq_len, stream)


def get_attention_weights(q, k, w, scale, batch, num_heads, query_len, key_len, head_dim, causal,
                          stream=0):
    load().tl_get_attention_weights(q, k, w, scale, batch, num_heads, query_len, key_len, head_dim,
                                    int(causal), stream)


def attn_decode_gqa(q, view: KVView, seq_lens, Hq, Hkv, D, scale, out, stream=0):
    import numpy as np
    lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    _check(load().tl_attn_decode_gqa(q, C.byref(view), lens.ctypes.data, lens.size, Hq, Hkv, D,
                                     scale, out, stream))


def attn_decode_gqa_noalloc(q, view: KVView, seq_lens, Hq, Hkv, D, scale, out, stream=0):
    """tl_attn_decode_gqa_noalloc: tl_attn_decode_gqa with the library's
    static device scratch instead of any allocation."""
    import numpy as np
    lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    _check(load().tl_attn_decode_gqa_noalloc(q, C.byref(view), lens.ctypes.data, lens.size, Hq,
                                             Hkv, D, scale, out, stream))


def attn_noalloc_scratch_bytes() -> int:
    return load().tl_attn_noalloc_scratch_bytes()


def attention_decode(q, k, v, out, scale, batch, num_heads, seq_len, head_dim, stream=0):
    """tiny_llm::kernels::attention_decode (void; errors go to the log and
    tl_last_error)."""
    load().tl_attention_decode(q, k, v, out, scale, batch, num_heads, seq_len, head_dim, stream)


SCORE_VALU = 0
SCORE_MFMA = 1
SCORE_AUTO = 2
SCORE_MMA = 3


def set_score_path(path: int):
    """0 = VALU dot products, 1 = MFMA over an LDS-transposed K tile,
    2 = auto (VALU for every supported group), 3 = both contractions on MFMA
    (head_dim 64 and 128; other head_dims take the auto kernel)."""
    _check(load().tl_attn_set_score_path(path))


def get_score_path() -> int:
    return load().tl_attn_get_score_path()


def set_waves(waves: int):
    """Waves per attention workgroup: 0 = auto, 4 or 8."""
    _check(load().tl_attn_set_waves(waves))


def get_waves() -> int:
    return load().tl_attn_get_waves()


def set_head_fuse(mode: int):
    """Head-fused decode plans: 0 = auto, 1 = off, 2 / 4 / 8 = that many kv
    heads per workgroup where a plan with it applies."""
    _check(load().tl_attn_set_head_fuse(mode))


def get_head_fuse() -> int:
    return load().tl_attn_get_head_fuse()


def set_fused_merge(on: bool):
    """Multi-chunk decode plans merge their partials in a second launch
    (False, the default) or inside the attention launch (True); same bits."""
    _check(load().tl_attn_set_fused_merge(1 if on else 0))


def get_fused_merge() -> bool:
    return bool(load().tl_attn_get_fused_merge())


def set_prefill_waves(waves: int):
    """Waves per prefill-attention workgroup: 0 = auto, 4 or 8."""
    _check(load().tl_prefill_set_waves(waves))


def get_prefill_waves() -> int:
    return load().tl_prefill_get_waves()


def prefill_plan_waves(prefix_lens, num_tokens, num_q_heads, num_kv_heads, head_dim, num_cus=0) -> int:
    """The waves per workgroup the prefill entry points choose (under the
    current setting) for sequences with prefix_lens[i] cached and
    num_tokens[i] new tokens; num_cus 0 = the current device's."""
    import numpy as np
    p = np.ascontiguousarray(prefix_lens, dtype=np.int32)
    t = np.ascontiguousarray(num_tokens, dtype=np.int32)
    if p.shape != t.shape:
        raise ValueError("prefix_lens and num_tokens differ in length")
    out = C.c_int(0)
    _check(load().tl_prefill_plan_waves(p.ctypes.data if p.size else None, t.ctypes.data if t.size else None,
                                        int(p.size), num_q_heads,
                                        num_kv_heads, head_dim, num_cus, C.byref(out)))
    return out.value


_HEAD_FUSE_CODES = {"current": -1, "auto": 0, "off": 1, 2: 2, 4: 4, 8: 8}


def attn_plan(seq_lens, num_kv_heads, num_cus=256, forced_chunk=0, waves=0, with_rows=True,
              head_fuse="current", head_dim=128):
    """The decode attention launch plan for these attended lengths (host
    only): a dict of tl_attn_plan_info plus part_base and the work list as
    (entry, chunk) pairs in launch order.  head_fuse: "current" = the plan the
    decode entry points make now, under this process's settings (head-fuse
    mode, waves, score path, TL_ATTN_CHUNK; forced_chunk / waves of 0 mean
    the process setting); "auto" / "off" / 2 / 4 / 8 = the codes of
    set_head_fuse, as if set."""
    import numpy as np
    if isinstance(head_fuse, bool) or head_fuse not in _HEAD_FUSE_CODES:
        raise ValueError(f"head_fuse must be one of {list(_HEAD_FUSE_CODES)}, not {head_fuse!r}")
    code = _HEAD_FUSE_CODES[head_fuse]
    lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    n = lens.size
    info = AttnPlanInfo()
    args = (lens.ctypes.data if n else None, n, num_kv_heads, head_dim, num_cus, forced_chunk, waves,
            code, int(with_rows), C.byref(info))
    _check(load().tl_attn_plan(*args, None, None))
    part = np.zeros(n + 1, dtype=np.int32)
    work = np.zeros(max(1, 2 * info.work_items), dtype=np.int32)
    _check(load().tl_attn_plan(*args, part.ctypes.data, work.ctypes.data))
    out = {name: getattr(info, name) for name, _ in AttnPlanInfo._fields_}
    out["part_base"] = part
    out["work"] = work[:2 * info.work_items].reshape(-1, 2)
    return out


def fill_normal(seed, first, stddev, out, n, stream=0):
    """out[j] = element first + j of the seeded normal fp16 stream
    (tl_fill_normal_f16; the oracle's orc_fill_normal_f16 element for
    element)."""
    _check(load().tl_fill_normal_f16(seed, first, stddev, out, n, stream))


class NormalStreams:
    """Seeded fp16 normal streams drawn on the device in call order: each seed
    is one stream, and every draw continues it where the last draw of that
    seed ended (tl_fill_normal_f16), so a sequence of draws defines the same
    values on any host and torch build.  Draws return torch tensors."""

    def __init__(self, stream=0):
        self.stream = stream
        self.offset = {}

    def draw(self, seed, shape, stddev=1.0):
        import math
        import torch
        t = torch.empty(shape, dtype=torch.float16, device="cuda")
        n = math.prod(shape) if isinstance(shape, (tuple, list)) else int(shape)
        first = self.offset.get(seed, 0)
        fill_normal(seed, first, stddev, t.data_ptr(), n, self.stream)
        self.offset[seed] = first + n
        return t


def profile_enable(on: bool = True):
    load().tl_profile_enable(1 if on else 0)


def profile_reset():
    load().tl_profile_reset()


def profile_query(kernel: str):
    ms, n = C.c_double(), C.c_longlong()
    _check(load().tl_profile_query(kernel.encode(), C.byref(ms), C.byref(n)))
    return ms.value, n.value


def w8a16_matmul(input, weight, scales, output, M, N, K, group_size, stream=0):
    """kernels::w8a16_matmul over device pointers."""
    _check(load().tl_w8a16_matmul(input, weight, scales, output, M, N, K, group_size, stream))


def w8a16_matmul_residual(input, weight, scales, hidden, M, N, K, group_size, stream=0,
                          packed=False):
    """hidden = fp16(hidden + fp16(input @ dequant(weight, scales))), in place."""
    _check(load().tl_w8a16_matmul_residual(input, weight, scales, hidden, M, N, K, group_size,
                                           int(packed), stream))


def w8a16_pack(weight, K, N, packed, stream=0):
    """Repack weight [K][N] int8 into the MFMA-fragment layout (K*N bytes)."""
    _check(load().tl_w8a16_pack(weight, K, N, packed, stream))


def w8a16_set_path(path: int):
    """0 = MFMA where the shape allows, 1 = always the reference-order kernel."""
    _check(load().tl_w8a16_set_path(path))
