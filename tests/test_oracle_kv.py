"""Pins the oracle's KVCacheManager restatement.

Ports every live KV test of the reference (tests/test_kv_cache.cpp:43-287),
its disabled property tests (:298-443, run here over all small cases), and
the cache round trips of tests/test_transformer.cu (:141-194, :302-446).
The layout test checks the pool against the layout the reference documents
in kv_cache.cpp:70-71 ("[Layer 0 K][Layer 0 V][Layer 1 K]..." per slot),
built by concatenating regions rather than by an offset formula."""
import itertools

import numpy as np
import pytest


def make(orc, num_layers=2, num_heads=4, head_dim=64, max_seq_len=128, max_batch_size=4):
    # KVCacheTest::createConfig defaults (test_kv_cache.cpp:23-32)
    return orc.KVCacheOracle(num_layers, num_heads, head_dim, max_seq_len, max_batch_size)


# ---------------------------------------------------------------- live tests
def test_initialization_allocates_memory(orc):
    c = make(orc)
    assert c.total() > 0 and c.used() == 0 and c.active() == 0


def test_allocate_sequence_returns_valid_id(orc):
    c = make(orc)
    sid, err = c.allocate(64)
    assert err is None and sid >= 0 and c.has(sid) and c.seq_len(sid) == 0


def test_allocate_multiple_sequences(orc):
    c = make(orc, 2, 4, 64, 128, 4)
    ids = [c.allocate(64)[0] for _ in range(4)]
    assert c.active() == 4 and len(set(ids)) == 4


def test_exhaustion_returns_error(orc):
    c = make(orc, 2, 4, 64, 128, 2)
    assert c.allocate(64)[1] is None and c.allocate(64)[1] is None
    sid, err = c.allocate(64)
    assert sid is None and "exhausted" in err


def test_release_sequence_frees_slot(orc):
    c = make(orc, 2, 4, 64, 128, 2)
    s1, _ = c.allocate(64)
    c.allocate(64)
    c.release(s1)
    assert not c.has(s1) and c.active() == 1
    assert c.allocate(64)[1] is None


def test_get_cache_returns_valid_pointers(orc):
    c = make(orc)
    sid, _ = c.allocate(64)
    for layer in range(2):
        (k, v), err = c.get_cache(sid, layer)
        assert err is None and k != v


def test_get_cache_for_invalid_sequence_returns_error(orc):
    c = make(orc)
    r, err = c.get_cache(999, 0)
    assert r is None and "not found" in err


def test_invalid_max_len_returns_error(orc):
    c = make(orc, 2, 4, 64, 128, 4)
    for bad in (0, -1, 256):
        sid, err = c.allocate(bad)
        assert sid is None and err


def test_memory_accounting_is_correct(orc):
    c = make(orc, 2, 4, 64, 128, 4)
    total = c.total()
    assert c.free() == total and c.used() == 0
    c.allocate(64)
    one = c.used()
    assert one > 0 and c.free() == total - one
    c.allocate(64)
    assert c.used() == 2 * one


def test_append_does_not_advance_visible_length(orc):
    c = make(orc, 2, 4, 8, 32, 2)
    sid, _ = c.allocate(16)
    n = 3 * 4 * 8
    k = np.full(n, 0x3C00, np.uint16)  # 1.0
    v = np.full(n, 0x4000, np.uint16)  # 2.0
    assert c.append(sid, 0, k, v, 3) is None
    assert c.seq_len(sid) == 0
    c.advance(sid, 3)
    assert c.seq_len(sid) == 3


def test_invalid_layer_returns_error(orc):
    c = make(orc, 2, 4, 8, 32, 2)
    sid, _ = c.allocate(16)
    assert c.get_cache(sid, -1)[0] is None
    assert c.get_cache(sid, 2)[0] is None


def test_invalid_append_inputs_do_not_advance(orc):
    c = make(orc, 2, 4, 8, 32, 2)
    sid, _ = c.allocate(16)
    assert c.append(sid, -1, None, None, 0) == "new_k is null"
    one = np.zeros(32, np.uint16)
    assert "num_tokens must be positive" in c.append(sid, 0, one, one, 0)
    assert "Invalid layer_idx" in c.append(sid, 2, one, one, 1)
    assert "sequence not found" in c.append(sid + 7, 0, one, one, 1)
    assert c.seq_len(sid) == 0


def test_append_overflow_is_rejected(orc):
    c = make(orc, 1, 1, 8, 32, 1)
    sid, _ = c.allocate(4)
    row = np.zeros(8 * 5, np.uint16)
    assert "cache overflow" in c.append(sid, 0, row, row, 5)
    assert c.append(sid, 0, row, row, 4) is None


def test_advance_clamps_to_capacity(orc):
    c = make(orc, 2, 4, 8, 32, 2)
    sid, _ = c.allocate(5)
    c.advance(sid, 100)
    assert c.seq_len(sid) == 5


def test_advance_ignores_non_positive(orc):
    c = make(orc, 2, 4, 8, 32, 2)
    sid, _ = c.allocate(5)
    assert c.advance(sid, 0) and c.advance(sid, -3)
    assert c.seq_len(sid) == 0


def test_invalid_config_rejected(orc):
    for bad in [(0, 1, 1, 1, 1), (1, 0, 1, 1, 1), (1, 1, 0, 1, 1), (1, 1, 1, 0, 1), (1, 1, 1, 1, 0)]:
        obj, err = orc.KVCacheOracle.try_create(*bad)
        assert obj is None and "invalid configuration" in err


# ---------------------------------------------------- disabled property tests
@pytest.mark.parametrize("num_allocs", range(1, 9))
def test_allocation_invariant(orc, num_allocs):
    c = make(orc, 2, 4, 64, 128, 8)
    ids = []
    for _ in range(num_allocs):
        sid, err = c.allocate(64)
        assert err is None and c.has(sid) and c.seq_len(sid) == 0
        for layer in range(2):
            assert c.get_cache(sid, layer)[1] is None
        ids.append(sid)
    assert c.active() == len(ids)


@pytest.mark.parametrize("pattern", list(itertools.product([False, True], repeat=4)))
def test_release_invariant(orc, pattern):
    c = make(orc, 2, 4, 64, 128, 4)
    ids = [c.allocate(64)[0] for _ in range(4)]
    used, active = c.used(), c.active()
    released = 0
    for sid, rel in zip(ids, pattern):
        if rel:
            c.release(sid)
            assert not c.has(sid)
            released += 1
    assert c.active() == active - released
    if released:
        assert c.used() < used


@pytest.mark.parametrize("num_ops", range(1, 21))
def test_memory_invariant(orc, num_ops):
    c = make(orc, 2, 4, 64, 128, 4)
    total = c.total()
    for i in range(num_ops):
        assert c.used() + c.free() == total
        assert c.used() == c.active() * c.slot_bytes()
        if c.active() < 4 and i % 2 == 0:
            c.allocate(64)
        elif c.active() > 0:
            for j in range(100):
                if c.has(j):
                    c.release(j)
                    break
    assert c.used() + c.free() == total


def test_exhaustion_invariant(orc):
    c = make(orc, 2, 4, 64, 128, 3)
    for _ in range(3):
        assert c.allocate(64)[1] is None
    assert c.allocate(64)[1] is not None
    assert c.active() == 3
    c.release(0)
    assert c.allocate(64)[1] is None


def test_ids_are_never_reused_and_slot_is_lowest_free(orc):
    c = make(orc, 1, 1, 8, 16, 3)
    a, b, d = (c.allocate(4)[0] for _ in range(3))
    assert (a, b, d) == (0, 1, 2)
    c.release(b)
    e, _ = c.allocate(4)
    assert e == 3 and c.slot_of(e) == 1  # lowest free slot, fresh id


# ------------------------------------------------------------- layout / data
def _tagged(rng, n):
    return rng.integers(0, 0x7C00, size=n, dtype=np.uint16)  # finite halves


def test_pool_layout_matches_documented_order(orc):
    L, H, D, M, B = 2, 3, 8, 16, 3
    c = make(orc, L, H, D, M, B)
    rng = np.random.default_rng(11)
    ids = [c.allocate(M)[0] for _ in range(B)]
    regions = {}
    for s, sid in enumerate(ids):
        for layer in range(L):
            k = _tagged(rng, M * H * D)
            v = _tagged(rng, M * H * D)
            assert c.append(sid, layer, k, v, M) is None
            regions[(s, layer, "K")] = k
            regions[(s, layer, "V")] = v
    expected = np.concatenate([regions[(s, layer, kind)]
                               for s in range(B) for layer in range(L) for kind in ("K", "V")])
    assert np.array_equal(c.pool(), expected)


def test_append_retrieve_round_trip(orc):
    # TransformerTest.KVCacheAppendRetrieve (test_transformer.cu:141-194)
    c = make(orc, 2, 4, 32, 64, 2)
    sid, _ = c.allocate(32)
    rng = np.random.default_rng(200)
    k, v = _tagged(rng, 4 * 4 * 32), _tagged(rng, 4 * 4 * 32)
    c.append(sid, 0, k, v, 4)
    assert c.seq_len(sid) == 0
    c.advance(sid, 4)
    (ko, vo), _ = c.get_cache(sid, 0)
    pool = c.pool()
    assert np.array_equal(pool[ko:ko + k.size], k) and np.array_equal(pool[vo:vo + v.size], v)


@pytest.mark.parametrize("L,H,M,D", [(1, 2, 32, 16), (4, 8, 128, 64), (3, 5, 77, 24)])
def test_cache_preserves_data_all_layers(orc, L, H, M, D):
    # KVCachePreservesData (test_transformer.cu:302-381)
    c = make(orc, L, H, D, M, 2)
    sid, _ = c.allocate(M // 2)
    rng = np.random.default_rng(L * 100 + H)
    data = [(_tagged(rng, 4 * H * D), _tagged(rng, 4 * H * D)) for _ in range(L)]
    for layer, (k, v) in enumerate(data):
        assert c.append(sid, layer, k, v, 4) is None
    pool = c.pool()
    for layer, (k, v) in enumerate(data):
        (ko, vo), _ = c.get_cache(sid, layer)
        assert np.array_equal(pool[ko:ko + k.size], k) and np.array_equal(pool[vo:vo + v.size], v)


def test_sequential_append_equivalence(orc):
    # SequentialAppendEquivalence (test_transformer.cu:383-446)
    H, D = 5, 40
    c = make(orc, 1, H, D, 64, 2)
    sid, _ = c.allocate(64)
    rng = np.random.default_rng(3)
    ks, vs = [], []
    for _ in range(8):
        k, v = _tagged(rng, H * D), _tagged(rng, H * D)
        c.append(sid, 0, k, v, 1)
        c.advance(sid, 1)
        ks.append(k)
        vs.append(v)
    assert c.seq_len(sid) == 8
    (ko, vo), _ = c.get_cache(sid, 0)
    pool = c.pool()
    assert np.array_equal(pool[ko:ko + 8 * H * D], np.concatenate(ks))
    assert np.array_equal(pool[vo:vo + 8 * H * D], np.concatenate(vs))


def test_release_leaves_device_bytes_stale(orc):
    c = make(orc, 1, 2, 8, 16, 1)
    sid, _ = c.allocate(16)
    rng = np.random.default_rng(5)
    k, v = _tagged(rng, 3 * 16), _tagged(rng, 3 * 16)
    c.append(sid, 0, k, v, 3)
    before = c.pool().copy()
    c.release(sid)
    sid2, _ = c.allocate(16)
    assert c.seq_len(sid2) == 0 and np.array_equal(c.pool(), before)
