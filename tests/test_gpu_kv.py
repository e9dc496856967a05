"""GPU: KVCacheManager over HIP vs the oracle.

Every reference KV test (tests/test_kv_cache.cpp:43-287) runs against the
product, and whole pools are compared bit-for-bit (uint16) with the oracle
after identical operation sequences: appendKV, the fused batched append,
release / re-allocate (stale bytes included) and paged block maps."""
import numpy as np
import pytest

from devutil import read_dev, stream, to_dev

pytestmark = pytest.mark.gpu


class Pair:
    """The product manager and the oracle driven with the same operations."""

    def __init__(self, tl, orc, L, H, D, M, B):
        self.tl = tl
        self.g = tl.KVCacheManager(L, H, D, M, B)
        self.o = orc.KVCacheOracle(L, H, D, M, B)
        self.L, self.H, self.D, self.M, self.B = L, H, D, M, B
        self.keep = []

    def allocate(self, max_len):
        a, ea = self.g.allocateSequence(max_len)
        b, eb = self.o.allocate(max_len)
        assert a == b and (ea is None) == (eb is None), (a, b, ea, eb)
        if ea is not None:
            assert ea == eb
        return a

    def release(self, sid):
        assert self.g.releaseSequence(sid) == self.o.release(sid)

    def append(self, sid, layer, k, v, n):
        dk, dv = to_dev(k), to_dev(v)
        self.keep += [dk, dv]
        e1 = self.g.appendKV(sid, layer, dk.data_ptr(), dv.data_ptr(), n, stream())
        e2 = self.o.append(sid, layer, k, v, n)
        assert e1 == e2, (e1, e2)

    def advance(self, sid, n):
        assert self.g.advanceSeqLen(sid, n) == self.o.advance(sid, n)

    def check_state(self, ids):
        for s in ids:
            assert self.g.getSeqLen(s) == self.o.seq_len(s)
            assert self.g.hasSequence(s) == self.o.has(s)
            assert self.g.slot_of(s) == self.o.slot_of(s)
        assert self.g.getUsedMemory() == self.o.used()
        assert self.g.getTotalMemory() == self.o.total()
        assert self.g.getActiveSequenceCount() == self.o.active()

    def pool_equal(self):
        n = self.o.pool().size
        return np.array_equal(read_dev(self.g.pool(), n), self.o.pool())


def rnd(rng, n):
    return rng.integers(0, 0x7C00, size=n, dtype=np.uint16)


# ------------------------------------------------ reference tests, product side
def test_reference_kv_tests_on_product(tl):
    m = tl.KVCacheManager(2, 4, 64, 128, 4)
    assert m.getTotalMemory() > 0 and m.getUsedMemory() == 0 and m.getActiveSequenceCount() == 0
    sid, err = m.allocateSequence(64)
    assert err is None and sid >= 0 and m.hasSequence(sid) and m.getSeqLen(sid) == 0
    ids = [sid] + [m.allocateSequence(64)[0] for _ in range(3)]
    assert len(set(ids)) == 4 and m.getActiveSequenceCount() == 4
    none, err = m.allocateSequence(64)
    assert none is None and "exhausted" in err
    assert m.releaseSequence(ids[0]) is None and not m.hasSequence(ids[0])
    assert m.allocateSequence(64)[1] is None
    for layer in range(2):
        k, v = m.getCache(ids[1], layer)
        assert k and v and k != v
    assert m.getCache(999, 0) == (0, 0)
    assert m.getCache(ids[1], -1) == (0, 0) and m.getCache(ids[1], 2) == (0, 0)
    for bad in (0, -1, 256):
        assert m.allocateSequence(bad)[0] is None
    assert "not found" in m.releaseSequence(12345)


def test_memory_accounting_on_product(tl):
    m = tl.KVCacheManager(2, 4, 64, 128, 4)
    total = m.getTotalMemory()
    assert m.getFreeMemory() == total
    m.allocateSequence(64)
    one = m.getUsedMemory()
    assert one == m.slot_bytes() and m.getFreeMemory() == total - one
    m.allocateSequence(64)
    assert m.getUsedMemory() == 2 * one


def test_append_does_not_advance_and_clamps(tl):
    m = tl.KVCacheManager(2, 4, 8, 32, 2)
    sid, _ = m.allocateSequence(16)
    k = to_dev(np.full(3 * 32, 0x3C00, np.uint16))
    v = to_dev(np.full(3 * 32, 0x4000, np.uint16))
    assert m.appendKV(sid, 0, k.data_ptr(), v.data_ptr(), 3, stream()) is None
    assert m.getSeqLen(sid) == 0
    m.advanceSeqLen(sid, 3)
    assert m.getSeqLen(sid) == 3
    assert m.appendKV(sid, -1, 0, 0, 0) == "new_k is null"
    assert "Invalid layer_idx" in m.appendKV(sid, 2, k.data_ptr(), v.data_ptr(), 1)
    assert m.getSeqLen(sid) == 3
    assert m.advanceSeqLen(sid, 0) and m.advanceSeqLen(sid, -3)
    m.advanceSeqLen(sid, 100)
    assert m.getSeqLen(sid) == 16
    assert "cache overflow" in m.appendKV(sid, 0, k.data_ptr(), v.data_ptr(), 1)


def test_create_rejects_invalid_config(tl):
    obj, err = tl.KVCacheManager.create(num_layers=0, num_heads=1, head_dim=8, max_seq_len=8,
                                        max_batch_size=1)
    assert obj is None and "invalid configuration" in err


# ------------------------------------------------------- bit-exact pool parity
def test_pool_bit_exact_under_random_ops(tl, orc):
    rng = np.random.default_rng(1234)
    L, H, D, M, B = 3, 4, 32, 48, 5
    p = Pair(tl, orc, L, H, D, M, B)
    assert p.pool_equal()  # zeroed at create
    live = []
    for step in range(120):
        op = rng.integers(0, 10)
        if op < 2 and len(live) < B:
            live.append(p.allocate(int(rng.integers(1, M + 1))))
        elif op < 3 and live:
            sid = live.pop(int(rng.integers(0, len(live))))
            p.release(sid)
        elif op < 8 and live:
            sid = live[int(rng.integers(0, len(live)))]
            n = int(rng.integers(1, 6))
            layer = int(rng.integers(-1, L + 1))  # includes invalid layers
            p.append(sid, layer, rnd(rng, n * H * D), rnd(rng, n * H * D), n)
        elif live:
            p.advance(live[int(rng.integers(0, len(live)))], int(rng.integers(-1, 4)))
        p.check_state(live + [999])
    assert p.pool_equal()


@pytest.mark.parametrize("L,H,D", [(1, 8, 128), (2, 4, 64), (4, 2, 32), (1, 1, 256)])
def test_batched_append_bit_exact(tl, orc, L, H, D):
    """tl_kv_batch_append == n*L appendKV(n=1) calls (kv_cache.cpp:226-233)."""
    rng = np.random.default_rng(L * 10 + H)
    M, B = 64, 6
    p = Pair(tl, orc, L, H, D, M, B)
    ids = [p.allocate(M) for _ in range(B)]
    p.release(ids[1])  # a hole: batch slots are not contiguous
    ids = [i for i in ids if i != ids[1]]
    for sid in ids:
        n = int(rng.integers(0, 20))
        for layer in range(L):
            if n:
                p.append(sid, layer, rnd(rng, n * H * D), rnd(rng, n * H * D), n)
        if n:
            p.advance(sid, n)
    batch = tl.DecodeBatch(p.g, len(ids), H)
    order = list(rng.permutation(ids))
    for step in range(3):
        batch.prepare(order, stream())
        nk = rnd(rng, L * len(order) * H * D)
        nv = rnd(rng, L * len(order) * H * D)
        dk, dv = to_dev(nk), to_dev(nv)
        batch.append(0, L, dk.data_ptr(), dv.data_ptr(), stream())
        rows = nk.reshape(L, len(order), H * D), nv.reshape(L, len(order), H * D)
        for i, sid in enumerate(order):
            for layer in range(L):
                assert p.o.append(int(sid), layer, rows[0][layer, i], rows[1][layer, i], 1) is None
        for sid in order:
            p.advance(int(sid), 1)
        assert p.pool_equal()


def test_batch_prepare_rejects_bad_batches(tl):
    m = tl.KVCacheManager(1, 2, 32, 16, 3)
    a, _ = m.allocateSequence(2)
    b, _ = m.allocateSequence(16)
    batch = tl.DecodeBatch(m, 3, 4)
    with pytest.raises(tl.TinyLLMError, match="duplicate"):
        batch.prepare([a, a])
    with pytest.raises(tl.TinyLLMError, match="not found"):
        batch.prepare([a, 77])
    m.advanceSeqLen(a, 2)
    with pytest.raises(tl.TinyLLMError, match="cache overflow"):
        batch.prepare([a, b])
    with pytest.raises(tl.TinyLLMError):
        tl.DecodeBatch(m, 3, 3)  # 3 query heads over 2 kv heads


def test_paged_pool_append_bit_exact(tl, orc):
    """Paged block map: appendKV / batched append land where the block map
    says; checked against the oracle pool written through the same map."""
    rng = np.random.default_rng(77)
    L, H, D, M, B = 2, 2, 64, 64, 4
    per_slot = M // 16
    perm = rng.permutation(B * per_slot).astype(np.int32)
    g = tl.KVCacheManager(L, H, D, M, B)
    assert g.setBlockMap(16, perm) is None
    o = orc.KVCacheOracle(L, H, D, M, B)
    pool = o.pool()
    phys = (perm // per_slot) * (2 * L * per_slot) + perm % per_slot
    keep = []

    def write(slot, layer, t0, k, v, n):
        for i in range(n):
            t = t0 + i
            pblk = phys[slot * per_slot + t // 16]
            off = layer * 2 * M * H * D + pblk * 16 * H * D + (t % 16) * H * D
            pool[off:off + H * D] = k[i * H * D:(i + 1) * H * D]
            pool[off + M * H * D:off + M * H * D + H * D] = v[i * H * D:(i + 1) * H * D]

    ids = [g.allocateSequence(M)[0] for _ in range(B)]
    assert "paged" in g.getCacheChecked(ids[0], 0)[1]
    for sid in ids:
        n = int(rng.integers(1, 40))
        for layer in range(L):
            k, v = rnd(rng, n * H * D), rnd(rng, n * H * D)
            dk, dv = to_dev(k), to_dev(v)
            keep += [dk, dv]
            assert g.appendKV(sid, layer, dk.data_ptr(), dv.data_ptr(), n, stream()) is None
            write(g.slot_of(sid), layer, 0, k, v, n)
        g.advanceSeqLen(sid, n)
    batch = tl.DecodeBatch(g, B, H)
    batch.prepare(ids, stream())
    nk, nv = rnd(rng, L * B * H * D), rnd(rng, L * B * H * D)
    dk, dv = to_dev(nk), to_dev(nv)
    batch.append(0, L, dk.data_ptr(), dv.data_ptr(), stream())
    for i, sid in enumerate(ids):
        for layer in range(L):
            r = (layer * B + i) * H * D
            write(g.slot_of(sid), layer, g.getSeqLen(sid), nk[r:r + H * D], nv[r:r + H * D], 1)
    assert np.array_equal(read_dev(g.pool(), pool.size), pool)
    assert "no live sequences" in g.setBlockMap(16, perm)


def test_batch_commit_advances_every_sequence(tl):
    """DecodeBatch.commit(n) == advanceSeqLen(seq, n) for every prepared
    sequence (inference_engine.cpp:291), with the reference's clamp and
    error on non-positive n (kv_cache.cpp:240-259)."""
    g = tl.KVCacheManager(1, 2, 64, 64, 4)
    ids = [g.allocateSequence(m)[0] for m in (64, 10, 64)]
    g.advanceSeqLen(ids[1], 9)
    batch = tl.DecodeBatch(g, 4, 2)
    batch.prepare(ids, stream())
    batch.commit(1)
    assert [g.getSeqLen(s) for s in ids] == [1, 10, 1]
    batch.prepare_lengths(ids, [1, 10, 1], stream())
    batch.commit(5)  # clamps at each sequence's max_len
    assert [g.getSeqLen(s) for s in ids] == [6, 10, 6]
    with pytest.raises(tl.TinyLLMError, match="positive"):
        batch.commit(0)
