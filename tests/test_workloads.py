"""CPU: the synthetic workload definitions used by bench.py and the tests."""
import numpy as np

import workloads


def test_headline_config_shape_and_bytes():
    c = workloads.config(3)
    assert (c.batch, c.hq, c.hkv, c.head_dim, c.num_layers) == (64, 32, 8, 128, 1)
    assert np.all(c.contexts == 8192) and c.steps == 100
    # step 1: K+V over 8193 tokens + Q/O + append = 2,149,318,656 B
    assert workloads.step_bytes(c.contexts, 32, 8, 128) == 2_149_318_656


def test_config1_and_2():
    c1 = workloads.config(1)
    assert list(c1.contexts) == [128, 256, 384, 512] and c1.head_dim == 64 and c1.group == 1
    c2 = workloads.config(2)
    assert c2.num_layers == 32 and c2.batch == 16 and c2.contexts.min() >= 512
    assert c2.contexts.max() <= 4096 and c2.max_seq_len >= c2.contexts.max() + c2.steps
    assert np.array_equal(c2.contexts, workloads.config(2).contexts)  # seeded


def test_ragged_lengths_and_permutation():
    c4 = workloads.config(4)
    assert c4.batch == 128 and c4.block_tokens == 16
    assert c4.contexts.min() >= 1 and c4.contexts.max() <= 32768
    assert 1200 < np.median(c4.contexts) < 3400
    perm = workloads.block_permutation(1000, workloads.seed(4, 4))
    assert np.array_equal(np.sort(perm), np.arange(1000))


def test_churn_events_respect_capacity():
    sim = workloads.ChurnSim(steps=200)
    total = 0
    for ev in sim.events():
        for p, life in zip(ev.arrivals, ev.lifetimes):
            assert 256 <= p <= 4096 and 1 <= life and p + life <= 5120
        total += len(ev.arrivals)
    assert 300 < total < 500  # Poisson(2) x 200 steps


class _FakeManager:
    """Host stand-in for the library objects ChurnDriver drives: the
    reference's slot allocator (lowest free slot, monotone ids) plus a log of
    every device call."""

    def __init__(self, slots):
        self.free = list(range(slots))
        self.len, self.slot, self.next_id, self.log = {}, {}, 0, []

    def allocateSequence(self, max_len):
        if not self.free:
            return None, "KV cache exhausted"
        self.free.sort()
        sid = self.next_id
        self.next_id += 1
        self.slot[sid] = self.free.pop(0)
        self.len[sid] = 0
        return sid, None

    def releaseSequence(self, sid):
        self.free.append(self.slot.pop(sid))
        del self.len[sid]
        self.log.append(("release", sid))

    def getUsedMemory(self):
        return len(self.slot)

    # PrefillBatch
    def prepare(self, ids, counts, stream=0):
        self._pf = list(zip(ids, counts))

    def append(self, layer, k, v, stream=0):
        self.log.append(("prompts", list(self._pf)))

    def commit(self, n=None):
        if n is None:  # PrefillBatch.commit
            for sid, c in self._pf:
                self.len[sid] += c
        else:          # DecodeBatch.commit
            for sid in self._dec:
                self.len[int(sid)] += n


class _FakeBatch:
    def __init__(self, mgr):
        self.mgr = mgr

    def prepare(self, ids, stream=0):
        self.mgr._dec = [int(s) for s in ids]

    def decode(self, layer, q, nk, nv, out, scale, stream=0):
        self.mgr.log.append(("decode", [(s, self.mgr.len[s]) for s in self.mgr._dec]))

    def commit(self, n):
        self.mgr.commit(n)


def test_churn_driver_replays_events_like_the_reference_engine():
    """ChurnDriver (the benchmark's config-5 step) on host stand-ins: every
    arrival is allocated and its prompt appended from consecutive source rows
    (groups of at most src_rows tokens), every live sequence decodes once per
    step in admission order and grows by one token, and a sequence is
    released exactly when its lifetime ends."""
    M, slots = 5120, 1280
    mgr = _FakeManager(slots)
    batch = _FakeBatch(mgr)
    drv = workloads.ChurnDriver(mgr, batch, mgr, slots=slots, max_seq_len=M, hq=64, hkv=8,
                                head_dim=128, src_rows=6000)
    life, born, order = {}, {}, []
    for ev in workloads.ChurnSim(steps=300).events():
        mgr.log.clear()
        rec = drv.step(ev, 0, q=0, nk=0, nv=0, out=0, scale=1.0, src_k=0, src_v=0, record=True)
        assert [p for _, p, _ in rec.admitted] == ev.arrivals and rec.rejected == 0
        groups = [e[1] for e in mgr.log if e[0] == "prompts"]
        assert [sid for g in groups for sid, _ in g] == [sid for sid, _, _ in rec.admitted]
        for g in groups:
            assert sum(c for _, c in g) <= 6000
        rows = [r for _, _, r in rec.admitted]
        for (sid, p, r), l in zip(rec.admitted, ev.lifetimes):
            life[sid], born[sid] = max(1, l), ev.step
            order.append(sid)
        # source rows: consecutive within a launch group, from row 0
        i = 0
        for g in groups:
            acc = 0
            for sid, c in g:
                assert rows[i] == acc
                acc += c
                i += 1
        live_before = [s for s in order if s in life and born[s] <= ev.step]
        dec = [e[1] for e in mgr.log if e[0] == "decode"]
        if live_before:
            assert len(dec) == 1 and [s for s, _ in dec[0]] == live_before
            assert list(rec.decoded_ids) == live_before
            assert list(rec.decoded_lens) == [ln for _, ln in dec[0]]
        ended = [s for s in live_before if ev.step - born[s] + 1 == life[s]]
        assert sorted(rec.released) == sorted(ended)
        assert [e[1] for e in mgr.log if e[0] == "release"] == rec.released
        for s in ended:
            del life[s]
        order = [s for s in order if s in life]
    ids, lens = drv.live()
    assert list(ids) == order and all(mgr.len[int(s)] == ln for s, ln in zip(ids, lens))
    assert drv.steps == 300 and drv.peak >= len(ids) > 100
