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
