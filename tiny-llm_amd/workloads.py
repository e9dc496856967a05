"""Synthetic workloads of the five decode configurations (host-side logic).

Shapes follow the benchmark configurations of the KV decode path: one decode
step = append one token per live sequence (per layer) into the cache, then
GQA decode attention over attended = context + 1 tokens.  Seeds are
20261201 + 1000*cfg + stream, stream 0=Q, 1=K, 2=V, 3=lengths, 4=block
permutation, 5=arrival/finish events.  Everything here is deterministic numpy.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEED_BASE = 20261201


def seed(cfg: int, stream: int) -> int:
    return SEED_BASE + 1000 * cfg + stream


@dataclass
class DecodeConfig:
    name: str
    cfg: int
    num_layers: int
    batch: int
    hq: int
    hkv: int
    head_dim: int
    max_seq_len: int
    steps: int
    kv_std: float = 1.0
    q_std: float = 1.0
    block_tokens: int = 0  # 0: reference (slot) layout
    contexts: np.ndarray = field(default=None, repr=False)

    @property
    def group(self) -> int:
        return self.hq // self.hkv

    @property
    def scale(self) -> float:
        return 1.0 / float(np.sqrt(self.head_dim))


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def config(cfg: int, steps: int | None = None) -> DecodeConfig:
    """Configurations 1-4 (5 is the churn simulation, see ChurnSim)."""
    if cfg == 1:
        ctx = np.array([128, 256, 384, 512], dtype=np.int32)
        c = DecodeConfig("cfg1_mha_b4_d64", 1, 1, 4, 8, 8, 64, 528, steps or 1)
    elif cfg == 2:
        rng = np.random.default_rng(seed(2, 3))
        ctx = rng.integers(512, 4097, size=16).astype(np.int32)
        c = DecodeConfig("cfg2_llama2_7b_32L_b16", 2, 32, 16, 32, 32, 128, 0, steps or 3, kv_std=0.5)
        c.max_seq_len = _round_up(int(ctx.max()) + c.steps, 16)
    elif cfg == 3:
        ctx = np.full(64, 8192, dtype=np.int32)
        c = DecodeConfig("cfg3_llama3_8b_gqa_b64_ctx8k", 3, 1, 64, 32, 8, 128, 0, steps or 100)
        c.max_seq_len = max(8448, _round_up(8192 + c.steps + 1, 64))
    elif cfg == 4:
        ctx = lognormal_lengths(128, median=2048, sigma=1.0, lo=1, hi=32768, seed_=seed(4, 3))
        c = DecodeConfig("cfg4_ragged_paged_b128", 4, 1, 128, 32, 8, 128, 0, steps or 3,
                         block_tokens=16)
        c.max_seq_len = _round_up(int(ctx.max()) + c.steps, 64)
    else:
        raise ValueError(f"no fixed-batch configuration {cfg}")
    c.contexts = ctx
    return c


def lognormal_lengths(n, median, sigma, lo, hi, seed_):
    rng = np.random.default_rng(seed_)
    x = np.round(np.exp(rng.normal(np.log(median), sigma, size=n)))
    return np.clip(x, lo, hi).astype(np.int32)


def block_permutation(num_blocks: int, seed_: int) -> np.ndarray:
    """Seeded random permutation of the pool's logical blocks (cfg 4)."""
    return np.random.default_rng(seed_).permutation(num_blocks).astype(np.int32)


def step_bytes(contexts, hq, hkv, d, layers=1, paged_block=0) -> int:
    """Algorithmic HBM bytes of one decode step (append + attention):
    K+V cache read of S_b = ctx_b + 1 tokens, Q read + O write, new K/V read
    + append write, and the block-table / length reads of paged layouts."""
    s = np.asarray(contexts, dtype=np.int64) + 1
    b = s.size
    per_layer = int(s.sum()) * hkv * d * 2 * 2 + 2 * b * hq * d * 2 + 2 * b * hkv * d * 2 * 2
    if paged_block:
        per_layer += 4 * b + 4 * int(((s + paged_block - 1) // paged_block).sum())
    return per_layer * layers


def attention_bytes(contexts, hq, hkv, d) -> int:
    """Algorithmic bytes of the attention kernel alone for one layer:
    K+V read over S_b = ctx_b + 1 tokens, Q read, O write."""
    s = np.asarray(contexts, dtype=np.int64) + 1
    return int(s.sum()) * hkv * d * 4 + 2 * s.size * hq * d * 2


@dataclass
class ChurnEvent:
    step: int
    arrivals: list          # prompt lengths of sequences arriving this step
    lifetimes: list         # decode steps each arrival lives


class ChurnSim:
    """Configuration 5: Poisson(lam) arrivals per step, prompt U{256..4096},
    lifetime Geometric(p) steps (capped so prompt + lifetime <= max_seq_len)."""

    def __init__(self, steps=1000, lam=2.0, p=1.0 / 512, prompt_lo=256, prompt_hi=4096,
                 max_seq_len=5120, slots=1280, hq=64, hkv=8, head_dim=128, seed_=None):
        self.steps, self.lam, self.p = steps, lam, p
        self.prompt_lo, self.prompt_hi = prompt_lo, prompt_hi
        self.max_seq_len, self.slots = max_seq_len, slots
        self.hq, self.hkv, self.head_dim = hq, hkv, head_dim
        self.rng = np.random.default_rng(seed(5, 5) if seed_ is None else seed_)

    def events(self):
        for t in range(self.steps):
            k = int(self.rng.poisson(self.lam))
            prompts = self.rng.integers(self.prompt_lo, self.prompt_hi + 1, size=k).tolist()
            lifes = self.rng.geometric(self.p, size=k).tolist()
            lifes = [min(l, self.max_seq_len - pr) for l, pr in zip(lifes, prompts)]
            yield ChurnEvent(t, prompts, lifes)
