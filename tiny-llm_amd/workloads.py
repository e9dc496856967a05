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


def fixed_pool_len(cfg: DecodeConfig, steps: int) -> int:
    """max_seq_len of the benchmark's pool for configurations 1-4: the
    longest context plus `steps` appended tokens and one more, rounded up to
    64 tokens; configuration 3 keeps at least 8448 (8192 + 256 decode
    steps)."""
    m = _round_up(int(cfg.contexts.max()) + steps + 1, 64)
    return max(m, 8448) if cfg.cfg == 3 else m


@dataclass
class ChurnStep:
    """What one ChurnDriver.step did (record=True)."""
    admitted: list          # (seq id, prompt tokens, first source row) in arrival order
    rejected: int           # arrivals refused (no slot / no blocks)
    preempted: list         # seq ids released before the decode for lack of blocks
    decoded_ids: np.ndarray | None   # the decode batch, in batch order
    decoded_lens: np.ndarray | None  # their lengths before this step's token
    released: list          # seq ids that finished after the step


class ChurnDriver:
    """Configuration 5 on the library: replays ChurnSim events over a
    KVCacheManager exactly as the benchmark times them.  Per step:

      * each arrival allocateSequence(max_seq_len); on a block pool it is
        admitted only while the free blocks cover its prompt plus one block
        per live sequence;
      * the admitted prompts' K/V are appended with PrefillBatch
        prepare/append/commit (the bytes of appendKV(seq, 0, rows, prompt) +
        advanceSeqLen per arrival), the arrivals of a step taking
        consecutive source rows from row 0, one launch group per src_rows
        tokens;
      * on a block pool, the newest sequences are released while the blocks
        a step opens (one per sequence at a block boundary) exceed the free
        ones;
      * one decode step over every live sequence in admission order:
        DecodeBatch prepare, decode (fused append of the row of q/nk/nv at
        the entry's batch position + attention), commit(1);
      * sequences whose lifetime ended or whose length reached max_seq_len
        are released.

    mgr / batch / prompts_in are tinyllm_kv objects; the buffers are device
    addresses: src_k/src_v [src_rows][Hkv*D], q [slots][Hq][D], nk/nv
    [slots][Hkv*D], out [slots][Hq][D]."""

    def __init__(self, mgr, batch, prompts_in, *, slots, max_seq_len, hq, hkv, head_dim,
                 src_rows, blocks=False, block_tokens=16):
        self.mgr, self.batch, self.prompts_in = mgr, batch, prompts_in
        self.M, self.hq, self.hkv, self.d = max_seq_len, hq, hkv, head_dim
        self.src_rows, self.blocks, self.bt = src_rows, blocks, block_tokens
        self.ids = np.zeros(slots, dtype=np.int32)
        self.rem = np.zeros(slots, dtype=np.int64)
        self.len = np.zeros(slots, dtype=np.int64)
        self.n = 0
        self.nbytes = self.attn_nbytes = self.rejected = self.preempted = 0
        self.live_sum = self.peak = self.used_sum = self.steps = 0
        self.last_attn_bytes = self.last_decoded = 0

    def _append_prompts(self, new, src_k, src_v, stream):
        rows, i = [], 0
        while i < len(new):
            ids, counts, tok = [], [], 0
            while i < len(new) and tok + new[i][1] <= self.src_rows:
                ids.append(new[i][0])
                counts.append(new[i][1])
                rows.append(tok)
                tok += new[i][1]
                i += 1
            if not ids:
                raise ValueError(f"prompt of {new[i][1]} tokens exceeds {self.src_rows} source rows")
            self.prompts_in.prepare(ids, counts, stream)
            self.prompts_in.append(0, src_k, src_v, stream)
            self.prompts_in.commit()
        return rows

    def step(self, ev, stream, *, q, nk, nv, out, scale, src_k, src_v, record=False):
        mgr, M, bt, n = self.mgr, self.M, self.bt, self.n
        row_bytes = self.hkv * self.d * 2
        new, pending, rejected = [], 0, 0
        for prompt, life in zip(ev.arrivals, ev.lifetimes):
            sid, err = mgr.allocateSequence(M)
            if err is None and self.blocks and mgr.freeBlocks() < pending + -(-prompt // bt) + n:
                mgr.releaseSequence(sid)  # admit only with a block of headroom per live seq
                err = "exhausted"
            if err is not None:
                rejected += 1
                continue
            new.append((sid, prompt))
            pending += -(-prompt // bt)
            self.nbytes += 2 * prompt * row_bytes * 2  # read + write of K and V
            self.ids[n], self.rem[n], self.len[n] = sid, max(1, life), prompt
            n += 1
        rows = self._append_prompts(new, src_k, src_v, stream) if new else []
        preempted = []
        if self.blocks:
            # A step opens a block for every sequence at a block boundary;
            # when the pool cannot back them, the newest sequences are
            # preempted (released) first.
            need = int(np.count_nonzero(self.len[:n] % bt == 0))
            while need > mgr.freeBlocks() and n:
                n -= 1
                need -= int(self.len[n] % bt == 0)
                assert mgr.releaseSequence(int(self.ids[n])) is None
                preempted.append(int(self.ids[n]))
        self.used_sum += mgr.getUsedMemory()
        dec_ids = dec_lens = None
        self.last_attn_bytes = 0
        self.last_decoded = n
        if n:
            self.batch.prepare(self.ids[:n], stream)
            self.batch.decode(0, q, nk, nv, out, scale, stream)
            self.batch.commit(1)
            sb = step_bytes(self.len[:n], self.hq, self.hkv, self.d)
            self.nbytes += sb
            self.attn_nbytes += sb
            self.last_attn_bytes = sb
            if record:
                dec_ids, dec_lens = self.ids[:n].copy(), self.len[:n].copy()
        self.live_sum += n
        self.peak = max(self.peak, n)
        self.rejected += rejected
        self.preempted += len(preempted)
        self.steps += 1
        self.rem[:n] -= 1
        self.len[:n] += 1
        fin = (self.rem[:n] == 0) | (self.len[:n] >= M)
        released = []
        if fin.any():
            released = [int(s) for s in self.ids[:n][fin]]
            for s in released:
                assert mgr.releaseSequence(s) is None
            keep = ~fin
            k = int(np.count_nonzero(keep))
            self.ids[:k], self.rem[:k], self.len[:k] = \
                self.ids[:n][keep], self.rem[:n][keep], self.len[:n][keep]
            n = k
        self.n = n
        if not record:
            return None
        return ChurnStep([(s, p, r) for (s, p), r in zip(new, rows)], rejected, preempted,
                         dec_ids, dec_lens, released)

    def live(self):
        """(seq ids, lengths) of the live sequences in admission order."""
        return self.ids[:self.n].copy(), self.len[:self.n].copy()

    def release_all(self):
        for s in self.ids[:self.n]:
            self.mgr.releaseSequence(int(s))
        self.n = 0
