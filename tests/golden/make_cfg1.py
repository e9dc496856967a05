#!/usr/bin/env python3
"""Writes the config-1 golden fixture (cfg1_decode.npz + cfg1_decode.json).

Config 1 of the benchmark set: one layer, batch 4, 8 query / 8 kv heads
(MHA), head_dim 64, contexts 128/256/384/512, fp16 Q/K/V from N(0,1), one
decode step = appendKV(n=1) per sequence then attention over context + 1
tokens with scale 1/8 (the decode branch of TransformerLayer::attention,
src/transformer.cpp:222-237).

Inputs come from the in-repo seeded generator (splitmix64 -> Box-Muller ->
fp16 RNE) with seeds 20261201 + 1000*1 + stream (0 = Q, 1 = K, 2 = V); K and
V of all sequences are drawn as one stream each, the prefill tokens of
sequences 0..3 in order followed by the 4 new tokens.  The fixture stores
the small inputs (Q, new K/V rows), SHA-256 digests of the large ones (the
prefill K/V streams) and of the expected cache pool after the step, and the
expected attention output in fp32 and as fp16 bits.

The expected values are the oracle's (oracle/kv_oracle.c, a restatement of
src/kv_cache.cpp and kernels/attention.cu:11-112); the reference holds no
vectors of its own for this path.  Run from the repository root:
    python3 tests/golden/make_cfg1.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))

CTX = [128, 256, 384, 512]
B, HQ, HKV, D, M, L = 4, 8, 8, 64, 528, 1
SEED = 20261201 + 1000 * 1


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def inputs(orc):
    tokens = sum(CTX) + B
    q = orc.normal_f16(SEED + 0, (B, HQ, D))
    k = orc.normal_f16(SEED + 1, (tokens, HKV * D))
    v = orc.normal_f16(SEED + 2, (tokens, HKV * D))
    return q, k, v


def run_oracle(orc, q, k, v):
    kv = orc.KVCacheOracle(L, HKV, D, M, B)
    ids, off = [], 0
    for c in CTX:
        sid, err = kv.allocate(M)
        assert err is None, err
        assert kv.append(sid, 0, k[off:off + c], v[off:off + c], c) is None
        kv.advance(sid, c)
        off += c
        ids.append(sid)
    for i, sid in enumerate(ids):  # the decode step's append (n = 1)
        assert kv.append(sid, 0, k[off + i], v[off + i], 1) is None
    lens = np.array([c + 1 for c in CTX], dtype=np.int32)
    view = orc.cache_view(kv.pool(), L, HKV, D, M, 0, [kv.slot_of(s) for s in ids])
    o32, o16 = orc.attn_decode_gqa(q, view, lens, HQ, HKV, D, 1.0 / 8.0)
    return kv.pool().copy(), lens, o32, o16


def main():
    import oracle as orc
    orc.build()
    q, k, v = inputs(orc)
    pool, lens, o32, o16 = run_oracle(orc, q, k, v)
    off = sum(CTX)
    np.savez_compressed(os.path.join(HERE, "cfg1_decode.npz"), q=q, new_k=k[off:], new_v=v[off:],
                        lens=lens, out_f32=o32, out_f16=o16)
    meta = {"config": "cfg1_mha_b4_d64", "contexts": CTX, "batch": B, "q_heads": HQ,
            "kv_heads": HKV, "head_dim": D, "max_seq_len": M, "layers": L, "scale": 0.125,
            "seeds": {"q": SEED, "k": SEED + 1, "v": SEED + 2},
            "sha256": {"q": sha(q), "k_stream": sha(k), "v_stream": sha(v), "pool_after_step": sha(pool)}}
    with open(os.path.join(HERE, "cfg1_decode.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("wrote cfg1_decode.npz / cfg1_decode.json")


if __name__ == "__main__":
    main()
