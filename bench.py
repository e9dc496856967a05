#!/usr/bin/env python3
"""Benchmark of the KV-cache decode hot path on one MI355X.

Headline workload: Llama-3-8B-shaped GQA decode, one
layer, 32 query / 8 KV heads, head_dim 128, batch 64, context 8192, fp16 KV
drawn from N(0,1).  A step = the decode branch of TransformerLayer::attention
for the whole batch: DecodeBatch.prepare (host snapshot + one metadata
upload), fused append of one token per sequence, split-K GQA attention over
S = context + 1 tokens, merge, then advanceSeqLen per sequence (host).  Each
timed step appends one token (S: 8193 -> 8192 + steps).  Warm-up steps run
the same kernels without advancing the lengths.

Prints ONE JSON line.  `value` is achieved HBM throughput in GB/s computed
from the algorithmic bytes of each step (K+V cache read of S_b tokens, Q read
+ O write, new K/V read + append write) over the measured step time.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "tiny-llm_amd"))

METRIC = ("decode attn+KV append µs/step and achieved HBM GB/s (% of peak), "
          "8B GQA b64 ctx8k")
HBM_PEAK_GBPS = 8000.0
PMC_SUMMARY = os.path.join(REPO, "profiles", "attn_decode_kernel_cfg3_pmc.txt")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-baseline", dest="cpu_baseline", action="store_true", default=True)
    ap.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU work of the cpu_baseline sample")
    ap.add_argument("--q-heads", type=int, default=0,
                    help="override the number of query heads (64 gives the group-8 head shape of "
                         "the churn configuration on the same batch/context); 0 = config 3's 32")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="only run one device-to-device copy of this many MiB (HBM counter "
                         "calibration for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(cfg, target_s: float):
    """The oracle (C restatement of the reference path) on host cores: a
    bounded sample of the same workload -- 8 of the 64 sequences at full
    context, full decode steps (appendKV + attention + advance)."""
    import numpy as np
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as orc
    import workloads

    nseq, ctx = 8, int(cfg.contexts[0])
    Hkv, Hq, D = cfg.hkv, cfg.hq, cfg.head_dim
    M = ctx + 64
    kv = orc.KVCacheOracle(1, Hkv, D, M, nseq)
    rng = np.random.default_rng(workloads.seed(3, 1))
    ids = []
    for _ in range(nseq):
        sid, _ = kv.allocate(M)
        k = rng.standard_normal(ctx * Hkv * D, dtype=np.float32).astype(np.float16).view(np.uint16)
        v = rng.standard_normal(ctx * Hkv * D, dtype=np.float32).astype(np.float16).view(np.uint16)
        kv.append(sid, 0, k, v, ctx)
        kv.advance(sid, ctx)
        ids.append(sid)
    threads = cpu_threads()
    q = rng.standard_normal((nseq, Hq, D), dtype=np.float32).astype(np.float16).view(np.uint16)
    nk = rng.standard_normal((nseq, Hkv * D), dtype=np.float32).astype(np.float16).view(np.uint16)
    steps, total_bytes, t_used = 0, 0, 0.0
    while t_used < target_s and steps < 64:
        lens = np.array([kv.seq_len(s) + 1 for s in ids])
        t0 = time.perf_counter()
        for i, sid in enumerate(ids):
            kv.append(sid, 0, nk[i], nk[i], 1)
        view = orc.cache_view(kv.pool(), 1, Hkv, D, M, 0, [kv.slot_of(s) for s in ids])
        orc.attn_decode_gqa(q, view, lens, Hq, Hkv, D, cfg.scale, nthreads=threads)
        for sid in ids:
            kv.advance(sid, 1)
        t_used += time.perf_counter() - t0
        total_bytes += workloads.step_bytes(lens - 1, Hq, Hkv, D)
        steps += 1
    return {"value": round(total_bytes / t_used / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle C restatement, {nseq} of {cfg.batch} sequences at context {ctx}, "
                      f"{steps} full decode steps (append+attention), {t_used:.1f} s, "
                      f"{threads} OpenMP threads, cpu={_cpu_model()}"}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def read_pmc(workload: str):
    """HBM bytes per launch of attn_chunk from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, calibrated with a copy kernel)."""
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                line = line.strip()
                if line.startswith("{"):
                    d = json.loads(line)
                    if d.get("workload") == workload:
                        return d.get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the KV decode path is not sharded across GPUs here.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch  # HIP runtime first: one runtime in the process
    if args.calib_copy_mib:
        n = args.calib_copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes": n}))
        return
    import tinyllm_kv as tl
    import workloads

    cfg = workloads.config(3, steps=args.steps)
    if args.q_heads:
        cfg.hq = args.q_heads
        cfg.name += f"_hq{args.q_heads}"
    B, Hq, Hkv, D, ctx0 = cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim, int(cfg.contexts[0])
    M = ((ctx0 + args.steps + 1 + 63) // 64) * 64
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream().cuda_stream

    mgr = tl.KVCacheManager(cfg.num_layers, Hkv, D, M, B)
    gen = torch.Generator(device=dev)
    gen.manual_seed(workloads.seed(3, 1))
    ids = []
    for _ in range(B):  # prefill through appendKV, as InferenceEngine::prefill does
        sid, err = mgr.allocateSequence(M)
        assert err is None, err
        k = torch.randn((ctx0, Hkv * D), generator=gen, device=dev, dtype=torch.float16)
        v = torch.randn((ctx0, Hkv * D), generator=gen, device=dev, dtype=torch.float16)
        assert mgr.appendKV(sid, 0, k.data_ptr(), v.data_ptr(), ctx0, stream) is None
        mgr.advanceSeqLen(sid, ctx0)
        ids.append(sid)
    K = args.steps
    nsteps_in = max(1, K)
    q = torch.randn((nsteps_in, B, Hq, D), generator=gen, device=dev, dtype=torch.float16)
    nk = torch.randn((nsteps_in, B, Hkv * D), generator=gen, device=dev, dtype=torch.float16)
    nv = torch.randn((nsteps_in, B, Hkv * D), generator=gen, device=dev, dtype=torch.float16)
    out = torch.empty((B, Hq, D), device=dev, dtype=torch.float16)
    batch = tl.DecodeBatch(mgr, B, Hq)
    torch.cuda.synchronize()

    def step(i, advance):
        batch.prepare(ids, stream)
        j = i % nsteps_in
        batch.decode(0, q[j].data_ptr(), nk[j].data_ptr(), nv[j].data_ptr(), out.data_ptr(),
                     cfg.scale, stream)
        if advance:
            for sid in ids:
                mgr.advanceSeqLen(sid, 1)

    for i in range(args.warmup):
        step(i, advance=False)
    torch.cuda.synchronize()

    # Timed region: K full steps, no per-kernel hooks (hipEventRecord between
    # kernels inserts markers that widen the inter-kernel gaps).
    ctx_per_step = []
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    ev0.record()
    for i in range(K):
        ctx_per_step.append(mgr.getSeqLen(ids[0]))
        step(i, advance=True)
    ev1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    elapsed_ms = ev0.elapsed_time(ev1)

    # Kernel-timing pass: the same steps (lengths not advanced) with hipEvents
    # around every launch on the launch stream.
    tl.profile_reset()
    tl.profile_enable(True)
    kpass = max(10, min(K, 30))
    for i in range(kpass):
        step(i, advance=False)
    torch.cuda.synchronize()
    tl.profile_enable(False)
    chunk_ms, chunk_n = tl.profile_query("attn_chunk")
    merge_ms, merge_n = tl.profile_query("attn_merge")
    app_ms, app_n = tl.profile_query("kv_append")
    tl.profile_reset()
    ctx_kpass = mgr.getSeqLen(ids[0])

    total_bytes = sum(workloads.step_bytes(np.full(B, c), Hq, Hkv, D) for c in ctx_per_step)
    attn_bytes = [workloads.attention_bytes(np.full(B, ctx_kpass), Hq, Hkv, D)]
    ms_per_step = elapsed_ms / K
    value = total_bytes / (elapsed_ms * 1e-3) / 1e9
    chunk_avg_ms = chunk_ms / max(1, chunk_n)
    achieved = (sum(attn_bytes) / len(attn_bytes)) / (chunk_avg_ms * 1e-3) / 1e9
    traffic = read_pmc(cfg.name)

    sp = tl.get_score_path()
    score_kind = "mfma" if sp == 1 or (sp == 2 and Hq // Hkv >= 8) else "valu"
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "frac_of_peak": round(value / HBM_PEAK_GBPS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: KV and Q from N(0,1) (torch.randn, seeded), prefilled via appendKV",
        "config": {"workload": cfg.name, "layers": 1, "batch": B, "q_heads": Hq, "kv_heads": Hkv,
                   "head_dim": D, "context_start": ctx0, "attended_first": ctx_per_step[0] + 1,
                   "attended_last": ctx_per_step[-1] + 1, "chunk_tokens": batch.info()["chunk_tokens"],
                   "work_items": batch.info()["work_items"],
                   "parallelism": "single GPU"},
        "kernel_timing": f"hipEvent pairs around each launch, separate pass of {kpass} steps at "
                         f"context {ctx_kpass}",
        "kernels_us": {"attn_chunk": round(chunk_avg_ms * 1e3, 2),
                       "attn_merge": round(merge_ms / max(1, merge_n) * 1e3, 2),
                       "kv_append": round(app_ms / max(1, app_n) * 1e3, 2)},
        "host_wall_us_per_step": round(t_wall / K * 1e6, 2),
        "roofline": {"kernel": f"attn_decode_kernel<D={D},G={Hq // Hkv},{score_kind}>",
                     "bound": "hbm",
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic},
        "cpu_baseline": None,
    }
    if args.cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
