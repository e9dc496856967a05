#!/usr/bin/env python3
"""Benchmark of the KV-cache decode hot path on one MI355X.

Default (the driver's line) = configuration 3: Llama-3-8B-shaped GQA decode,
one layer, 32 query / 8 KV heads, head_dim 128, batch 64, context 8192, fp16
KV drawn from N(0,1), 100 timed steps.  A step is the decode branch of
TransformerLayer::attention (src/transformer.cpp:222-237) for the whole
batch plus InferenceEngine::decodeStep's commit (inference_engine.cpp:291):
DecodeBatch.prepare (host snapshot + one metadata upload), per layer the
fused append of one token per sequence + split-K GQA attention over
S = context + 1 tokens (+ merge when a sequence spans several chunks), then
advanceSeqLen(seq, 1) for every sequence.  Each timed step appends one token
(S: 8193 -> 8192 + steps); warm-up steps run the same kernels without
advancing the lengths.

--config 2 / 4 / 5 measure the other configurations of the same path
(32-layer MHA; ragged paged batch 128; allocation churn with group 8).

Prints ONE JSON line.  `value` is achieved HBM throughput in GB/s: the
algorithmic bytes of every step (K+V cache read of S_b tokens, Q read + O
write, new K/V read + append write, block-table reads when paged, prompt
appends under churn) over the measured time of the timed steps.
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
CPU_FORM = ("orc_attn_decode_gqa_fast: AVX2/F16C, eight tokens per register for the scores, "
            "eight d for P.V, each K/V row read once per GQA group; the checker's bits")
GEN_NOTE = ("seeded splitmix64 -> Box-Muller -> fp16 streams drawn on the device by "
            "tl_fill_normal_f16, seed 20261201 + 1000*set + stream; the oracle's generator "
            "element for element")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0,
                    help="timed steps (default: 100 for configs 2-4, 1000 for config 5)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=(1, 2, 3, 4, 5),
                    help="1: latency of the small MHA case; 2-4: fixed batches; 5: churn")
    ap.add_argument("--path", default="decode",
                    choices=("decode", "project", "oproj", "prefill", "legacy"),
                    help="decode: append + attention (the headline); legacy: the reference's "
                         "attention_decode entry point at the shape of its own performance table "
                         "(B=1, H=32, D=128, S = 128 / 512 / 2048 / 8192); project: the decode step's "
                         "fused QKV W8A16 projection writing K/V into the cache; oproj: the W8A16 "
                         "o_proj + residual (Llama-3-8B layer shapes, batch 64); prefill: prompt "
                         "tokens appended and attended causally over the cache")
    ap.add_argument("--weights", default="packed", choices=("packed", "reference"),
                    help="project/oproj: int8 weights packed once at load (tl_w8a16_pack), or in the "
                         "reference's row-major [K][N] layout as the drop-in entry points take them")
    ap.add_argument("--prefill-seqs", type=int, default=4, help="prefill: prompts per step")
    ap.add_argument("--prefill-tokens", type=int, default=2048, help="prefill: new tokens per prompt")
    ap.add_argument("--prefill-prefix", type=int, default=0,
                    help="prefill: tokens already cached per prompt (chunked continuation)")
    ap.add_argument("--prefill-heads", default="32,8,128",
                    help="prefill: q heads, kv heads, head_dim (default Llama-3-8B's)")
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="prefill, project, oproj: untimed back-to-back calls for about this "
                         "long before the timed ones, so the kernels are timed at the clock the "
                         "GPU settles at under sustained load (0: off)")
    ap.add_argument("--cpu-baseline", dest="cpu_baseline", action="store_true", default=True)
    ap.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU work of the cpu_baseline sample (at least one full step)")
    ap.add_argument("--q-heads", type=int, default=0,
                    help="override the number of query heads of configs 2-4 (64 on config 3 "
                         "gives the group-8 head shape of config 5 at batch 64 / context 8192)")
    ap.add_argument("--alloc", default="slots", choices=("slots", "blocks"),
                    help="pool of configs 2, 3 and 5: slots = the reference's full-length slot "
                         "per sequence; blocks = blocks handed out as sequences grow")
    ap.add_argument("--block-tokens", type=int, default=16, help="tokens per block of --alloc blocks")
    ap.add_argument("--kv-gib", type=float, default=0.0,
                    help="config 5: HBM budget of the KV pool in GiB (default: 1280 full slots)")
    ap.add_argument("--max-seq-len", type=int, default=0,
                    help="configs 1-4: max_seq_len of the pool (default: the context plus the "
                         "appended steps, rounded up to 64 tokens)")
    ap.add_argument("--launch-log", default="",
                    help="append the algorithmic bytes of every decode attention launch (fused "
                         "append included), in launch order, as JSON lines to this file "
                         "(profiling runs: matched against rocprofv3 --pmc dispatches)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="only run one device-to-device copy of this many MiB (HBM counter "
                         "calibration for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


def cpu_counts():
    """(CPUs this process may run on, OpenMP threads the CPU baseline uses).
    A one-GPU box allots 16 host CPUs to the job, so at most 16 threads run
    whatever the affinity mask shows."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return n, max(1, min(16, n))


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def d2h(dst_ptr: int, src_ptr: int, nbytes: int):
    """hipMemcpy device -> host (the caller synchronised the device)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    rc = hip.hipMemcpy(dst_ptr, src_ptr, nbytes, 2)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy D2H failed: {rc}")


def host_bits(t):
    """fp16 device tensor -> numpy uint16 bit patterns."""
    import numpy as np
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def cpu_baseline_fixed(st, target_s: float):
    """The oracle (the C restatement of the reference's path) on the host
    cores, on the inputs the GPU run ended with: the device pool is copied
    byte for byte into the oracle's pool (same layout), then full-batch decode
    steps run -- per layer the step's K/V row of every sequence written at its
    tail (appendKV), attention of every sequence over its cache, then
    advanceSeqLen -- until target_s of work (at least one step, at most what
    the pool's max_seq_len leaves)."""
    import numpy as np
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as orc
    import workloads

    build = orc.use_native_build()
    mgr, ids, L, Hq, Hkv, D, M = st["mgr"], st["ids"], st["L"], st["Hq"], st["Hkv"], st["D"], st["M"]
    B = len(ids)
    o = orc.KVCacheOracle(L, Hkv, D, M, B)
    oids = [o.allocate(M)[0] for _ in ids]
    assert [o.slot_of(x) for x in oids] == [mgr.slot_of(x) for x in ids]
    st["torch"].cuda.synchronize()
    pool = o.pool()
    d2h(pool.ctypes.data, mgr.pool(), pool.nbytes)
    lens = np.array([mgr.getSeqLen(x) for x in ids], dtype=np.int64)
    for x, n in zip(oids, lens):
        assert o.advance(x, int(n)) is None
    qh = [host_bits(st["q"][layer]) for layer in range(L)]
    nkh = [host_bits(st["nk"][layer]) for layer in range(L)]
    nvh = [host_bits(st["nv"][layer]) for layer in range(L)]
    row, kvpl = Hkv * D, Hkv * M * D
    bs = st["block_tokens"]
    if bs:  # block map over the slot pool: the GPU's physical blocks
        bt = np.array([mgr.blockTable(x)[0] for x in ids], dtype=np.int32)
        lg = bs.bit_length() - 1
        views = [orc.paged_view(pool, L, Hkv, D, M, layer, bt, lg) for layer in range(L)]
    else:
        slots = [o.slot_of(x) for x in oids]
        views = [orc.cache_view(pool, L, Hkv, D, M, layer, slots) for layer in range(L)]
    nproc, threads = cpu_counts()
    room = int(M - lens.max())
    steps, total_bytes, t_used = 0, 0, 0.0
    while steps < room and (steps == 0 or t_used < target_s):
        t0 = time.perf_counter()
        for layer in range(L):
            for i, x in enumerate(oids):
                if bs:
                    t = int(lens[i])
                    e = layer * 2 * kvpl + int(bt[i, t >> lg]) * bs * row + (t & (bs - 1)) * row
                    pool[e:e + row] = nkh[layer][i]
                    pool[e + kvpl:e + kvpl + row] = nvh[layer][i]
                else:
                    o.append(x, layer, nkh[layer][i], nvh[layer][i], 1)
            orc.attn_decode_gqa(qh[layer], views[layer], lens + 1, Hq, Hkv, D, st["scale"],
                                nthreads=threads, fast=True)
        for x in oids:
            o.advance(x, 1)
        t_used += time.perf_counter() - t0
        total_bytes += workloads.step_bytes(lens, Hq, Hkv, D, layers=L, paged_block=bs)
        lens += 1
        steps += 1
    return {"value": round(total_bytes / t_used / 1e9, 3), "unit": "GB/s",
            "us_per_step": round(t_used / steps * 1e6, 1), "cores": threads, "kind": "port",
            "sample": f"oracle C restatement ({CPU_FORM}; {build}) on the GPU run's final cache "
                      f"(copied byte for byte), full batch of {B} sequences x {L} layer(s), "
                      f"{steps} decode steps (append + attention + advance), {t_used:.1f} s, "
                      f"{threads} OpenMP threads of {nproc} CPUs in the affinity mask, "
                      f"cpu={_cpu_model()}"}


def cpu_baseline_churn(st, target_s: float):
    """Configuration 5 on the host cores: the oracle replays the same
    seeded event sequence on the reference's slot allocator -- every arrival
    allocated and its prompt appended (the same source rows as the GPU run),
    every finished sequence released -- and runs full decode steps
    (append + attention over every live sequence + advance) on evenly spaced
    steps until target_s of attention work; the other steps advance the
    bookkeeping only.  value = bytes of the sampled decode steps / their
    time."""
    import numpy as np
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as orc
    import workloads

    build = orc.use_native_build()
    K, M, slots, Hq, Hkv, D = st["K"], st["M"], st["slots"], st["Hq"], st["Hkv"], st["D"]
    o = orc.KVCacheOracle(1, Hkv, D, M, slots)
    sim = workloads.ChurnSim(steps=K, hq=Hq, hkv=Hkv, head_dim=D, max_seq_len=M, slots=slots)
    nproc, threads = cpu_counts()
    every = max(1, K // 20)
    live, length = {}, {}
    t_book, t_dec, dec_bytes, dec_steps, live_sampled = 0.0, 0.0, 0, 0, 0
    for ev in sim.events():
        t0 = time.perf_counter()
        row = 0  # a step's arrivals take consecutive source rows, as on the GPU
        for prompt, life in zip(ev.arrivals, ev.lifetimes):
            sid, err = o.allocate(M)
            if err is not None:
                continue
            if row + prompt > len(st["src_k"]):
                row = 0
            o.append(sid, 0, st["src_k"][row:row + prompt], st["src_v"][row:row + prompt], prompt)
            row += prompt
            o.advance(sid, prompt)
            live[sid] = max(1, life)
            length[sid] = prompt
        ids = list(live)
        t_book += time.perf_counter() - t0
        sample = ids and ev.step % every == every - 1 and (dec_steps == 0 or t_dec < target_s)
        t0 = time.perf_counter()
        for i, sid in enumerate(ids):
            o.append(sid, 0, st["nk"][i], st["nv"][i], 1)
        if sample:
            lens = np.fromiter((length[x] + 1 for x in ids), dtype=np.int64, count=len(ids))
            view = orc.cache_view(o.pool(), 1, Hkv, D, M, 0, [o.slot_of(x) for x in ids])
            orc.attn_decode_gqa(st["q"][:len(ids)], view, lens, Hq, Hkv, D, st["scale"],
                                nthreads=threads, fast=True)
        for sid in ids:
            o.advance(sid, 1)
            live[sid] -= 1
            length[sid] += 1
            if live[sid] == 0 or length[sid] >= M:
                del live[sid]
                del length[sid]
                o.release(sid)
        dt = time.perf_counter() - t0
        if sample:
            t_dec += dt
            dec_bytes += workloads.step_bytes(lens - 1, Hq, Hkv, D)
            dec_steps += 1
            live_sampled += len(ids)
        else:
            t_book += dt
    return {"value": round(dec_bytes / t_dec / 1e9, 3) if t_dec else None, "unit": "GB/s",
            "us_per_step": round(t_dec / max(1, dec_steps) * 1e6, 1), "cores": threads,
            "kind": "port",
            "sample": f"oracle C restatement ({CPU_FORM}; {build}) replaying the same {K}-step "
                      f"event sequence on the "
                      f"reference's slot allocator: {dec_steps} full decode steps (every {every}th "
                      f"step, {live_sampled / max(1, dec_steps):.0f} live sequences on average) "
                      f"timed, {t_dec:.1f} s; bookkeeping, prompt and token appends of all steps "
                      f"{t_book:.1f} s (not in value); {threads} OpenMP threads of {nproc} CPUs, "
                      f"cpu={_cpu_model()}"}


def log_launches(path: str, n: int, nbytes: int, seqs: int):
    with open(path, "a") as f:
        for _ in range(n):
            f.write(json.dumps({"attn_bytes": int(nbytes), "seqs": int(seqs)}) + "\n")


def read_pmc(workload: str):
    """HBM bytes per launch of attn_decode_kernel for this workload from a
    committed rocprofv3 --pmc summary (profiles/attn_decode_kernel_*_pmc.txt:
    FETCH_SIZE + WRITE_SIZE, calibrated with a copy kernel) and the file it
    came from, or (None, None) when no summary covers the workload.  The
    counters cannot be read from inside this process, so the figure is the
    profile's, not this run's."""
    import glob
    for path in sorted(glob.glob(os.path.join(REPO, "profiles", "attn_decode_kernel_*_pmc.txt"))):
        try:
            with open(path) as f:
                for line in f:
                    line = line.strip()
                    if line.startswith("{"):
                        d = json.loads(line)
                        if d.get("workload") == workload and "traffic_bytes_per_launch" in d:
                            return d["traffic_bytes_per_launch"], os.path.relpath(path, REPO)
        except (OSError, ValueError):
            continue
    return None, None


def kernel_stats(tl):
    out = {}
    for k in ("attn_chunk", "attn_merge", "kv_append"):
        ms, n = tl.profile_query(k)
        out[k] = (ms, n)
    return out


def fixed_batch(args, tl, torch, workloads, np):
    """Configurations 1-4: a fixed batch prefilled through appendKV, then K
    decode steps over every layer."""
    cfg = workloads.config(args.config)
    if args.q_heads:
        cfg.hq = args.q_heads
        cfg.name += f"_hq{args.q_heads}"
    K = args.steps or 100
    B, Hq, Hkv, D, L = cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim, cfg.num_layers
    ctx = cfg.contexts.astype(np.int64)
    bt = cfg.block_tokens
    M = workloads.fixed_pool_len(cfg, K)  # the parity tests build the same pool
    if args.max_seq_len:
        if args.max_seq_len < ctx.max() + K + 1 or (bt and args.max_seq_len % bt):
            raise SystemExit(f"--max-seq-len {args.max_seq_len} cannot hold the context and "
                             f"{K} steps" + (f" in {bt}-token blocks" if bt else ""))
        M = args.max_seq_len
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream().cuda_stream

    blocks = args.alloc == "blocks" and not bt
    if blocks:  # every sequence's blocks, in the order the prefill and steps take them
        bb = args.block_tokens
        need = int(((ctx + K + args.warmup + 1 + bb - 1) // bb).sum())
        mgr = tl.KVCacheManager(L, Hkv, D, M, B, block_tokens=bb, num_blocks=need)
    else:
        mgr = tl.KVCacheManager(L, Hkv, D, M, B)
    if bt:  # config 4: 16-token blocks behind a seeded random permutation
        perm = workloads.block_permutation(B * M // bt, workloads.seed(cfg.cfg, 4))
        assert mgr.setBlockMap(bt, perm) is None
    ns = tl.NormalStreams(stream)  # seeded device streams: Q 0, K 1, V 2 (workloads.seed)
    s_q, s_k, s_v = (workloads.seed(cfg.cfg, i) for i in range(3))
    ids = []
    for b in range(B):  # prefill through appendKV, as InferenceEngine::prefill does
        sid, err = mgr.allocateSequence(M)
        assert err is None, err
        c = int(ctx[b])
        for layer in range(L):
            k = ns.draw(s_k, (c, Hkv * D), cfg.kv_std)
            v = ns.draw(s_v, (c, Hkv * D), cfg.kv_std)
            assert mgr.appendKV(sid, layer, k.data_ptr(), v.data_ptr(), c, stream) is None
        mgr.advanceSeqLen(sid, c)
        ids.append(sid)
    q = ns.draw(s_q, (L, B, Hq, D), cfg.q_std)
    nk = ns.draw(s_k, (L, B, Hkv * D), cfg.kv_std)  # the K / V streams continue
    nv = ns.draw(s_v, (L, B, Hkv * D), cfg.kv_std)
    out = torch.empty((B, Hq, D), device=dev, dtype=torch.float16)
    batch = tl.DecodeBatch(mgr, B, Hq)
    torch.cuda.synchronize()

    paged_block = bt or (args.block_tokens if blocks else 0)

    def step(advance):
        batch.prepare(ids, stream)
        if args.launch_log:
            att = np.array([mgr.getSeqLen(s) for s in ids], dtype=np.int64)
            log_launches(args.launch_log, L, workloads.step_bytes(att, Hq, Hkv, D, 1, paged_block),
                         B)
        for layer in range(L):
            batch.decode(layer, q[layer].data_ptr(), nk[layer].data_ptr(), nv[layer].data_ptr(),
                         out.data_ptr(), cfg.scale, stream)
        if advance:
            batch.commit(1)

    for _ in range(args.warmup):
        step(advance=False)
    torch.cuda.synchronize()

    # Timed region: K full steps, no per-kernel hooks (hipEventRecord between
    # kernels inserts markers that widen the inter-kernel gaps).
    lens0 = np.array([mgr.getSeqLen(s) for s in ids], dtype=np.int64)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    ev0.record()
    for _ in range(K):
        step(advance=True)
    ev1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    elapsed_ms = ev0.elapsed_time(ev1)
    info = batch.info()
    # kv heads per attention workgroup of the last timed step's plan (1: per
    # head; 2, 4, 8: head-fused), as the library's planner makes it
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    att_last = np.array([mgr.getSeqLen(s) + 1 for s in ids], dtype=np.int32)
    plan = tl.attn_plan(att_last, Hkv, num_cus=cus, head_fuse="current", head_dim=D)
    heads_per_wg = plan["head_fused"] or 1
    fused_items = ("chunks" if plan["fused_chunked"] else "interleaved tiles") if plan["head_fused"] else None

    # The plan of every timed step, for that step's attended lengths (ragged
    # plans can change as the lengths grow): {plan: steps}.
    def plan_name(p):
        return (f"chunk {p['chunk_tokens']}, {p['work_items']} items, "
                + (f"{p['head_fused']} kv heads per workgroup" if p["head_fused"] else "per head")
                + (", merge" if p["any_multi"] else ""))
    step_plans = {}
    for i in range(K):
        p_i = tl.attn_plan((lens0 + i + 1).astype(np.int32), Hkv, num_cus=cus, head_fuse="current",
                           head_dim=D, with_rows=False)
        step_plans[plan_name(p_i)] = step_plans.get(plan_name(p_i), 0) + 1

    # Per-step pass: the same steps (lengths not advanced) with one event
    # between consecutive steps, for the spread of the step time.
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    evs[0].record()
    for i in range(K):
        step(advance=False)
        evs[i + 1].record()
    torch.cuda.synchronize()
    per_step = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(K)]) * 1e3

    # Kernel-timing pass: the same steps (lengths not advanced) with hipEvents
    # around every launch on the launch stream.
    tl.profile_reset()
    tl.profile_enable(True)
    kpass = max(10, min(K, 30))
    for _ in range(kpass):
        step(advance=False)
    torch.cuda.synchronize()
    tl.profile_enable(False)
    ks = kernel_stats(tl)
    tl.profile_reset()
    lens_k = np.array([mgr.getSeqLen(s) for s in ids], dtype=np.int64)

    total_bytes = sum(workloads.step_bytes(lens0 + i, Hq, Hkv, D, layers=L,
                                           paged_block=bt or (args.block_tokens if blocks else 0))
                      for i in range(K))
    attn_bytes = workloads.attention_bytes(lens_k, Hq, Hkv, D)
    if bt or blocks:
        b_ = bt or args.block_tokens
        attn_bytes += 4 * B + 4 * int(((lens_k + 1 + b_ - 1) // b_).sum())
    conf = {"workload": cfg.name, "layers": L, "batch": B, "q_heads": Hq, "kv_heads": Hkv,
            "max_seq_len": M,
            "head_dim": D, "context_first": int(lens0.min()), "context_max_first": int(lens0.max()),
            "context_sum_first": int(lens0.sum()),
            "block_tokens": args.block_tokens if blocks else bt, "kv_std": cfg.kv_std,
            "alloc": "blocks" if blocks else ("permuted blocks" if bt else "full-length slots"),
            "chunk_tokens": info["chunk_tokens"], "work_items": info["work_items"],
            "kv_heads_per_workgroup": heads_per_wg, "head_fused_items": fused_items,
            "timed_step_plans": step_plans,
            "parallelism": "single GPU"}
    data = (f"synthetic: KV ~ N(0,1)*{cfg.kv_std}, Q ~ N(0,1) ({GEN_NOTE}), prefilled "
            f"via appendKV" + (", 16-token blocks behind a seeded random permutation" if bt else ""))
    cpu = None
    if args.cpu_baseline and not blocks:
        cpu = cpu_baseline_fixed(dict(mgr=mgr, ids=ids, L=L, Hq=Hq, Hkv=Hkv, D=D, M=M, q=q, nk=nk,
                                      nv=nv, block_tokens=bt, scale=cfg.scale, torch=torch),
                                 args.cpu_seconds)
    return dict(cfg=cfg, K=K, elapsed_ms=elapsed_ms, t_wall=t_wall, total_bytes=total_bytes,
                attn_bytes=attn_bytes, ks=ks, kpass=kpass, conf=conf, data=data,
                per_step_us=per_step, cpu=cpu,
                kpass_desc=f"separate pass of {kpass} steps (lengths not advanced)")


def churn(args, tl, torch, workloads, np):
    """Configuration 5: Poisson(2) arrivals per step (prompt U{256..4096}
    appended through appendKV), geometric(1/512) lifetimes, release on
    finish; every step appends one token to and attends over every live
    sequence (64 q / 8 kv heads, D=128).  Run twice with the same seed: once
    timed without hooks, once with per-launch hipEvents."""
    K = args.steps or 1000
    sim_args = dict(steps=K)
    Hq, Hkv, D, M, slots, bt = 64, 8, 128, 5120, 1280, args.block_tokens
    slot_bytes = M * Hkv * D * 2 * 2
    budget = int(args.kv_gib * (1 << 30)) if args.kv_gib else slots * slot_bytes
    blocks = args.alloc == "blocks"
    if blocks:
        nblocks = budget // (bt * Hkv * D * 2 * 2)
    else:
        slots = min(slots, budget // slot_bytes)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream().cuda_stream
    ns = tl.NormalStreams(stream)  # seeded device streams: Q 0, K 1, V 2 (workloads.seed)
    s_q, s_k, s_v = (workloads.seed(5, i) for i in range(3))
    # prompt K/V: a step's arrivals take consecutive rows of these, from row 0
    src_rows = 32768
    src_k = ns.draw(s_k, (src_rows, Hkv * D))
    src_v = ns.draw(s_v, (src_rows, Hkv * D))
    q = ns.draw(s_q, (slots, Hq, D))
    nk = ns.draw(s_k, (slots, Hkv * D))
    nv = ns.draw(s_v, (slots, Hkv * D))
    out = torch.empty((slots, Hq, D), device=dev, dtype=torch.float16)
    scale = 1.0 / float(np.sqrt(D))
    if blocks:
        mgr = tl.KVCacheManager(1, Hkv, D, M, slots, block_tokens=bt, num_blocks=nblocks)
    else:
        mgr = tl.KVCacheManager(1, Hkv, D, M, slots)
    batch = tl.DecodeBatch(mgr, slots, Hq)
    prompts_in = tl.PrefillBatch(mgr, slots, Hq)  # the batched append of a step's prompts
    bufs = dict(q=q.data_ptr(), nk=nk.data_ptr(), nv=nv.data_ptr(), out=out.data_ptr(),
                scale=scale, src_k=src_k.data_ptr(), src_v=src_v.data_ptr())

    def run(profile):
        sim = workloads.ChurnSim(hq=Hq, hkv=Hkv, head_dim=D, max_seq_len=M, slots=slots, **sim_args)
        events = list(sim.events())  # drawn before the clock starts
        # the step logic the parity tests replay (workloads.ChurnDriver)
        drv = workloads.ChurnDriver(mgr, batch, prompts_in, slots=slots, max_seq_len=M, hq=Hq,
                                    hkv=Hkv, head_dim=D, src_rows=src_rows, blocks=blocks,
                                    block_tokens=bt)
        if profile:
            tl.profile_reset()
            tl.profile_enable(True)
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record()
        step_ev = []
        for ev in events:
            if profile:
                e = torch.cuda.Event(enable_timing=True)
                e.record()
                step_ev.append(e)
            drv.step(ev, stream, **bufs)
            if args.launch_log and drv.last_attn_bytes:
                log_launches(args.launch_log, 1, drv.last_attn_bytes, drv.last_decoded)
        ev1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = ev0.elapsed_time(ev1)
        per_step = None
        if profile and step_ev:
            step_ev.append(ev1)
            per_step = np.array([step_ev[i].elapsed_time(step_ev[i + 1])
                                 for i in range(len(step_ev) - 1)]) * 1e3
        drv.release_all()
        ks = None
        if profile:
            tl.profile_enable(False)
            ks = kernel_stats(tl)
            tl.profile_reset()
        return dict(ms=ms, wall=wall, nbytes=drv.nbytes, attn_nbytes=drv.attn_nbytes,
                    rejected=drv.rejected, per_step=per_step, preempted=drv.preempted,
                    used_avg=drv.used_sum / sim.steps, live_avg=drv.live_sum / sim.steps,
                    live_peak=drv.peak, ks=ks)

    for _ in range(1 if args.warmup else 0):  # one short untimed pass warms the kernels
        sim_args["steps"] = min(K, 50)
        run(profile=False)
    sim_args["steps"] = K
    timed = run(profile=False)
    prof = run(profile=True)
    ks = prof["ks"]
    # algorithmic bytes of the average attention launch (fused append
    # included, prompt appends excluded) over the profiled pass
    launches = max(1, ks["attn_chunk"][1])
    conf = {"workload": "cfg5_churn_g8" + ("_blocks" if blocks else ""), "layers": 1, "q_heads": Hq, "kv_heads": Hkv,
            "head_dim": D, "max_seq_len": M, "slots": slots, "arrivals_per_step": 2.0,
            "prompt": "U{256..4096}", "lifetime": "geometric(1/512)",
            "live_avg": round(timed["live_avg"], 1), "live_peak": timed["live_peak"],
            "rejected": timed["rejected"], "parallelism": "single GPU",
            "alloc": f"blocks of {bt} tokens" if blocks else "full-length slots",
            "kv_pool_gib": round(budget / (1 << 30), 2),
            "kv_used_avg_gib": round(timed["used_avg"] / (1 << 30), 2)}
    if blocks:
        conf["preempted"] = timed["preempted"]
    cpu = None
    if args.cpu_baseline:
        cpu = cpu_baseline_churn(dict(K=K, M=M, slots=slots, Hq=Hq, Hkv=Hkv, D=D, scale=scale,
                                      src_k=host_bits(src_k), src_v=host_bits(src_v),
                                      q=host_bits(q), nk=host_bits(nk), nv=host_bits(nv)),
                                 args.cpu_seconds)
    return dict(cfg=None, K=K, elapsed_ms=timed["ms"], t_wall=timed["wall"],
                total_bytes=timed["nbytes"], attn_bytes=prof["attn_nbytes"] / launches, ks=ks,
                kpass=K, conf=conf, per_step_us=prof["per_step"], cpu=cpu,
                data=f"synthetic: KV/Q ~ N(0,1) ({GEN_NOTE}); Poisson/uniform/geometric "
                     "events from the seeded simulator",
                kpass_desc=f"second run of the same {K}-step event sequence")


def prefill_bench(args, tl, torch, np):
    """Prefill into the cache at Llama-3-8B attention shapes (32 q / 8 kv
    heads, head_dim 128; --prefill-heads for others): --prefill-seqs prompts of --prefill-tokens new tokens
    on top of --prefill-prefix cached ones, one layer.  A step is
    PrefillBatch.prepare + run: one launch that attends every new token
    causally over its sequence's cache (keys at or past the write position
    read from the new K/V rows) and writes the new rows into the cache (the
    append).  The cache is
    rewound after each step (lengths are not committed), so every step
    repeats the same work."""
    import workloads
    Hq, Hkv, D = (int(x) for x in args.prefill_heads.split(","))
    nseq, n, p0 = args.prefill_seqs, args.prefill_tokens, args.prefill_prefix
    heads_tag = "" if (Hq, Hkv, D) == (32, 8, 128) else f"_h{Hq}x{Hkv}d{D}"
    K = args.steps or 20
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream().cuda_stream
    ns = tl.NormalStreams(stream)
    s_q, s_k, s_v = (workloads.seed(7, i) for i in range(3))  # prefill: stream set 7
    M = ((p0 + n + 63) // 64) * 64
    mgr = tl.KVCacheManager(1, Hkv, D, M, nseq)
    ids = [mgr.allocateSequence(M)[0] for _ in range(nseq)]
    if p0:
        pk = ns.draw(s_k, (p0, Hkv * D))
        for sid in ids:
            assert mgr.appendKV(sid, 0, pk.data_ptr(), pk.data_ptr(), p0, stream) is None
            mgr.advanceSeqLen(sid, p0)
    T = nseq * n
    # the workgroup size the planner takes for this launch (prefill_waves)
    waves = tl.prefill_plan_waves([p0] * nseq, [n] * nseq, Hq, Hkv, D)
    q = ns.draw(s_q, (T, Hq, D))
    nk = ns.draw(s_k, (T, Hkv * D))
    nv = ns.draw(s_v, (T, Hkv * D))
    out = torch.empty((T, Hq, D), device=dev, dtype=torch.float16)
    pb = tl.PrefillBatch(mgr, nseq, Hq)
    scale = 1.0 / float(np.sqrt(D))

    def call():
        pb.prepare(ids, [n] * nseq, stream)
        pb.run(0, q.data_ptr(), nk.data_ptr(), nv.data_ptr(), out.data_ptr(), scale, stream)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    # The kernel is MFMA-bound, so its time follows the shader clock, which
    # under sustained load ramps for tens of milliseconds (on the box: about
    # 1.85 to 2.2 GHz over the first ~50 ms, the cycle count per launch
    # unchanged).  Settle before timing: back-to-back steps, untimed.
    settle_calls, t_settle = 0, time.perf_counter()
    while args.settle_ms > 0 and (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for _ in range(8):
            call()
        settle_calls += 8
        torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    ev0.record()
    for _ in range(K):
        call()
    ev1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    ms = ev0.elapsed_time(ev1) / K
    tl.profile_reset()
    tl.profile_enable(True)
    for _ in range(min(K, 10)):
        call()
    torch.cuda.synchronize()
    tl.profile_enable(False)
    a_ms, a_n = tl.profile_query("attn_prefill")
    c_ms, c_n = tl.profile_query("kv_append")
    tl.profile_reset()
    a_avg, c_avg = a_ms / max(1, a_n), c_ms / max(1, c_n)
    # causal attention FLOPs: QK^T and PV, 2 flops per multiply-add, query j
    # of a prompt attending p0 + j + 1 keys
    keys = nseq * (n * p0 + n * (n + 1) // 2)
    flops = 4.0 * D * Hq * keys
    tflops = flops / (a_avg * 1e-3) / 1e12
    peak = 2500.0
    return {
        "metric": "prefill attention TFLOP/s (causal GQA over the cache), Llama-3-8B heads",
        "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
        "settle": {"ms": args.settle_ms, "steps": settle_calls,
                   "why": "untimed back-to-back steps after the warm-up: the MFMA-bound kernel "
                          "follows the shader clock, which ramps under sustained load"},
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": f"synthetic: Q/K/V ~ N(0,1) ({GEN_NOTE})",
        "config": {"workload": f"llama3_8b_prefill_{nseq}x{n}" + (f"_prefix{p0}" if p0 else "") + heads_tag,
                   "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "prompts": nseq,
                   "new_tokens": n, "cached_prefix": p0, "attended_keys": keys,
                   "workgroup_waves": waves},
        "kernels_us": {"attn_prefill": round(a_avg * 1e3, 2), "kv_append": round(c_avg * 1e3, 2)},
        "host_wall_us_per_step": round(t_wall / K * 1e6, 2),
        "roofline": {"kernel": f"attn_prefill_kernel<{D},{Hq // Hkv},contiguous,{waves} waves>", "bound": "mfma",
                     "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4), "traffic": None},
        "cpu_baseline": None,
    }


def legacy_bench(args, tl, torch, np):
    """attention_decode (kernels/attention.cuh:15-18), the call an unchanged
    TransformerLayer::attention makes (src/transformer.cpp:236-237), at the
    shape the reference's own performance table quotes: B=1, H=32, D=128,
    S in {128, 512, 2048, 8192} (docs/en/performance/benchmarks.md:60-69),
    compact [B][H][S][D] K/V.  Two timings per S, K calls each, back to back:
    `cold` rotates over copies of Q/K/V whose total exceeds 1 GiB, so every
    call streams its K/V from HBM (the headline form); `hot` repeats one
    copy, whose K/V (at most 134 MB) then stays in the 256 MB MALL.  `value`
    is the cold µs per call at S = 8192."""
    import workloads
    B, H, D = 1, 32, 128
    seq_lens = (128, 512, 2048, 8192)
    published_us = {128: 24.0, 512: 52.0, 2048: 180.0, 8192: 680.0}  # RTX A6000, reference docs
    K = args.steps or 200
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream().cuda_stream
    ns = tl.NormalStreams(stream)
    s_q, s_k, s_v = (workloads.seed(6, i) for i in range(3))  # legacy: stream set 6
    scale = 1.0 / float(np.sqrt(D))
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    rows, cpu_rows = [], []
    for S in seq_lens:
        kv_bytes = 2 * B * H * S * D * 2
        nbytes = kv_bytes + 2 * B * H * D * 2  # K + V read, Q read, O write
        R = max(2, min(256, -(-(1 << 30) // kv_bytes)))
        kc = ns.draw(s_k, (R, B, H, S, D))
        vc = ns.draw(s_v, (R, B, H, S, D))
        qc = ns.draw(s_q, (R, B, H, D))
        out = torch.empty((B, H, D), device=dev, dtype=torch.float16)

        def call(i):
            tl.attention_decode(qc[i].data_ptr(), kc[i].data_ptr(), vc[i].data_ptr(), out.data_ptr(),
                                scale, B, H, S, D, stream)

        def timed(rotate):
            for i in range(args.warmup):
                call(i % R if rotate else 0)
            torch.cuda.synchronize()
            torch.cuda._sleep(50_000_000)  # the host queues every call meanwhile
            ev0.record()
            for i in range(K):
                call(i % R if rotate else 0)
            ev1.record()
            torch.cuda.synchronize()
            return ev0.elapsed_time(ev1) / K * 1e3
        cold_us, hot_us = timed(True), timed(False)
        tl.profile_reset()
        tl.profile_enable(True)
        for i in range(min(K, 50)):
            call(i % R)
        torch.cuda.synchronize()
        tl.profile_enable(False)
        c_ms, c_n = tl.profile_query("attn_chunk")
        m_ms, m_n = tl.profile_query("attn_merge")
        tl.profile_reset()
        k_us = c_ms / max(1, c_n) * 1e3
        rows.append({"seq_len": S, "cold_us": round(cold_us, 2), "hot_us": round(hot_us, 2),
                     "cold_gbps": round(nbytes / (cold_us * 1e-6) / 1e9, 1),
                     "cold_frac": round(nbytes / (cold_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                     "kernel_us": round(k_us, 2),
                     "merge_us": round(m_ms / max(1, m_n) * 1e3, 2), "merge_launches": m_n,
                     "bytes": nbytes, "reference_published_us": published_us[S]})
        if args.cpu_baseline:
            cpu_rows.append(cpu_baseline_legacy(qc[0], kc[0], vc[0], B, H, S, D, scale, torch))
        del kc, vc, qc
    last = rows[-1]
    k_gbps = last["bytes"] / (last["kernel_us"] * 1e-6) / 1e9
    cpu = None
    if cpu_rows:
        c = cpu_rows[-1]
        cpu = {"value": c["gbps"], "unit": "GB/s", "cores": c["threads"], "kind": "port",
               "us_per_call": c["us"], "per_seq_len": cpu_rows,
               "sample": f"oracle C restatement of attention_decode ({CPU_FORM}, built with gcc "
                         f"-O3 -march=native on this host) on copy 0 of each S, "
                         f"cpu={_cpu_model()}"}
    return {
        "metric": "attention_decode µs/call (reference entry point, compact K/V), B=1 H=32 "
                  "D=128 S=8192",
        "value": last["cold_us"], "unit": "us", "n_gpus": 1, "steps": K, "warmup": args.warmup,
        "ms_per_step": round(last["cold_us"] / 1e3, 5), "us_per_step": last["cold_us"],
        "higher_is_better": False, "scaling": "weak",
        "vs_baseline": round(last["cold_us"] / published_us[8192], 4),
        "vs_baseline_note": "µs ratio to the reference's own published figure (680 µs on an RTX "
                            "A6000, docs/en/performance/benchmarks.md:69): below 1 is faster",
        "dtype": "fp16", "data": f"synthetic: Q/K/V ~ N(0,1) ({GEN_NOTE})",
        "config": {"workload": "legacy_attention_decode_b1_h32_d128", "batch": B, "heads": H,
                   "head_dim": D, "seq_lens": list(seq_lens), "timing": "cold (rotating copies)"},
        "per_seq_len": rows,
        "roofline": {"kernel": "attn_decode_kernel<D=128,G=1> (+ attn_merge_kernel)", "bound": "hbm",
                     "achieved": round(k_gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(k_gbps / HBM_PEAK_GBPS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }


def cpu_baseline_legacy(q, k, v, B, H, S, D, scale, torch):
    """The oracle's restatement of attention_decode (compact view, its
    vectorised timing form, the native build) on the same Q/K/V, one OpenMP
    thread per (b, h) row up to the box's 16, timed over at least 0.2 s."""
    import numpy as np
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as orc
    orc.use_native_build()
    qh, kh, vh = host_bits(q), host_bits(k), host_bits(v)
    view = orc.compact_view(kh, vh, B, H, S, D)
    _, threads = cpu_counts()
    lens = np.full(B, S, dtype=np.int32)
    n, t = 0, 0.0
    while n == 0 or t < 0.2:
        t0 = time.perf_counter()
        orc.attn_decode_gqa(qh, view, lens, H, H, D, scale, nthreads=threads, fast=True)
        t += time.perf_counter() - t0
        n += 1
    us = t / n * 1e6
    nbytes = 2 * B * H * S * D * 2 + 2 * B * H * D * 2
    return {"seq_len": S, "us": round(us, 1), "gbps": round(nbytes / (us * 1e-6) / 1e9, 3),
            "threads": threads}


def gemm_bench(args, tl, torch, np):
    """W8A16 projection kernels at Llama-3-8B layer shapes (hidden 4096, 32 q /
    8 kv heads, head_dim 128, group 128) for a decode batch of 64.  Weights of
    16 layers rotate, so that every call streams its weights from HBM (16 x 25
    MB > the 256 MB MALL).  project: one launch computes Q into a buffer and K/V
    straight into the cache at each sequence's write position; oproj: hidden +=
    fp16(attn_out @ W_o).

    Two timings: `back_to_back` queues the calls behind a GPU sleep so that
    they run one after another as in a decode step (the batch's metadata is
    prepared once, as once per step for every layer), and `isolated` issues
    each call (project: with its prepare and commit) from the host and waits
    several microseconds of host work between kernels, so each starts cold.
    `value`, `kernels_us` and the roofline are the back-to-back ones."""
    import workloads
    B, hidden, Hq, Hkv, D, gs, sets = 64, 4096, 32, 8, 128, 128, 16
    K = args.steps or 100
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream().cuda_stream
    gen = torch.Generator(device=dev)
    gen.manual_seed(20261201 + 7)

    packed = args.weights == "packed"

    def weights(n):
        """int8 weights in the MFMA-fragment layout (packed once, as an engine
        would at load time) or in the reference's row-major layout, and their
        fp16 group scales."""
        w = torch.randint(-128, 128, (hidden, n), generator=gen, device=dev, dtype=torch.int8)
        wp = torch.empty_like(w) if packed else w
        if packed:
            tl.w8a16_pack(w.data_ptr(), hidden, n, wp.data_ptr(), stream)
        sc = (torch.rand(((hidden + gs - 1) // gs, n), generator=gen, device=dev) * 0.02 + 1e-3).half()
        return wp, sc
    ns = tl.NormalStreams(stream)
    x = ns.draw(workloads.seed(8, 0), (B, hidden))
    if args.path == "project":
        nq, nkv = Hq * D, Hkv * D
        W = [(weights(nq), weights(nkv), weights(nkv)) for _ in range(sets)]
        M = ((16 + 2 * K + args.warmup + 10 + 63) // 64) * 64
        mgr = tl.KVCacheManager(1, Hkv, D, M, B)
        ids = [mgr.allocateSequence(M)[0] for _ in range(B)]
        q_out = torch.empty((B, nq), device=dev, dtype=torch.float16)
        batch = tl.DecodeBatch(mgr, B, Hq)

        def kernel(i):
            (wq, sq), (wk, sk), (wv, sv) = W[i % sets]
            batch.project(0, x.data_ptr(), hidden, gs, wk.data_ptr(), sk.data_ptr(), wv.data_ptr(),
                          sv.data_ptr(), wq.data_ptr(), sq.data_ptr(), q_out.data_ptr(), stream,
                          packed=packed)

        def begin():
            batch.prepare(ids, stream)

        def end():
            batch.commit(1)
        n_out = nq + 2 * nkv
        nbytes = hidden * n_out + ((hidden + gs - 1) // gs) * n_out * 2 + B * hidden * 2 + B * n_out * 2
        desc = "fused QKV projection: q -> buffer, K/V rows -> cache at the write position"
    else:
        W = [weights(hidden) for _ in range(sets)]
        h = ns.draw(workloads.seed(8, 1), (B, hidden))
        n_out = hidden

        def kernel(i):
            w, sc = W[i % sets]
            tl.w8a16_matmul_residual(x.data_ptr(), w.data_ptr(), sc.data_ptr(), h.data_ptr(), B,
                                     hidden, hidden, gs, stream, packed=packed)

        def begin():
            pass

        def end():
            pass
        nbytes = hidden * hidden + ((hidden + gs - 1) // gs) * hidden * 2 + B * hidden * 2 + 2 * B * hidden * 2
        desc = "o_proj + residual: hidden += fp16(attn_out @ W_o)"
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(args.warmup):
        begin()
        kernel(i)
        end()
    torch.cuda.synchronize()
    # isolated: each call from the host, with its prepare / commit
    t_wall = time.perf_counter()
    ev0.record()
    for i in range(K):
        begin()
        kernel(i)
        end()
    ev1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    iso_ms = ev0.elapsed_time(ev1) / K

    # Host cost of queueing one call, to size the GPU sleep that lets the
    # host queue a whole burst before the first call runs.
    begin()
    torch.cuda.synchronize()
    torch.cuda._sleep(200_000_000)
    t_q = time.perf_counter()
    for i in range(64):
        kernel(i)
    enqueue_us = (time.perf_counter() - t_q) / 64 * 1e6
    torch.cuda.synchronize()
    end()
    # Settle: untimed back-to-back calls for about --settle-ms ahead of the
    # timed ones in the same queue, so the timed calls run at the clock the
    # GPU reaches under sustained load (the sleep ahead of a burst idles it).
    settle = int(args.settle_ms * 1e3 / max(iso_ms * 1e3, 1.0)) if args.settle_ms > 0 else 0
    sleep_cycles = int(max(200_000_000, 2.0 * (settle + K) * enqueue_us * 2.0e3))

    def burst(profile):
        """K calls queued behind a GPU sleep (and the settle calls): the
        kernels run back to back."""
        begin()
        torch.cuda.synchronize()
        torch.cuda._sleep(sleep_cycles)  # the host queues every call meanwhile
        for i in range(settle):
            kernel(i)
        if profile:
            tl.profile_reset()
            tl.profile_enable(True)
        ev0.record()
        for i in range(K):
            kernel(i)
        ev1.record()
        torch.cuda.synchronize()
        if profile:
            tl.profile_enable(False)
        end()
        return ev0.elapsed_time(ev1) / K
    ms = burst(False)
    burst(True)
    g_ms, g_n = tl.profile_query("w8a16")
    r_ms, r_n = tl.profile_query("w8a16_reduce")
    tl.profile_reset()
    g_avg = g_ms / max(1, g_n)
    r_avg = r_ms / max(1, r_n)
    flops = 2.0 * B * hidden * n_out
    kern_ms = g_avg + r_avg
    gbps = nbytes / (kern_ms * 1e-3) / 1e9
    kname = "w8a16_dec_kernel" if r_n == 0 else "w8a16_sk_kernel + w8a16_reduce_kernel"
    return {
        "metric": f"W8A16 {args.path} µs/call and achieved HBM GB/s, Llama-3-8B layer, batch 64",
        "value": round(nbytes / (ms * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16 x int8",
        "data": f"synthetic: x ~ N(0,1) ({GEN_NOTE}); int8 weights uniform ({args.weights} "
                "layout) and scales U(0.001, 0.021) (torch, seeded)",
        "config": {"workload": f"llama3_8b_{args.path}_b64", "batch": B, "hidden": hidden,
                   "out_columns": n_out, "group_size": gs, "weight_sets": sets,
                   "weights": args.weights, "what": desc, "timing": "back_to_back"},
        "kernels_us": {"w8a16": round(g_avg * 1e3, 2), "w8a16_reduce": round(r_avg * 1e3, 2)},
        "settle": {"ms": args.settle_ms, "calls": settle, "enqueue_us_per_call": round(enqueue_us, 2),
                   "why": "untimed back-to-back calls queued ahead of each timed burst: the "
                          "shader clock ramps under sustained load"},
        "isolated_us_per_call": round(iso_ms * 1e3, 2),
        "host_wall_us_per_call_isolated": round(t_wall / K * 1e6, 2),
        "roofline": {"kernel": kname, "bound": "hbm",
                     "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "tflops": round(flops / (kern_ms * 1e-3) / 1e12, 2),
                     "bytes_per_call": nbytes},
        "cpu_baseline": None,
    }


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

    torch.cuda.set_device(0)
    if args.path == "prefill":
        print(json.dumps(prefill_bench(args, tl, torch, np)), flush=True)
        return
    if args.path == "legacy":
        print(json.dumps(legacy_bench(args, tl, torch, np)), flush=True)
        return
    if args.path != "decode":
        print(json.dumps(gemm_bench(args, tl, torch, np)), flush=True)
        return
    r = churn(args, tl, torch, workloads, np) if args.config == 5 else \
        fixed_batch(args, tl, torch, workloads, np)
    K, conf = r["K"], r["conf"]
    Hq, Hkv, D = conf["q_heads"], conf["kv_heads"], conf["head_dim"]
    ms_per_step = r["elapsed_ms"] / K
    value = r["total_bytes"] / (r["elapsed_ms"] * 1e-3) / 1e9
    ks = r["ks"]
    chunk_ms, chunk_n = ks["attn_chunk"]
    merge_ms, merge_n = ks["attn_merge"]
    app_ms, app_n = ks["kv_append"]
    chunk_avg_ms = chunk_ms / max(1, chunk_n)
    achieved = r["attn_bytes"] / (chunk_avg_ms * 1e-3) / 1e9 if chunk_n else 0.0
    sp = tl.get_score_path()
    score_kind = "mfma" if sp == 1 and D <= 128 else "valu"
    traffic, traffic_src = read_pmc(conf["workload"])
    latency = args.config == 1
    if args.config == 3 and not args.q_heads:
        metric = METRIC
    elif latency:
        metric = f"decode attn+KV append latency µs/step, {conf['workload']}"
    else:
        metric = f"decode attn+KV append µs/step and achieved HBM GB/s (% of peak), {conf['workload']}"
    line = {
        "metric": metric,
        "value": round(ms_per_step * 1e3, 2) if latency else round(value, 2),
        "unit": "us" if latency else "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "achieved_gbps": round(value, 2),
        "frac_of_peak": round(value / HBM_PEAK_GBPS, 4),
        "higher_is_better": not latency,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": r["data"],
        "config": conf,
        "kernel_timing": "hipEvent pairs around each launch on its stream, " + r["kpass_desc"],
        "kernels_us": {"attn_chunk": round(chunk_avg_ms * 1e3, 2),
                       "attn_merge": round(merge_ms / max(1, merge_n) * 1e3, 2),
                       "kv_append": round(app_ms / max(1, app_n) * 1e3, 2)},
        "kernel_launches": {"attn_chunk": chunk_n, "attn_merge": merge_n, "kv_append": app_n},
        "host_wall_us_per_step": round(r["t_wall"] / K * 1e6, 2),
        "roofline": {"kernel": (f"attn_decode_kernel<D={D},G={Hq // Hkv},{score_kind},"
                               f"kv_heads_per_wg={conf.get('kv_heads_per_workgroup', 1)}>"),
                     "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic,
                     "traffic_source": (f"{traffic_src}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                                        "of this workload, calibrated by a 1 GiB copy; a committed "
                                        "profile, not this run" if traffic_src else None)},
        "cpu_baseline": r.get("cpu"),
        "library": tl.loaded_path(),
        "library_version": tl.version(),
        "device": {"name": torch.cuda.get_device_properties(0).name,
                   "cus": torch.cuda.get_device_properties(0).multi_processor_count,
                   "host": os.uname().nodename},
    }
    ps = r.get("per_step_us")
    if ps is not None and len(ps):
        line["step_us_stats"] = {"median": round(float(np.median(ps)), 2),
                                 "min": round(float(ps.min()), 2),
                                 "max": round(float(ps.max()), 2),
                                 "source": ("the profiled run of the same event sequence, one "
                                            "hipEvent per step" if args.config == 5 else
                                            "separate pass of the same steps (lengths not "
                                            "advanced), one hipEvent between steps")}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
