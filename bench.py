#!/usr/bin/env python
"""Headline benchmark: paged decode attention (+ KV page write) at C2 on one MI355X,
plus decode tokens/s of the Qwen2.5-1.5B decoder (C5) on the same line.

Workload: one layer of a batched decode step at Qwen2.5-1.5B
head shapes -- 12 query heads, 2 KV heads, head_dim 128, fp16, batch 64,
context lengths log-uniform in [128, 4096], block size 16, a 1.25x pool and
randomly permuted block tables.  A "step" is one layer's decode call
(fe_paged_decode_planned): the page write of each sequence's new token, split-K
attention over its paged K/V and the LSE merge, with every input resident in HBM.
The decode plan (fe_paged_decode_plan: the split-K partition and the block rows
of every workgroup) is computed once per model decode step and shared by its 28
layers; the timed region runs it before step 0, 28, 56, ... (ceil(steps / 28)
plan launches in `steps` steps, the share the record states).  --unplanned
times fe_paged_decode instead (partition and tables at the start of every
launch); the unplanned launch is also timed beside the planned one and reported
as roofline.us_per_launch_unplanned.

Timing: exactly --steps steps between two synchronisations, replayed from HIP
graphs (one graph cycling once over the rotating pools, replayed as often as it
fits, and one graph for the remaining steps), so the host launch path is not in
the loop.  Consecutive steps rotate over --pools copies of the KV pool (8 x
84.5 MB) so the 256 MB Infinity Cache cannot serve repeats.  value = algorithmic
bytes per step / wall time per step.  roofline.achieved = algorithmic bytes per
launch / (HIP-event time of the timed region on the launch stream / steps).

Also on the line:
* c3: the shared-prefix batch (B=256, 8 groups of 32 sharing 2048 tokens) through
  the plain decode and the cascade decode (fe_paged_decode_shared_prefix), as GB/s
  over the compulsory unique bytes and their fraction of 8 TB/s;
* c4: the mixed step -- the ragged prefill (unplanned, and with the step's plan
  charged 1/28) in TFLOP/s against the 2.5 PFLOP/s fp16 MFMA peak, the 48 decode
  rows in GB/s, and the whole step;
* c5: decode tok/s of the random-init Qwen2.5-1.5B (graph buckets 1, 2, 4 and 8,
  batch 64 eager and as a graph; contexts U{512..4096}), with the HBM bytes per
  step and their fraction of 8 TB/s;
* f32: C2's decode and C4's prefill on float32 q / K / V (the _f32 entry points;
  float32 is the reference's default cache dtype), in GB/s and TFLOP/s against
  8 TB/s and the 157.3 TFLOP/s fp32 MFMA peak;
* reference_microbench: the reference's kernel microbenchmark shape
  (src/flexengine/research/profiling/kernel.py:14-41: one request of 512 tokens,
  12/2 heads, D 128, per-request attention_for_request, 10 warm-up + 50 timed
  calls) on the HIP path, beside its published 0.537 ms/call;
* cpu_baseline: the reference's two attention routes (materialized SDPA,
  paged.py:27-35, and blockwise online softmax, paged.py:50-70) restated in
  PyTorch-CPU, timed on the host cores on C1 and C2.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
LAYERS = 28  # Qwen2.5-1.5B decoder layers sharing one decode plan per step
METRIC = "paged decode attn HBM GB/s (% peak) at B=64; decode tok/s Qwen2.5-1.5B"
# published by the reference for its fused Triton decode at the microbenchmark
# shape on an RTX 3080 Ti Laptop (README.md:278, docs/FINAL_REPORT.md:59-61)
REFERENCE_MICROBENCH_MS = 0.537

# HBM traffic per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this
# command, scaled by the counters' reading for a copy of known size.
TRAFFIC_FILE = REPO / "profiles" / "decode_c2_traffic.json"


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--pools", type=int, default=8, help="rotating KV pool copies (MALL flush)")
    p.add_argument("--target-splits", type=int, default=0)
    p.add_argument("--dtype", choices=("f16", "bf16"), default="f16",
                   help="element type of q / K / V (the configurations are quoted in f16)")
    p.add_argument("--unplanned", action="store_true",
                   help="time fe_paged_decode (no shared per-step plan)")
    p.add_argument("--cpu-seconds", type=float, default=6.0,
                   help="time budget per CPU-baseline route and config")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-c5", action="store_true", help="skip the Qwen2.5-1.5B decode tok/s")
    p.add_argument("--no-c3c4", action="store_true", help="skip the C3 and C4 figures")
    p.add_argument("--c3c4-iters", type=int, default=112)
    p.add_argument("--no-f32", action="store_true",
                   help="skip the float32 figures (C2 decode, C4 prefill on the _f32 entry points)")
    p.add_argument("--c5-steps", type=int, default=16)
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                   help="only run a device-to-device copy of MB MiB --steps times (calibrates the "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE counters against a known byte count)")
    return p.parse_args(argv)


def _progress(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def calibrate_copy(mb: int, steps: int) -> int:
    import torch

    src = torch.ones(mb << 20, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read_per_launch": src.numel(),
                      "bytes_written_per_launch": dst.numel(), "launches": steps}), flush=True)
    return 0


# ---------------------------------------------------------------------------------------
# CPU baseline
# ---------------------------------------------------------------------------------------

def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, budget_s: float, warm_max: int = 10, iters_max: int = 50):
    """kernel.py:32-41's shape within a time budget: up to 10 warm-up calls (at most a
    quarter of the budget), then up to 50 timed calls (stopping once the budget is
    spent).  Returns (seconds per call, warm-up calls, timed calls)."""
    t0 = time.perf_counter()
    warm = 0
    while warm < warm_max:
        fn()
        warm += 1
        if time.perf_counter() - t0 > budget_s / 4:
            break
    iters, t1 = 0, time.perf_counter()
    while iters < iters_max:
        fn()
        iters += 1
        if time.perf_counter() - t1 >= budget_s:
            break
    return (time.perf_counter() - t1) / iters, warm, iters


def cpu_baseline(budget_s: float) -> dict:
    """Both reference routes, restated in PyTorch-CPU, on C1 and C2 (full batches;
    each decode step first does the reference's index_put page write of the new
    token when the config has one).  `value` is the materialized route at C2."""
    import torch

    from flexengine_amd import workloads
    from oracle import torch_routes as TR

    share = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, min(share or 1, 16))
    torch.set_num_threads(threads)
    routes = {}
    for cfg, w in (("C1", workloads.c1_workload()), ("C2", workloads.c2_workload())):
        tables = [w.block_tables[b].tolist() for b in range(w.batch)]
        lens = w.context_lens.tolist()
        bs = w.block_size
        for name, fn in (("materialized", TR.decode_batch_materialized),
                         ("blockwise", TR.decode_batch_blockwise)):
            kp, vp = w.k_pool.clone(), w.v_pool.clone()

            def step():
                if w.k_new is not None:
                    for b, n in enumerate(lens):
                        blk = tables[b][(n - 1) // bs]
                        kp[blk, (n - 1) % bs] = w.k_new[b]
                        vp[blk, (n - 1) % bs] = w.v_new[b]
                return fn(w.q, kp, vp, tables, lens)

            sec, warm, iters = _timed(step, budget_s)
            _progress(f"CPU {cfg} {name}: {sec * 1e3:.1f} ms/step")
            routes[f"{cfg}_{name}"] = {
                "ms_per_step": round(sec * 1e3, 3),
                "GB_s": round(w.algorithmic_bytes() / sec / 1e9, 4),
                "sample": f"full {cfg} batch ({w.batch} seqs, {sum(lens)} tokens), "
                          f"{warm} warm-up + {iters} timed steps"}
    main = routes["C2_materialized"]
    return {"value": main["GB_s"], "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_step": main["ms_per_step"],
            "sample": "full C2 batch (64 seqs) on the materialized route (paged.py:27-35) with "
                      "its index_put page write, fp16, PyTorch-CPU restatement; "
                      + main["sample"],
            "routes": routes, "host_cpu_count": os.cpu_count(), "cpu_share": share,
            "cpu_model": _cpu_model(), "torch_threads": threads}


# ---------------------------------------------------------------------------------------
# GPU legs
# ---------------------------------------------------------------------------------------

def reference_microbench(dev) -> dict:
    """kernel.py:14-41 on the HIP path: one 512-token request, 12/2 heads, D 128,
    attention_for_request per call, 10 warm-up + 50 timed calls, perf_counter + sync."""
    import torch

    from flexengine_amd import attention
    from flexengine_amd.kv_cache import CacheLayout, PagedKVCache

    seq, hq, hkv, d = 512, 12, 2, 128
    cache = PagedKVCache(CacheLayout(1, (seq + 15) // 16 + 1, 16, hkv, d), device=dev)
    cache.reserve("r", seq)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    cache.write(0, "r", 0, torch.randn(seq, hkv, d, device=dev, generator=g).half(),
                torch.randn(seq, hkv, d, device=dev, generator=g).half())
    q = torch.randn(1, hq, d, device=dev, generator=g).half()
    pos = torch.tensor([seq - 1], device=dev)
    for _ in range(10):
        attention.attention_for_request(q, cache, 0, "r", seq, pos)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(50):
        attention.attention_for_request(q, cache, 0, "r", seq, pos)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / 50
    return {"shape": "B=1, 512 ctx, 12/2 heads, D 128, per-request attention_for_request",
            "ms_per_call": round(ms, 4), "reference_published_ms": REFERENCE_MICROBENCH_MS,
            "reference_hw": "RTX 3080 Ti Laptop (README.md:278)",
            "speedup_vs_published": round(REFERENCE_MICROBENCH_MS / ms, 1)}


def c5_decode(steps: int) -> dict:
    """Decode tok/s of the random-init Qwen2.5-1.5B at contexts U{512..4096}."""
    import torch

    from flexengine_amd import bench_model
    from flexengine_amd.model import Qwen2Config, Qwen2Model

    model = Qwen2Model(Qwen2Config(), "cuda:0", seed=5)
    res = {}
    for key, batch, mode in (("bucket1_graph", 1, "bucket"), ("bucket2_graph", 2, "bucket"),
                             ("bucket4_graph", 4, "bucket"), ("bucket8_graph", 8, "bucket"),
                             ("b64_eager", 64, "eager"), ("b64_graph", 64, "graph")):
        r = bench_model.run(model, batch, steps, 3, mode)
        _progress(f"C5 {key}: {r['tok_s']} tok/s")
        res[key] = {"tok_s": r["tok_s"], "ms_per_step": r["ms_per_step"],
                    "hbm_GB_s": r["hbm_GB_s"],
                    "pct_of_hbm_bound": round(100.0 * r["hbm_GB_s"] / HBM_PEAK_GBS, 1),
                    "hbm_bytes_per_step": r["hbm_bytes_per_step"], "steps": r["steps"],
                    "mean_context": r["mean_context"]}
        torch.cuda.empty_cache()
    res["workload"] = ("C5: random-init Qwen2.5-1.5B (28 layers, 12/2 heads, D 128, fp16), KV "
                       "N(0,1) with L ~ U{512..4096}, greedy; buckets via hipGraph replay")
    return res


def c3_c4(iters: int) -> tuple[dict, dict]:
    """C3 (plain and cascade decode) and C4 (prefill, decode rows, step), timed as
    flexengine_amd.bench_attention does (HIP graphs, rotating pool copies)."""
    import torch

    from flexengine_amd import bench_attention as BA
    from flexengine_amd import workloads

    w = workloads.c3_workload()
    hkv, d = w.k_pool.shape[2], w.k_pool.shape[3]
    unique = w.unique_tokens * 2 * hkv * d * 2 + 2 * w.q.numel() * 2
    plain = BA.bench_decode("C3", w, iters, 4, unique)
    cascade = BA.bench_decode("C3", w, iters, 4, unique, shared_prefix=True)
    del w
    torch.cuda.empty_cache()
    keys = ("us_per_call", "GB_s", "pct_hbm_peak", "effective_GB_s")
    c3 = {"plain": {k: plain[k] for k in keys}, "cascade": {k: cascade[k] for k in keys},
          "unique_bytes": unique, "logical_bytes": plain["bytes"],
          "workload": "C3: B=256 in 8 groups of 32 sharing 2048 tokens + tails U[16,2048], "
                      "12/2 heads, D 128, fp16, block 16; GB/s over the unique bytes"}
    c4 = BA.bench_c4(iters, 4)
    torch.cuda.empty_cache()
    c4["workload"] = ("C4: 4 prefill chunks of 256-512 tokens over 0-3072 cached + 48 decode "
                      "rows L~U[256,4096], 12/2 heads, D 128, fp16, block 16")
    c4["decode_pct_hbm_peak"] = round(100.0 * c4["decode_GB_s"] / HBM_PEAK_GBS, 1)
    return c3, c4


def f32_legs(iters: int) -> dict:
    """C2's decode and C4's prefill on float32 pools (fe_paged_decode_f32,
    fe_prefill_paged_f32; the reference's default cache dtype), timed as
    flexengine_amd.bench_attention does.  Not the headline: C2 and C4 are quoted
    in fp16."""
    import torch

    from flexengine_amd import bench_attention as BA
    from flexengine_amd import workloads

    dec = BA.bench_decode("C2", workloads.c2_workload(), iters, 4, dtype=torch.float32)
    torch.cuda.empty_cache()
    c4 = BA.bench_c4(iters, 4, torch.float32)
    torch.cuda.empty_cache()
    return {
        "c2_decode": {k: dec[k] for k in ("us_per_call", "bytes", "GB_s", "pct_hbm_peak")},
        "c4_prefill": {"us_per_call": c4["prefill_us"], "TFLOP_s": c4["prefill_TFLOP_s"],
                       "pct_mfma_fp32_peak": c4["pct_mfma_fp32_peak"]},
        "c4_decode_rows": {"us_per_call": c4["decode_us"], "GB_s": c4["decode_GB_s"]},
        "workload": "C2 and C4 with float32 q / K / V / out (unplanned; 4 bytes per element; "
                    "prefill against the 157.3 TFLOP/s fp32 MFMA peak)",
    }


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU mode: every GPU box here has one GPU", file=sys.stderr)
        return 2
    import torch

    from flexengine_amd import ops, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy, args.steps)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = workloads.c2_workload()
    d = w.to(dev)
    if args.dtype == "bf16":
        for name in ("q", "k_pool", "v_pool", "k_new", "v_new"):
            setattr(d, name, getattr(d, name).float().to(torch.bfloat16))
    n_pool = max(1, args.pools)
    pools = [(d.k_pool, d.v_pool)] + [(d.k_pool.clone(), d.v_pool.clone())
                                      for _ in range(n_pool - 1)]
    out = torch.empty_like(d.q)
    ws = ops.decode_workspace(dev, ops.decode_workspace_bytes(
        w.batch, 12, 128, w.block_tables.shape[1] * w.block_size, args.target_splits))
    nbytes = w.algorithmic_bytes()
    steps, warm = max(1, args.steps), max(0, args.warmup)
    planned = not args.unplanned
    nb, bs, hkv = d.k_pool.shape[0], d.k_pool.shape[1], d.k_pool.shape[2]
    plan = ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs,
                                 target_splits=args.target_splits) if planned else None

    def step(i: int) -> None:
        kp, vp = pools[i % n_pool]
        if planned and i % LAYERS == 0:    # one plan per model decode step of 28 layers
            ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs,
                                  target_splits=args.target_splits, out=plan)
        ops.paged_decode(d.q, kp, vp, d.block_tables, d.context_lens, k_new=d.k_new,
                         v_new=d.v_new, out=out, workspace=ws, target_splits=args.target_splits,
                         plan=plan)

    # graphs of whole periods of both the pool rotation and the plan: the cycle
    # graph replays steps 0 .. period-1, the rest graph steps 0 .. steps % period - 1
    period = n_pool * LAYERS // math.gcd(n_pool, LAYERS) if planned else n_pool
    for i in range(warm):                  # the requested warm-up steps, eager
        step(i)
    torch.cuda.synchronize()

    def record(count: int):
        if count == 0:
            return None
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(count):
                step(i)
        return g

    cycle = record(min(period, steps))
    rest = record(steps % period) if steps > period else None
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(max(1, steps // period)):
        cycle.replay()
    if rest is not None:
        rest.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_launch_ms = ev0.elapsed_time(ev1) / steps
    ms_per_step = wall * 1e3 / steps
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    achieved = nbytes / (per_launch_ms * 1e-3) / 1e9
    del cycle, rest
    # the other form of the launch (unplanned when the headline is planned), same method
    other_us = None
    if planned:
        def step_unplanned(i: int) -> None:
            kp, vp = pools[i % n_pool]
            ops.paged_decode(d.q, kp, vp, d.block_tables, d.context_lens, k_new=d.k_new,
                             v_new=d.v_new, out=out, workspace=ws,
                             target_splits=args.target_splits)
        for i in range(n_pool):
            step_unplanned(i)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n_pool * 7):
                step_unplanned(i)
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(2):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        other_us = e0.elapsed_time(e1) * 1e3 / (2 * n_pool * 7)
        del g
    del pools
    torch.cuda.empty_cache()

    traffic, traffic_src = None, None
    if TRAFFIC_FILE.exists():
        try:
            tj = json.loads(TRAFFIC_FILE.read_text())
            traffic = tj.get("bytes_per_launch")
            traffic_src = f"{TRAFFIC_FILE.relative_to(REPO)} ({tj.get('workload', '?')})"
        except (ValueError, OSError):
            pass

    _progress(f"C2: {per_launch_ms * 1e3:.2f} us per launch, {value:.0f} GB/s")
    micro = reference_microbench(dev)
    _progress(f"reference microbenchmark shape: {micro['ms_per_call']} ms/call")
    c3, c4 = (None, None) if args.no_c3c4 else c3_c4(args.c3c4_iters)
    if c3 is not None:
        _progress(f"C3 plain {c3['plain']['us_per_call']} us, cascade {c3['cascade']['us_per_call']} us;"
                  f" C4 prefill {c4['prefill_planned_us']} us planned, decode {c4['decode_us']} us")
    f32 = None if args.no_f32 else f32_legs(args.c3c4_iters)
    if f32 is not None:
        _progress(f"fp32: C2 decode {f32['c2_decode']['us_per_call']} us, "
                  f"C4 prefill {f32['c4_prefill']['us_per_call']} us")
    c5 = None if args.no_c5 else c5_decode(args.c5_steps)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)

    elem, sfx = ("Bf16", "_bf16") if args.dtype == "bf16" else ("Fp16", "")
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded N(0,1) q/K/V, random block tables; random-init weights for c5)",
        "config": {
            "workload": "C2: paged decode attention + KV page write, one layer, Qwen2.5-1.5B heads "
                        "(12 q / 2 kv / D 128), batch 64, ctx log-uniform [128,4096], block 16, "
                        "1.25x pool, permuted tables",
            "batch": w.batch,
            "context_tokens": int(w.context_lens.sum()),
            "algorithmic_bytes_per_step": nbytes,
            "rotating_pools": n_pool,
            "graph_replay": True,
            "target_splits": args.target_splits,
            "decode_plan": (f"fe_paged_decode_plan once per {LAYERS} steps inside the timed "
                            f"region ({-(-steps // LAYERS)} plan launches: one per model decode "
                            f"step of the {LAYERS}-layer model)") if planned else "none",
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel": (f"piece_decode_kernel<128, true, true, {elem}, false> (fe_paged_decode_planned"
                       f"{sfx}: page write + split-K attention + in-kernel LSE merge, one "
                       f"launch; achieved includes {-(-steps // LAYERS)} decode_plan_kernel "
                       f"launch(es) over the {steps} launches)")
                      if planned else
                      f"piece_decode_kernel<128, true, false, {elem}, false> (fe_paged_decode{sfx}: "
                      "page write + split-K attention + in-kernel LSE merge, one launch)",
            "us_per_launch": round(per_launch_ms * 1e3, 3),
            "us_per_launch_unplanned": None if other_us is None else round(other_us, 3),
        },
        "c3": c3,
        "c4": c4,
        "c5": c5,
        "f32": f32,
        "reference_microbench": micro,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
