#!/usr/bin/env python
"""Headline benchmark: paged decode attention (+ KV page write) at C2 on one MI355X.

Workload: one layer of a batched decode step at Qwen2.5-1.5B
head shapes -- 12 query heads, 2 KV heads, head_dim 128, fp16, batch 64,
context lengths log-uniform in [128, 4096], block size 16, a 1.25x pool and
randomly permuted block tables.  A "step" is one fe_paged_decode call: the page
write of each sequence's new token, split-K attention over its paged K/V and
the LSE merge, with every input resident in HBM.

value = algorithmic bytes of one step / wall time of one step (K steps between
synchronisations; the steps are replayed from a HIP graph so the host launch
path is not in the loop).  To keep the 256 MB Infinity Cache from serving
repeats, consecutive steps rotate over --pools independent copies of the KV
pool (8 x 84.5 MB by default).

Also reported on the same line: the roofline of the decode launch (HIP-event
duration per launch on the launch stream; algorithmic bytes / duration against
8 TB/s HBM3E) and the CPU baseline (the reference's materialized SDPA route
restated in PyTorch, timed on the host cores on the same C2 batch).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
METRIC = "paged decode attn HBM GB/s (% peak) at B=64; decode tok/s Qwen2.5-1.5B"

# Optional HBM traffic per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# (bytes, scaled by the copy-kernel calibration); see profiles/.
TRAFFIC_FILE = REPO / "profiles" / "decode_c2_traffic.json"


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--pools", type=int, default=8, help="rotating KV pool copies (MALL flush)")
    p.add_argument("--target-splits", type=int, default=0)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-graph", action="store_true", help="launch eagerly instead of graph replay")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                   help="only run a device-to-device copy of MB MiB --steps times (calibrates the "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE counters against a known byte count)")
    return p.parse_args(argv)


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


def cpu_baseline(w, budget_s: float) -> dict:
    """The reference's per-request materialized route (page write + gather +
    repeat_interleave + SDPA, fp16) over the C2 batch on the host cores."""
    import torch

    from oracle import torch_routes as TR

    threads = torch.get_num_threads()
    kp, vp = w.k_pool.clone(), w.v_pool.clone()
    tables = [w.block_tables[b].tolist() for b in range(w.batch)]
    lens = w.context_lens.tolist()
    bs = w.block_size

    def one_step():
        for b, n in enumerate(lens):
            pos = n - 1
            blk = tables[b][pos // bs]
            kp[blk, pos % bs] = w.k_new[b]        # the reference's index_put write
            vp[blk, pos % bs] = w.v_new[b]
        return TR.decode_batch_materialized(w.q, kp, vp, tables, lens)

    one_step()  # warm-up
    iters, t0 = 0, time.perf_counter()
    while True:
        one_step()
        iters += 1
        el = time.perf_counter() - t0
        if el >= budget_s or iters >= 50:
            break
    sec = el / iters
    return {"value": round(w.algorithmic_bytes() / sec / 1e9, 4), "unit": "GB/s", "cores": threads,
            "kind": "port", "ms_per_step": round(sec * 1e3, 3),
            "sample": f"full C2 batch (64 seqs, {sum(lens)} tokens), {iters} steps after 1 warm-up; "
                      "PyTorch-CPU restatement of the reference's materialized route "
                      "(paged.py:27-35) with its index_put page write, fp16"}


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the paged-attention "
              "hot path has no multi-GPU mode in this build", file=sys.stderr)
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
    pools = [(d.k_pool, d.v_pool)] + [(d.k_pool.clone(), d.v_pool.clone())
                                      for _ in range(max(1, args.pools) - 1)]
    out = torch.empty_like(d.q)
    ws = ops.decode_workspace(dev, ops.decode_workspace_bytes(
        w.batch, 12, 128, w.block_tables.shape[1] * w.block_size, args.target_splits))
    nbytes = w.algorithmic_bytes()

    def step(i: int) -> None:
        kp, vp = pools[i % len(pools)]
        ops.paged_decode(d.q, kp, vp, d.block_tables, d.context_lens, k_new=d.k_new,
                         v_new=d.v_new, out=out, workspace=ws, target_splits=args.target_splits)

    stream = torch.cuda.current_stream(dev)
    n_pool = len(pools)
    graph = None
    if not args.no_graph:
        for i in range(n_pool):      # warm-up outside capture
            step(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n_pool):
                step(i)
        stream = torch.cuda.current_stream(dev)

    def run(k: int, start_ev=None, end_ev=None) -> None:
        if graph is None:
            for i in range(k):
                if start_ev is not None:
                    start_ev[i].record(stream)
                step(i)
                if end_ev is not None:
                    end_ev[i].record(stream)
            return
        reps = k // n_pool
        for r in range(reps):
            if start_ev is not None:
                start_ev[r].record(stream)
            graph.replay()
            if end_ev is not None:
                end_ev[r].record(stream)

    steps = max(n_pool, (args.steps // n_pool) * n_pool)
    warm = max(n_pool, (args.warmup // n_pool) * n_pool)
    run(warm)
    torch.cuda.synchronize()
    n_ev = steps if graph is None else steps // n_pool
    ev0 = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    ev1 = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(steps, ev0, ev1)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_launch_ms = sum(a.elapsed_time(b) for a, b in zip(ev0, ev1)) / steps
    ms_per_step = wall * 1e3 / steps
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    achieved = nbytes / (per_launch_ms * 1e-3) / 1e9

    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("bytes_per_launch")
        except (ValueError, OSError):
            traffic = None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w, args.cpu_seconds)

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
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) q/K/V, random block tables)",
        "config": {
            "workload": "C2: paged decode attention + KV page write, one layer, Qwen2.5-1.5B heads "
                        "(12 q / 2 kv / D 128), batch 64, ctx log-uniform [128,4096], block 16, "
                        "1.25x pool, permuted tables",
            "batch": w.batch,
            "context_tokens": int(w.context_lens.sum()),
            "algorithmic_bytes_per_step": nbytes,
            "rotating_pools": n_pool,
            "graph_replay": graph is not None,
            "target_splits": args.target_splits,
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "piece_decode_kernel<128, true> (fe_paged_decode: page write + split-K "
                      "attention + in-kernel LSE merge, one launch)",
            "us_per_launch": round(per_launch_ms * 1e3, 3),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
