"""Per-configuration timings of the attention kernels (configs C1, C3, C4).

    python -m flexengine_amd.bench_attention [--iters 50] [--configs c1,c3,c4] [--dtype bf16]

bench.py measures the headline config (C2); this script times the others the
same way -- inputs resident in HBM, several rotating copies of the KV pool so
the 256 MB Infinity Cache cannot serve repeats, HIP events on the launch
stream -- and prints one JSON line per config:

* C1 (B=8, 14/2 heads, D 64, L ~ U{16..512}): decode latency and GB/s.
* C3 (B=256 in 8 groups sharing a 2048-token prefix): decode time, GB/s over
  the compulsory unique bytes, and the "effective" GB/s over the logical bytes,
  for the plain decode and for the shared-prefix (cascade) decode.
* C4 (mixed step): the ragged prefill launch in TFLOP/s over the valid
  query-key pairs against the 2.5 PFLOP/s fp16 MFMA peak (also with the
  step's plan, fe_prefill_plan once per 28 calls as in a 28-layer model step),
  the 48 decode rows in GB/s, and the whole step.

Calls are replayed from a HIP graph, so each figure is GPU time per call.
`--configs generic` times the shapes outside head_dim 64 / 128 (96, 80, 8: the
matrix-core kernels padded to 128 / 64 in 16 bits, the generic kernel in fp32; 160
padded to 256; 256; a group of 32 at D = 128) at C2's 64 context lengths, and C4's
prefill chunks at head_dim 96, 160 and 256.

`--dtype bf16` runs the bf16 entry points on the same values rounded to bf16;
`--dtype f32` the fp32 entry points on the values widened to float32 (bytes at
4 per element, the C4 prefill against the 157.3 TFLOP/s fp32 MFMA peak; no plan).
"""
from __future__ import annotations

import argparse
import json
import sys

import torch

from flexengine_amd import ops, workloads

HBM_PEAK = 8.0e12
# (head_dim, q heads, KV heads) of `--configs generic`
GENERIC_SHAPES = [(96, 12, 2), (80, 32, 8), (160, 16, 2), (256, 8, 1), (256, 16, 8),
                  (128, 32, 1), (8, 4, 2)]
LAYERS = 28  # Qwen2.5-1.5B: calls per model step that share one plan
MFMA_FP16_PEAK = 2.5e15
MFMA_FP32_PEAK = 157.3e12


def _timed(fn, iters: int, variants: int) -> float:
    """Mean GPU seconds per call of fn(i), i cycling over `variants` inputs.

    The `variants` calls are captured once into a HIP graph (after an eager warm-up
    that also sizes the workspaces) and the graph is replayed, so the figure is the
    GPU's time per call, not the host's launch rate; HIP events on the replay stream.
    """
    for i in range(variants):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(variants):
            fn(i)
    reps = max(2, iters // variants)
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / (reps * variants)


def _cast(w, dtype):
    """The workload (already on the device) with its 16-bit tensors in `dtype`."""
    if dtype == torch.float16:
        return w
    for name in ("q", "k_pool", "v_pool", "k_new", "v_new"):
        t = getattr(w, name, None)
        if t is not None:
            setattr(w, name, t.float().to(dtype))
    if getattr(w, "decode", None) is not None:
        w.decode.q = w.decode.q.float().to(dtype)
        w.decode.k_pool, w.decode.v_pool = w.k_pool, w.v_pool
    return w


def _pools(w, copies: int):
    return [(w.k_pool, w.v_pool)] + [(w.k_pool.clone(), w.v_pool.clone()) for _ in range(copies - 1)]


def bench_decode(name: str, w, iters: int, copies: int, unique_bytes: int | None = None,
                 shared_prefix: bool = False, dtype=torch.float16) -> dict:
    d = _cast(w.to("cuda:0"), dtype)
    pools = _pools(d, copies)
    out = torch.empty_like(d.q)
    if shared_prefix:
        go, pl = d.meta["group_offsets"].to("cuda:0"), d.meta["prefix_lens"].to("cuda:0")

    def step(i):
        kp, vp = pools[i % len(pools)]
        if shared_prefix:
            ops.paged_decode_shared_prefix(d.q, kp, vp, d.block_tables, d.context_lens, go, pl,
                                           out=out)
        else:
            ops.paged_decode(d.q, kp, vp, d.block_tables, d.context_lens, out=out)

    sec = _timed(step, iters, len(pools))
    logical = d.algorithmic_bytes(logical=True)
    kernel = "fe_paged_decode_shared_prefix" if shared_prefix else "fe_paged_decode"
    res = {"config": name, "kernel": kernel, "us_per_call": round(sec * 1e6, 2),
           "batch": w.batch, "context_tokens": int(w.context_lens.sum()),
           "bytes": logical, "GB_s": round(logical / sec / 1e9, 1),
           "pct_hbm_peak": round(100 * logical / sec / HBM_PEAK, 1)}
    if unique_bytes is not None:
        res.update({"unique_bytes": unique_bytes, "GB_s": round(unique_bytes / sec / 1e9, 1),
                    "pct_hbm_peak": round(100 * unique_bytes / sec / HBM_PEAK, 1),
                    "effective_GB_s": round(logical / sec / 1e9, 1)})
    return res


def bench_c4(iters: int, copies: int, dtype=torch.float16) -> dict:
    w = workloads.c4_workload()
    d = _cast(w.to("cuda:0"), dtype)
    pools = _pools(d, copies)
    out = torch.empty_like(d.q)
    max_q = int((w.q_offsets[1:] - w.q_offsets[:-1]).max())

    def prefill(i):
        kp, vp = pools[i % len(pools)]
        ops.prefill_paged(d.q, kp, vp, d.block_tables, d.q_offsets, d.context_lens, max_q, out=out)

    # one plan per model step of 28 layers (fe_prefill_plan), charged 1/28 per call
    # (16-bit pools: the fp32 prefill has no plan)
    hq, hkv = d.q.shape[1], d.k_pool.shape[2]
    plan = None
    if dtype != torch.float32:
        plan = ops.prefill_paged_plan(d.q_offsets, d.context_lens, d.q.shape[0], hq, hkv,
                                      d.block_tables.shape[1], d.k_pool.shape[1])

    def prefill_planned(i):
        kp, vp = pools[i % len(pools)]
        if i % LAYERS == 0:
            ops.prefill_paged_plan(d.q_offsets, d.context_lens, d.q.shape[0], hq, hkv,
                                   d.block_tables.shape[1], d.k_pool.shape[1], out=plan)
        ops.prefill_paged(d.q, kp, vp, d.block_tables, d.q_offsets, d.context_lens, max_q,
                          out=out, plan=plan)

    dec = d.decode
    dout = torch.empty_like(dec.q)

    def decode(i):
        kp, vp = pools[i % len(pools)]
        ops.paged_decode(dec.q, kp, vp, dec.block_tables, dec.context_lens, out=dout)

    def both(i):
        prefill(i)
        decode(i)

    # the decode rows and the prefill chunks are different sequences with their own
    # outputs and workspaces: the decode can run on a second stream (default
    # priority) beside the MFMA-bound prefill, forked and joined inside the graph
    side = torch.cuda.Stream()

    def both_overlapped(i):
        main = torch.cuda.current_stream()
        side.wait_stream(main)
        prefill(i)
        with torch.cuda.stream(side):
            decode(i)
        main.wait_stream(side)

    t_pre = _timed(prefill, iters, len(pools))
    t_plan = _timed(prefill_planned, iters, LAYERS) if plan is not None else None
    t_dec = _timed(decode, iters, len(pools))
    t_all = _timed(both, iters, len(pools))
    t_ovl = _timed(both_overlapped, iters, len(pools))
    flops = w.flops()
    dbytes = d.decode.algorithmic_bytes()
    # the MFMA peak of the arithmetic type: fp16 / bf16 (same dense rate) or fp32
    f32 = dtype == torch.float32
    peak, tag = (MFMA_FP32_PEAK, "fp32") if f32 else (MFMA_FP16_PEAK, "fp16")
    return {"config": "C4", "prefill_us": round(t_pre * 1e6, 2), "prefill_flops": flops,
            "prefill_TFLOP_s": round(flops / t_pre / 1e12, 1),
            f"pct_mfma_{tag}_peak": round(100 * flops / t_pre / peak, 2),
            "prefill_planned_us": None if t_plan is None else round(t_plan * 1e6, 2),
            f"pct_mfma_{tag}_peak_planned":
                None if t_plan is None else round(100 * flops / t_plan / peak, 2),
            "decode_us": round(t_dec * 1e6, 2), "decode_bytes": dbytes,
            "decode_GB_s": round(dbytes / t_dec / 1e9, 1), "step_us": round(t_all * 1e6, 2),
            "step_overlap_us": round(t_ovl * 1e6, 2),
            "prefill_tokens": int(w.q.shape[0]), "chunks": w.meta["n_new"], "cached": w.meta["cached"]}


def bench_generic_prefill(iters: int, copies: int, head_dim: int, dtype) -> dict:
    """C4's prefill chunks (offsets, contexts, tables) at another head_dim (16-bit:
    the tile kernel at 256, or padded to 128 / 256 for 96 / 160; fp32: the generic
    kernel): TFLOP/s over the valid query-key pairs."""
    w = workloads.c4_workload()
    gen = torch.Generator().manual_seed(96)
    nb, bs, hkv, _ = w.k_pool.shape
    hq = w.q.shape[1]

    def draw(*shape):
        return torch.randn(*shape, generator=gen).to(dtype).to("cuda:0")
    q = draw(w.q.shape[0], hq, head_dim)
    pools = [(draw(nb, bs, hkv, head_dim), draw(nb, bs, hkv, head_dim)) for _ in range(copies)]
    tables, offs, ctx = (t.to("cuda:0") for t in (w.block_tables, w.q_offsets, w.context_lens))
    out = torch.empty_like(q)
    max_q = int((w.q_offsets[1:] - w.q_offsets[:-1]).max())

    def prefill(i):
        kp, vp = pools[i % len(pools)]
        ops.prefill_paged(q, kp, vp, tables, offs, ctx, max_q, out=out)

    sec = _timed(prefill, iters, len(pools))
    flops = w.flops() // 128 * head_dim  # w.flops() counts 4 * Hq * 128 per pair
    return {"config": f"C4-prefill-d{head_dim}", "kernel": "fe_prefill_paged",
            "us_per_call": round(sec * 1e6, 2), "flops": flops,
            "TFLOP_s": round(flops / sec / 1e12, 2),
            "pct_mfma_fp16_peak": round(100 * flops / sec / MFMA_FP16_PEAK, 2)}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--iters", type=int, default=200)
    p.add_argument("--copies", type=int, default=4, help="rotating KV pool copies")
    p.add_argument("--configs", default="c1,c3,c4")
    p.add_argument("--dtype", choices=("f16", "bf16", "f32"), default="f16")
    args = p.parse_args(argv)
    dt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[args.dtype]
    if not torch.cuda.is_available():
        print("bench_attention needs a ROCm GPU", file=sys.stderr)
        return 2
    cfgs = args.configs.split(",")
    if "c1" in cfgs:
        print(json.dumps(bench_decode("C1", workloads.c1_workload(), args.iters, args.copies * 8,
                                      dtype=dt) | {"dtype": args.dtype}), flush=True)
    if "c3" in cfgs:
        w = workloads.c3_workload()
        hkv, d = w.k_pool.shape[2], w.k_pool.shape[3]
        # compulsory bytes: every distinct K/V row once, plus q and out
        size = torch.tensor([], dtype=dt).element_size()
        unique = w.unique_tokens * 2 * hkv * d * size + 2 * w.q.numel() * size
        print(json.dumps(bench_decode("C3", w, args.iters, args.copies, unique, dtype=dt)
                         | {"dtype": args.dtype}), flush=True)
        print(json.dumps(bench_decode("C3", w, args.iters, args.copies, unique,
                                      shared_prefix=True, dtype=dt) | {"dtype": args.dtype}),
              flush=True)
    if "c4" in cfgs:
        print(json.dumps(bench_c4(args.iters, args.copies, dt) | {"dtype": args.dtype}),
              flush=True)
    if "generic" in cfgs:
        # the generic kernel's shapes (head_dim other than 64 / 128, decode groups
        # above 16) at C2's 64 context lengths
        lens = workloads.c2_lengths()
        for d, hq, hkv in GENERIC_SHAPES:
            w = workloads.make_decode_workload(f"G-d{d}-{hq}x{hkv}", 5, len(lens), hq, hkv, d,
                                               lens)
            print(json.dumps(bench_decode(w.name, w, args.iters, args.copies, dtype=dt)
                             | {"dtype": args.dtype, "head_dim": d, "q_heads": hq,
                                "kv_heads": hkv}), flush=True)
        for d in (96, 160, 256):
            print(json.dumps(bench_generic_prefill(args.iters, args.copies, d, dt)
                             | {"dtype": args.dtype}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
