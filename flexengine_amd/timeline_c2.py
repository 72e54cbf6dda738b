"""Per-workgroup timeline of the planned C2 decode launch (piece_decode_kernel).

    python -m flexengine_amd.build --timeline      # on a build host: libfe_paged_timeline.so
    python -m flexengine_amd.timeline_c2 [--launches 6]

Runs C2 (bench.py's headline workload: fe_paged_decode_planned with the fused
page write, 8 rotating KV pools) on the diagnostic build, in which thread 0 of
every workgroup records s_memrealtime stamps (100 MHz, one clock for the
device) at the kernel's phase boundaries: 0 start, 1 piece known (plan header
read), 2 wave 0's tile loop ended, 3 the four waves combined, 4 output stored
(unsplit) or partial stored and ticket drawn (split), 5 merge issued (the last
piece of a split row).  Each timed launch follows 24 warm-up launches; the
stamps are cleared before it.  Prints a markdown summary: the launch's extent
from the stamps, every phase's duration on each workgroup, when loops end and
merges finish across the grid, and the per-XCD start offsets (workgroup i runs
on XCD i % 8).
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys

import numpy as np

from flexengine_amd.build import TIMELINE_LIB_PATH

# the diagnostic build must be the one loaded (before the first import of _lib)
os.environ["FE_PAGED_LIB"] = str(TIMELINE_LIB_PATH)

import torch  # noqa: E402

from flexengine_amd import _lib, ops, workloads  # noqa: E402

TICK_US = 0.01  # s_memrealtime runs at 100 MHz
SLOTS = 16
PHASES = ["start", "piece known", "loop end", "combined", "stored / ticket", "merged"]


def run(launches: int, pools: int = 8) -> np.ndarray:
    lib = _lib.load()
    lib.fe_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.fe_timeline_read.restype = ctypes.c_int
    lib.fe_timeline_clear.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    w = workloads.c2_workload()
    d = w.to(dev)
    nb, bs, hkv = d.k_pool.shape[0], d.k_pool.shape[1], d.k_pool.shape[2]
    kvs = [(d.k_pool, d.v_pool)] + [(d.k_pool.clone(), d.v_pool.clone()) for _ in range(pools - 1)]
    out = torch.empty_like(d.q)
    plan = ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs)
    grid = (plan.buffer.numel() // 4 - 16) // (8 + 256) * hkv  # (target + 2B) * Hkv workgroups

    def call(i):
        kp, vp = kvs[i % len(kvs)]
        ops.paged_decode(d.q, kp, vp, d.block_tables, d.context_lens, k_new=d.k_new,
                         v_new=d.v_new, out=out, plan=plan)

    stamps = []
    for rep in range(launches):
        for i in range(24):
            call(i)
        torch.cuda.synchronize()
        assert lib.fe_timeline_clear() == 0
        call(rep)
        torch.cuda.synchronize()
        buf = np.zeros(grid * SLOTS, dtype=np.uint64)
        assert lib.fe_timeline_read(buf.ctypes.data, grid) == 0
        stamps.append(buf.reshape(grid, SLOTS).astype(np.int64))
    return np.stack(stamps)


def _q(x, qs=(10, 50, 90)):
    return " / ".join(f"{np.percentile(x, q):.2f}" for q in qs) + f" / {x.max():.2f}"


def summarize(st: np.ndarray) -> str:
    lines = []
    ends, starts_xcd, loop_ends, merges, phase = [], [], [], [], {k: [] for k in range(1, 6)}
    for t in st:
        t0 = t[:, 0].min()
        found = (t[:, 6] & 1) == 1
        last = np.maximum(t[:, 4], t[:, 5])
        ends.append((last.max() - t0) * TICK_US)
        starts = (t[:, 0] - t0) * TICK_US
        xcd = np.arange(len(t)) % 8
        starts_xcd.append([np.median(starts[xcd == x]) for x in range(8)])
        loop_ends.append((t[found, 2] - t0) * TICK_US)
        merged = t[:, 6] == 7
        merges.append((t[merged, 5] - t0) * TICK_US)
        for k in range(1, 6):
            sel = found & (t[:, k] > 0) & (t[:, k - 1 if k != 5 else 4] > 0)
            prev = t[sel, k - 1 if k != 5 else 4]
            phase[k].append((t[sel, k] - prev) * TICK_US)
    t = st[-1]
    found = (t[:, 6] & 1) == 1
    lines.append(f"Launches: {len(st)}; workgroups per launch: {len(t)} "
                 f"({int(found.sum())} with a piece, {int((t[:, 6] == 7).sum())} merging, "
                 f"{int((t[:, 6] == 3).sum())} split non-merging).")
    lines.append("")
    lines.append("| Measure (µs) | p10 / median / p90 / max |")
    lines.append("|---|---|")
    lines.append(f"| launch extent from the stamps (first start to last store), per launch | "
                 f"{' '.join(f'{e:.2f}' for e in ends)} |")
    names = {1: "start → piece known (plan header)", 2: "piece known → wave 0's loop end",
             3: "loop end → waves combined", 4: "combined → stored / ticket drawn",
             5: "ticket → merge issued (merging pieces)"}
    for k in range(1, 6):
        lines.append(f"| {names[k]} | {_q(np.concatenate(phase[k]))} |")
    lines.append(f"| loop end, from the launch's first start | {_q(np.concatenate(loop_ends))} |")
    lines.append(f"| merge issued, from the launch's first start | {_q(np.concatenate(merges))} |")
    sx = np.array(starts_xcd)
    lines.append("")
    lines.append("Median start of each XCD's workgroups after the launch's first start (µs), "
                 "median over launches:")
    lines.append("")
    lines.append("| XCD | " + " | ".join(str(x) for x in range(8)) + " |")
    lines.append("|---|" + "---|" * 8)
    lines.append("| start | " + " | ".join(f"{v:.2f}" for v in np.median(sx, axis=0)) + " |")
    toks = t[found, 7]
    loop = (t[found, 2] - t[found, 1]) * TICK_US
    lines.append("")
    lines.append("Wave 0's loop time by piece size (last launch):")
    lines.append("")
    lines.append("| piece tokens | pieces | loop µs p10 / median / p90 / max |")
    lines.append("|---|---|---|")
    for lo, hi in ((1, 64), (65, 128), (129, 192), (193, 256), (257, 320), (321, 100000)):
        sel = (toks >= lo) & (toks <= hi)
        if sel.any():
            lines.append(f"| {lo}–{hi if hi < 100000 else '…'} | {int(sel.sum())} | {_q(loop[sel])} |")
    return "\n".join(lines)


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--launches", type=int, default=6)
    args = p.parse_args(argv)
    if not torch.cuda.is_available():
        print("timeline_c2 needs a ROCm GPU", file=sys.stderr)
        return 2
    if not TIMELINE_LIB_PATH.exists():
        print(f"{TIMELINE_LIB_PATH.name} is not built: python -m flexengine_amd.build --timeline",
              file=sys.stderr)
        return 2
    print(summarize(run(args.launches)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
