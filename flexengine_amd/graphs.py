"""Decode steps recorded as HIP graphs, one graph per batch bucket.

The public surface is that of FlexEngine's DecodeGraphManager
(src/flexengine/engine/execution/cuda_graph.py:18-125), which its engine
drives (src/flexengine/engine/runtime.py:43-49,215-240): the constructor
(device, buckets=(1, 2, 4, 8)), bucket_for, eligible, capture(bucket, decode,
example_inputs), staging_addresses, has_capture, replay(active_count, inputs),
run, record_fallback, and stats / stats_delta with the keys captures, replays,
fallbacks, padded_slots and graph_pool_bytes.  Semantics kept: an active batch
of n rows replays the smallest bucket >= n with rows n.. padded (inputs zero,
active mask 0); staging tensors keep their addresses for the life of the
graph; batches above every bucket run eagerly and count as fallbacks;
ValueError for a bucket that cannot be captured and for inputs that do not
match the capture.  On ROCm torch.cuda.CUDAGraph is a hipGraph, so a replay
launches the whole recorded step -- HIP kernels, library GEMMs, elementwise
ops -- as one graph.

Organisation:

* A `_BucketGraph` owns every buffer whose address its graph recorded: the
  staging inputs, the active mask, the output, and each library workspace the
  decode asked for while it was warmed up and captured
  (ops.hold_workspaces()).  The library replaces a per-device workspace with a
  larger one when a call needs more bytes; the record keeps the older buffer
  alive, so capturing bucket 8 after bucket 1, or an eager step of 64 rows
  between replays, never leaves an earlier graph writing into freed memory.
* Bucket lookup is a table indexed by the active count.
* Replay copies the active rows into the staging tensors and clears only the
  padded tail (a copy and a fill per input); the mask likewise.

Rules for what is captured: no host synchronisation, no allocation outside the
graph pool, and no hipMemsetAsync node (clear with a fill kernel instead); the
paged-attention kernels and the model's decode step keep all three.
"""
from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass, field

import torch

from flexengine_amd import ops

_STAT_KEYS = ("captures", "replays", "fallbacks", "padded_slots", "graph_pool_bytes")


@dataclass
class _BucketGraph:
    rows: int
    graph: torch.cuda.CUDAGraph
    staging: dict[str, torch.Tensor]
    mask: torch.Tensor
    output: torch.Tensor
    workspaces: list[torch.Tensor] = field(default_factory=list)

    def addresses(self) -> dict[str, int]:
        addrs = {name: t.data_ptr() for name, t in self.staging.items()}
        addrs["active_mask"] = self.mask.data_ptr()
        addrs["output"] = self.output.data_ptr()
        return addrs


class DecodeGraphManager:
    def __init__(self, device: str | torch.device = "cuda:0", buckets=(1, 2, 4, 8)):
        self.device = torch.device(device)
        sizes = sorted({int(b) for b in buckets})
        if not sizes or sizes[0] < 1:
            raise ValueError(f"bucket sizes must be positive integers, got {tuple(buckets)}")
        self.buckets = tuple(sizes)
        # _fit[n] = smallest bucket holding n rows, for n = 0 .. largest bucket
        self._fit: list[int | None] = [None] * (sizes[-1] + 1)
        smallest_above = None
        for n in range(sizes[-1], 0, -1):
            if n in sizes:
                smallest_above = n
            self._fit[n] = smallest_above
        self._graphs: dict[int, _BucketGraph] = {}
        self._stats = dict.fromkeys(_STAT_KEYS, 0)

    # ---- bucket selection ------------------------------------------------------------

    def bucket_for(self, active_count: int) -> int | None:
        """Smallest bucket holding active_count rows; None for counts < 1 or above
        every bucket."""
        return self._fit[active_count] if 0 < active_count < len(self._fit) else None

    def eligible(self, active_count: int) -> bool:
        return (self.device.type == "cuda" and torch.cuda.is_available()
                and self.bucket_for(active_count) is not None)

    def has_capture(self, bucket: int) -> bool:
        return bucket in self._graphs

    # ---- capture ---------------------------------------------------------------------

    def capture(self, bucket: int, decode: Callable[..., torch.Tensor],
                example_inputs: Mapping[str, torch.Tensor]) -> None:
        """Records decode(**staging, active_mask=mask) for a batch of `bucket` rows;
        example_inputs give the staging tensors' shapes and first contents."""
        if bucket not in self.buckets or not self.eligible(bucket):
            raise ValueError(f"bucket {bucket} cannot be captured (buckets {self.buckets}, "
                             f"device {self.device})")
        if not example_inputs:
            raise ValueError("capture needs at least one staged input")
        for name, t in example_inputs.items():
            if t.device != self.device or t.ndim == 0 or t.shape[0] != bucket:
                raise ValueError(f"staged input {name!r} must be on {self.device} with "
                                 f"{bucket} rows")
        staging = {name: t.clone() for name, t in example_inputs.items()}
        ndim = next(iter(staging.values())).ndim
        mask = torch.ones((bucket,) + (1,) * (ndim - 1), device=self.device)
        with ops.hold_workspaces() as held:
            graph, output, pool_bytes = self._record(decode, staging, mask)
        self._graphs[bucket] = _BucketGraph(bucket, graph, staging, mask, output, list(held))
        self._stats["captures"] += 1
        self._stats["graph_pool_bytes"] += pool_bytes

    def _record(self, decode: Callable[..., torch.Tensor], staging: dict[str, torch.Tensor],
                mask: torch.Tensor):
        """(graph, output, graph-pool bytes) of decode on the staging tensors."""
        cur = torch.cuda.current_stream(self.device)
        # one eager run first, on a side stream, so lazy set-up (library handles,
        # workspace growth) happens before the capture starts
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            decode(**staging, active_mask=mask)
        cur.wait_stream(side)
        torch.cuda.synchronize(self.device)
        pool_before = torch.cuda.memory_reserved(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            output = decode(**staging, active_mask=mask)
        return graph, output, max(0, torch.cuda.memory_reserved(self.device) - pool_before)

    def staging_addresses(self, bucket: int) -> dict[str, int]:
        return self._graphs[bucket].addresses()

    def workspaces(self, bucket: int) -> list[torch.Tensor]:
        """The library workspaces the bucket's graph recorded (held by its record)."""
        return list(self._graphs[bucket].workspaces)

    # ---- replay ----------------------------------------------------------------------

    def replay(self, active_count: int, inputs: Mapping[str, torch.Tensor]) -> torch.Tensor:
        """Runs the graph of the bucket holding active_count rows on `inputs` (each
        with active_count rows); returns a copy of the output's active rows."""
        bucket = self.bucket_for(active_count)
        rec = self._graphs.get(bucket) if bucket is not None else None
        if rec is None:
            raise ValueError(f"no graph captured for {active_count} active rows")
        if set(inputs) != set(rec.staging):
            raise ValueError(f"replay inputs {sorted(inputs)} differ from the captured "
                             f"{sorted(rec.staging)}")
        n = active_count
        for name, src in inputs.items():
            dst = rec.staging[name]
            if src.shape[0] != n or src.shape[1:] != dst.shape[1:]:
                raise ValueError(f"input {name!r} of shape {tuple(src.shape)} does not fit the "
                                 f"staging {tuple(dst.shape)} with {n} active rows")
        for name, src in inputs.items():
            dst = rec.staging[name]
            dst[:n].copy_(src)
            if n < rec.rows:
                dst[n:].zero_()
        rec.mask[:n].fill_(1)
        if n < rec.rows:
            rec.mask[n:].zero_()
        rec.graph.replay()
        self._stats["replays"] += 1
        self._stats["padded_slots"] += rec.rows - n
        return rec.output[:n].clone()

    def run(self, decode: Callable[..., torch.Tensor], inputs: Mapping[str, torch.Tensor]) -> torch.Tensor:
        """Replays the graph of the batch's bucket when one is captured, otherwise
        runs decode(**inputs) eagerly and counts a fallback."""
        if not inputs:
            raise ValueError("decode needs at least one input")
        n = next(iter(inputs.values())).shape[0]
        if self.bucket_for(n) in self._graphs:
            return self.replay(n, inputs)
        self._stats["fallbacks"] += 1
        return decode(**inputs)

    # ---- statistics ------------------------------------------------------------------

    def record_fallback(self) -> None:
        self._stats["fallbacks"] += 1

    def stats(self) -> dict[str, int]:
        return dict(self._stats)

    def stats_delta(self, before: Mapping[str, int]) -> dict[str, int]:
        now = self.stats()
        if set(before) != set(now):
            raise ValueError(f"stats snapshot keys {sorted(before)} differ from {sorted(now)}")
        return {key: now[key] - before[key] for key in now}
