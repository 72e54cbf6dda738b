"""Fixed-bucket HIP-graph capture and replay for decode steps.

Same interface and behaviour as FlexEngine's DecodeGraphManager
(src/flexengine/engine/execution/cuda_graph.py:18-125): buckets (1, 2, 4, 8),
an active batch of n runs in the smallest bucket >= n with rows n..bucket-1
padded (staging zeroed, active mask 0), staging buffers keep stable device
addresses, and batches larger than every bucket run eagerly and are counted as
fallbacks.  On ROCm torch.cuda.CUDAGraph is a hipGraph (hipStreamBeginCapture
/ hipGraphInstantiate / hipGraphLaunch), so replays launch the whole captured
decode step -- HIP kernels, GEMMs and elementwise ops -- as one graph.

Capture rules for the decoded step: no host synchronisation, no allocation
outside the graph pool, and no hipMemsetAsync node (clear buffers with a fill
kernel instead); the paged-attention kernels satisfy all three.
"""
from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass

import torch


@dataclass
class _Captured:
    graph: torch.cuda.CUDAGraph
    inputs: dict[str, torch.Tensor]
    active_mask: torch.Tensor
    output: torch.Tensor


class DecodeGraphManager:
    def __init__(self, device: str | torch.device = "cuda:0", buckets=(1, 2, 4, 8)):
        self.device = torch.device(device)
        self.buckets = tuple(sorted(set(buckets)))
        if not self.buckets or self.buckets[0] <= 0:
            raise ValueError("buckets must be positive")
        self._graphs: dict[int, _Captured] = {}
        self._counters = {"captures": 0, "replays": 0, "fallbacks": 0, "padded_slots": 0,
                          "graph_pool_bytes": 0}

    def bucket_for(self, active_count: int) -> int | None:
        """Smallest bucket holding active_count rows; None if none does (or count <= 0)."""
        if active_count <= 0:
            return None
        for bucket in self.buckets:
            if active_count <= bucket:
                return bucket
        return None

    def eligible(self, active_count: int) -> bool:
        return (self.device.type == "cuda" and torch.cuda.is_available()
                and self.bucket_for(active_count) is not None)

    def capture(self, bucket: int, decode: Callable[..., torch.Tensor],
                example_inputs: Mapping[str, torch.Tensor]) -> None:
        """Records decode(**static_inputs, active_mask=mask) for one bucket."""
        if bucket not in self.buckets or not self.eligible(bucket):
            raise ValueError("bucket is not eligible for graph capture")
        if not example_inputs:
            raise ValueError("capture requires inputs")
        for tensor in example_inputs.values():
            if tensor.device != self.device or tensor.shape[0] != bucket:
                raise ValueError("capture inputs must use the configured device and bucket batch size")
        static = {name: tensor.clone() for name, tensor in example_inputs.items()}
        first = next(iter(static.values()))
        mask = torch.ones((bucket,) + (1,) * (first.ndim - 1), device=self.device)
        # warm-up on a side stream so lazy initialisation (GEMM handles, workspaces)
        # happens outside the capture
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            decode(**static, active_mask=mask)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        reserved_before = torch.cuda.memory_reserved(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            output = decode(**static, active_mask=mask)
        self._graphs[bucket] = _Captured(graph, static, mask, output)
        self._counters["captures"] += 1
        self._counters["graph_pool_bytes"] += max(0, torch.cuda.memory_reserved(self.device) - reserved_before)

    def staging_addresses(self, bucket: int) -> dict[str, int]:
        cap = self._graphs[bucket]
        addrs = {name: t.data_ptr() for name, t in cap.inputs.items()}
        addrs["active_mask"] = cap.active_mask.data_ptr()
        addrs["output"] = cap.output.data_ptr()
        return addrs

    def has_capture(self, bucket: int) -> bool:
        return bucket in self._graphs

    def replay(self, active_count: int, inputs: Mapping[str, torch.Tensor]) -> torch.Tensor:
        bucket = self.bucket_for(active_count)
        if bucket is None or bucket not in self._graphs:
            raise ValueError("no captured graph for active batch")
        cap = self._graphs[bucket]
        if set(inputs) != set(cap.inputs):
            raise ValueError("replay input names differ from capture")
        for name, src in inputs.items():
            dst = cap.inputs[name]
            if src.shape[0] != active_count or src.shape[1:] != dst.shape[1:]:
                raise ValueError("replay input shape differs from capture")
            dst.zero_()
            dst[:active_count].copy_(src)
        cap.active_mask.zero_()
        cap.active_mask[:active_count] = 1
        cap.graph.replay()
        self._counters["replays"] += 1
        self._counters["padded_slots"] += bucket - active_count
        return cap.output[:active_count].clone()

    def run(self, decode: Callable[..., torch.Tensor], inputs: Mapping[str, torch.Tensor]) -> torch.Tensor:
        """Replays the bucket's graph if one is captured, else runs decode eagerly."""
        if not inputs:
            raise ValueError("decode requires inputs")
        active_count = next(iter(inputs.values())).shape[0]
        if self.bucket_for(active_count) in self._graphs:
            return self.replay(active_count, inputs)
        self._counters["fallbacks"] += 1
        return decode(**inputs)

    def record_fallback(self) -> None:
        self._counters["fallbacks"] += 1

    def stats(self) -> dict[str, int]:
        return dict(self._counters)

    def stats_delta(self, before: Mapping[str, int]) -> dict[str, int]:
        now = self.stats()
        if set(before) != set(now):
            raise ValueError("graph statistics snapshot has different fields")
        return {name: now[name] - before[name] for name in now}
