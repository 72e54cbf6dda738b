"""Graph-replayed decode steps of the package's Qwen2 model.

The engine side of FlexEngine's CUDA-graph decode path
(src/flexengine/engine/runtime.py:43-49,201-240) on hipGraph:

* at start-up, one scratch request reserves max(buckets) * block_size slots;
  its blocks pad the block tables of rows that hold no request
  (runtime.py:45-49,201-213);
* a step whose chunks are all single tokens runs in the smallest captured
  bucket >= the active count, capturing the bucket on first use with the
  model's decode_static; batches above every bucket, and any RuntimeError or
  ValueError during capture or replay, are counted as fallbacks and return
  None so the caller runs the eager path (runtime.py:215-240).
"""
from __future__ import annotations

import torch

from flexengine_amd.graphs import DecodeGraphManager

SCRATCH_ID = "__flex_graph_scratch__"


class GraphDecodeStep:
    def __init__(self, model, cache, max_model_len: int, manager: DecodeGraphManager | None = None):
        self.model = model
        self.cache = cache
        self.manager = manager or DecodeGraphManager(cache.device)
        bs = cache.layout.block_size
        self.max_blocks = (max_model_len + bs - 1) // bs
        cache.reserve(SCRATCH_ID, max(self.manager.buckets) * bs)
        self.scratch_blocks = list(cache.tables[SCRATCH_ID])

    def graph_inputs(self, chunks, batch_size: int) -> dict[str, torch.Tensor]:
        """Padded staging rows (runtime.py:201-213): active rows carry their token,
        position and block table, padded rows and table tails a scratch block.  The
        tables are gathered on the device from the cache's mirror rows
        (fe_gather_tables): a step copies one row index per request, not its table.
        (Rows without a request are never written here -- their context length is 0 --
        so they need no scratch slot of their own, unlike the reference's.)"""
        if len(chunks) > batch_size:
            raise ValueError("more chunks than batch rows")
        ids = torch.zeros(batch_size, dtype=torch.long)
        positions = torch.zeros(batch_size, dtype=torch.long)
        bs = self.cache.layout.block_size
        for row, chunk in enumerate(chunks):
            if self.cache.available_slots(chunk.request_id) > self.max_blocks * bs:
                raise ValueError(f"request {chunk.request_id!r} holds more blocks than "
                                 f"max_model_len allows ({self.max_blocks})")
            ids[row] = chunk.input_ids[0]
            positions[row] = chunk.start
        requests = [c.request_id for c in chunks] + [None] * (batch_size - len(chunks))
        tables = self.cache.device_tables(requests, self.max_blocks, pad_block=self.scratch_blocks[0])
        dev = self.cache.device
        return {"input_ids": ids.to(dev), "positions": positions.to(dev), "block_tables": tables}

    def _decode(self, input_ids, positions, block_tables, active_mask):
        return self.model.decode_static(input_ids, positions, block_tables, active_mask, self.cache)

    def __call__(self, chunks) -> list[torch.Tensor] | None:
        """Logits per chunk from a graph replay, or None when the step must run eagerly."""
        if not chunks or not all(len(c.input_ids) == 1 for c in chunks):
            return None
        active = len(chunks)
        bucket = self.manager.bucket_for(active)
        if bucket is None:
            self.manager.record_fallback()
            return None
        try:
            if not self.manager.has_capture(bucket):
                self.manager.capture(bucket, self._decode, self.graph_inputs(chunks, bucket))
            output = self.manager.replay(active, self.graph_inputs(chunks, active))
            return [output[row] for row in range(active)]
        except (RuntimeError, ValueError):
            self.manager.record_fallback()
            return None
