"""FlexEngine attention-backend interface on the HIP kernels.

Two entry forms, matching the reference's plugin surface:

* per request: attention_for_request(q, cache, layer, request_id, length,
  positions, backend="hip") -- the signature of
  src/flexengine/inference/attention/paged.py:18-19.  One-token queries go to
  the fused decode kernel, multi-token chunks to the ragged prefill kernel.
* batched decode: paged_decode_batch(q, cache, layer, block_tables, positions,
  active_mask) -- the signature shared by triton_paged_decode_batch
  (src/flexengine/inference/kernels/paged_attention.py:142) and
  flashinfer_paged_decode_batch (inference/attention/flashinfer_backend.py:33).

`cache` is anything with the reference PagedKVCache's attributes: `.k` / `.v`
pools [layers, NB, BS, Hkv, D], `.tables` (request id -> block list) and
`.layout.kv_heads`; the reference's own PagedKVCache and
flexengine_amd.kv_cache.PagedKVCache both qualify.  The scale is 1/sqrt(D), as
in the reference (paged.py:26).  Errors: ValueError for bad shapes or an
unknown backend, RuntimeError when the HIP library or a GPU is missing --
there is no silent fallback.
"""
from __future__ import annotations

import math

import torch

from flexengine_amd import ops

BACKENDS = ("hip",)


def _check_query(q: torch.Tensor, positions: torch.Tensor, cache) -> int:
    if q.ndim != 3 or positions.ndim != 1 or len(q) != len(positions):
        raise ValueError("invalid query shape")
    if q.shape[1] % cache.layout.kv_heads:
        raise ValueError("Q heads must be a multiple of KV heads")
    return q.shape[1] // cache.layout.kv_heads


def attention_for_request(q: torch.Tensor, cache, layer: int, request_id: str, length: int,
                          positions: torch.Tensor, backend: str = "hip") -> torch.Tensor:
    """q [Q, Hq, D] at absolute positions `positions` (the last `Q` of `length`
    tokens); returns [Q, Hq, D] in q's dtype, causal per request."""
    _check_query(q, positions, cache)
    if backend not in BACKENDS:
        raise ValueError("Unknown attention backend")
    table_list = cache.tables[request_id]
    if length <= 0 or length > len(table_list) * cache.layout.block_size:
        raise ValueError("requested length is invalid/unreserved")
    table = torch.tensor([table_list], dtype=torch.int32).to(q.device, non_blocking=True)
    scale = 1.0 / math.sqrt(q.shape[-1])
    if len(q) == 1:
        ctx = torch.tensor([length], dtype=torch.int32).to(q.device, non_blocking=True)
        return ops.paged_decode(q, cache.k[layer], cache.v[layer], table, ctx, scale=scale)
    ctx = torch.tensor([length], dtype=torch.int32).to(q.device, non_blocking=True)
    offs = torch.tensor([0, len(q)], dtype=torch.int32).to(q.device, non_blocking=True)
    return ops.prefill_paged(q.contiguous(), cache.k[layer], cache.v[layer], table, offs, ctx,
                             len(q), scale=scale)


def context_lens_from_positions(positions: torch.Tensor, active_mask: torch.Tensor) -> torch.Tensor:
    """The batched contract's (positions, active_mask) -> int32 context lengths:
    length = position + 1 for active rows, 0 (-> zero output) otherwise
    (paged_attention.py:115,131,138)."""
    active = active_mask.reshape(-1) != 0
    return torch.where(active, positions.reshape(-1) + 1, torch.zeros_like(positions.reshape(-1))).to(
        torch.int32)


def paged_decode_batch(q: torch.Tensor, cache, layer: int, block_tables: torch.Tensor,
                       positions: torch.Tensor, active_mask: torch.Tensor, *,
                       k_new: torch.Tensor | None = None,
                       v_new: torch.Tensor | None = None) -> torch.Tensor:
    """Batched single-token decode: q [B, Hq, D], block_tables [B, W] (int32 or int64),
    positions [B] (query position = length - 1), active_mask [B] -> [B, Hq, D].

    With k_new/v_new ([B, Hkv, D]) the rows are first written at `positions`
    of each active sequence (the decode-step page write of qwen2.py:156-161),
    inside the same kernel launch.
    """
    if q.ndim != 3 or positions.shape != (q.shape[0],) or active_mask.reshape(-1).shape != (q.shape[0],):
        raise ValueError("invalid static decode inputs")
    if q.shape[1] % cache.layout.kv_heads:
        raise ValueError("Q heads must be a multiple of KV heads")
    ctx = context_lens_from_positions(positions, active_mask)
    tables = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    return ops.paged_decode(q, cache.k[layer], cache.v[layer], tables, ctx,
                            scale=1.0 / math.sqrt(q.shape[-1]), k_new=k_new, v_new=v_new)


def prefill_batch(q: torch.Tensor, cache, layer: int, block_tables: torch.Tensor,
                  q_offsets: torch.Tensor, context_lens: torch.Tensor, max_q_len: int) -> torch.Tensor:
    """Ragged chunked prefill of several requests in one launch (the per-request
    loop of qwen2.py:117-126 fused): q [total_q, Hq, D]."""
    return ops.prefill_paged(q, cache.k[layer], cache.v[layer], block_tables, q_offsets,
                             context_lens, max_q_len, scale=1.0 / math.sqrt(q.shape[-1]))
