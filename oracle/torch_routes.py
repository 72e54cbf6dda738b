"""PyTorch-CPU restatement of the reference's two attention routes.

TEST INFRASTRUCTURE ONLY (see oracle/paged_ref.py).  bench.py times these on
the host cores as the CPU baseline (`cpu_baseline.kind = "port"`); tests check
them against oracle/paged_ref.py.

materialized_route restates attention_for_request(..., "materialized"),
src/flexengine/inference/attention/paged.py:25-35, with the gather of
PagedKVCache.materialize (engine/kv_cache/allocator.py:107-114,129-134):
per request, index the pool with (table[p // bs], p % bs), repeat_interleave
the KV heads, and call scaled_dot_product_attention with the boolean mask
key_pos <= position, in the pool dtype.

blockwise_route restates the blockwise route, paged.py:50-70, walking pages
like PagedKVCache.iter_blocks (allocator.py:136-145): fp32 online softmax,
about ten small torch ops per page.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def _locators(table: list[int], start: int, count: int, block_size: int, device):
    slots = range(start, start + count)
    ids = torch.tensor([table[i // block_size] for i in slots], dtype=torch.long, device=device)
    offs = torch.tensor([i % block_size for i in slots], dtype=torch.long, device=device)
    return ids, offs


def materialized_route(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                       table: list[int], length: int, positions: torch.Tensor) -> torch.Tensor:
    """q [Q, Hq, D]; pools [NB, BS, Hkv, D] (one layer) -> [Q, Hq, D] in q.dtype."""
    ratio = q.shape[1] // k_pool.shape[2]
    ids, offs = _locators(table, 0, length, k_pool.shape[1], q.device)
    k, v = k_pool[ids, offs], v_pool[ids, offs]
    k = k.repeat_interleave(ratio, dim=1).transpose(0, 1).unsqueeze(0)
    v = v.repeat_interleave(ratio, dim=1).transpose(0, 1).unsqueeze(0)
    query = q.transpose(0, 1).unsqueeze(0)
    key_pos = torch.arange(length, device=q.device)
    mask = (key_pos.unsqueeze(0) <= positions.unsqueeze(1)).unsqueeze(0).unsqueeze(0)
    return F.scaled_dot_product_attention(query, k, v, attn_mask=mask, dropout_p=0.0,
                                          is_causal=False).squeeze(0).transpose(0, 1)


def blockwise_route(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                    table: list[int], length: int, positions: torch.Tensor) -> torch.Tensor:
    ratio = q.shape[1] // k_pool.shape[2]
    bs = k_pool.shape[1]
    scale = 1.0 / math.sqrt(q.shape[-1])
    q32 = q.float()
    run_max = torch.full((q.shape[0], q.shape[1]), -float("inf"))
    run_sum = torch.zeros_like(run_max)
    run_val = torch.zeros((*run_max.shape, q.shape[-1]), dtype=torch.float32)
    for j, bid in enumerate(table):
        start = j * bs
        if start >= length:
            break
        n = min(bs, length - start)
        kh = k_pool[bid, :n].float().repeat_interleave(ratio, dim=1)
        vh = v_pool[bid, :n].float().repeat_interleave(ratio, dim=1)
        scores = torch.einsum("qhd,thd->qht", q32, kh) * scale
        valid = (torch.arange(n) + start).unsqueeze(0) <= positions.unsqueeze(1)
        scores = scores.masked_fill(~valid.unsqueeze(1), -float("inf"))
        newmax = torch.maximum(run_max, scores.max(dim=-1).values)
        alpha = torch.exp(torch.where(torch.isfinite(run_max), run_max - newmax,
                                      torch.full_like(newmax, -float("inf"))))
        weights = torch.exp(scores - newmax.unsqueeze(-1))
        weights = torch.where(valid.unsqueeze(1), weights, torch.zeros_like(weights))
        run_val = run_val * alpha.unsqueeze(-1) + torch.einsum("qht,thd->qhd", weights, vh)
        run_sum = run_sum * alpha + weights.sum(-1)
        run_max = newmax
    return (run_val / run_sum.clamp_min(1e-12).unsqueeze(-1)).to(q.dtype)


def decode_batch_materialized(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                              tables: list[list[int]], context_lens: list[int]) -> torch.Tensor:
    """The per-request loop the reference engine runs for a decode batch (qwen2.py:117-126)."""
    out = torch.zeros_like(q)
    for b, length in enumerate(context_lens):
        if length <= 0:
            continue
        pos = torch.tensor([length - 1])
        out[b:b + 1] = materialized_route(q[b:b + 1], k_pool, v_pool, tables[b], length, pos)
    return out


def decode_batch_blockwise(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                           tables: list[list[int]], context_lens: list[int]) -> torch.Tensor:
    """The same per-request loop on the blockwise route (paged.py:50-70)."""
    out = torch.zeros_like(q)
    for b, length in enumerate(context_lens):
        if length <= 0:
            continue
        pos = torch.tensor([length - 1])
        out[b:b + 1] = blockwise_route(q[b:b + 1], k_pool, v_pool, tables[b], length, pos)
    return out
