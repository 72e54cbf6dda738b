"""CPU oracle for FlexEngine's paged-attention hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or, in the
bench, as the timed CPU baseline).  The product path (flexengine_amd) never
imports or calls it.

This is a numpy restatement of the reference's algorithm, computed in float64
where the reference accumulates in floating point, so that it is at least as
accurate as the reference's fp32-accumulated routes.  Each function cites the
reference file:line it restates (paths relative to the FlexEngine source tree,
src/flexengine/...).

How each function is pinned (tests/test_oracle.py):
  locators / write_kv / materialize / write_kv_decode
      - the reference's own known-answer test (test_allocator.py:11-29: arange
        rows written across a block boundary read back exactly);
      - the non-contiguous table scenario of test_attention.py:25-36;
      - brute force: every written slot holds its row, every other slot is
        unchanged (byte equality).
  attention_materialized
      - torch.nn.functional.scaled_dot_product_attention in float64 (an
        independent library routine) with the reference's boolean mask;
      - closed forms: L = 1 gives v[0]; constant keys give the mean of V;
        permutation invariance of physical blocks.
  attention_blockwise
      - equals attention_materialized to 1e-5 for the reference's own grid of
        lengths 1,3,4,5,15,16,17,34 x query counts 1,2,3 at
        CacheLayout(2,20,4,2,8) (test_attention.py:8-22).
  lse_merge / split_attention
      - scipy.special.logsumexp / softmax, and: merging the splits of a key
        range equals attention over the whole range.
  decode_reference / paged_decode_batch / prefill_reference
      - defined through attention_materialized over gathered pages; pinned by
        the above plus the inactive-row rule (exact zeros) of
        paged_attention.py:131,138, and prefill == per-query-row decode.
Plant-a-mistake tests in tests/test_oracle.py show that a wrong GQA head map, a
wrong scale or an off-by-one causal mask in this module fails those checks.
"""
from __future__ import annotations

import math

import numpy as np

# ------------------------------------------------------------------------------------
# KV pool: slot mapping, page write, gather
# ------------------------------------------------------------------------------------


def locators(table, start: int, count: int, block_size: int) -> tuple[np.ndarray, np.ndarray]:
    """(block id, in-block offset) of logical slots start..start+count-1.

    Restates PagedKVCache._locators, engine/kv_cache/allocator.py:107-114.
    """
    if start < 0 or count < 0 or start + count > len(table) * block_size:
        raise IndexError("KV slots not reserved")
    slots = np.arange(start, start + count)
    ids = np.asarray(table, dtype=np.int64)[slots // block_size]
    offs = slots % block_size
    return ids, offs


def write_kv(pool_k: np.ndarray, pool_v: np.ndarray, table, start: int, keys: np.ndarray,
             values: np.ndarray, block_size: int) -> None:
    """pool[table[p//bs], p%bs] = rows, for p in [start, start+n); in place.

    pool_k/pool_v: [NB, BS, Hkv, D] (one layer).  Restates PagedKVCache.write,
    engine/kv_cache/allocator.py:116-127 (without the shared-block refcount
    check, which is host bookkeeping).
    """
    if keys.shape != values.shape or keys.ndim != 3:
        raise ValueError("K/V shapes must be [tokens, kv_heads, head_dim]")
    ids, offs = locators(table, start, keys.shape[0], block_size)
    pool_k[ids, offs] = keys
    pool_v[ids, offs] = values


def materialize(pool: np.ndarray, table, length: int, block_size: int) -> np.ndarray:
    """Gathers logical rows 0..length-1 to a contiguous [length, Hkv, D].

    Restates PagedKVCache.materialize, engine/kv_cache/allocator.py:129-134.
    """
    if length <= 0:
        raise ValueError("length must be >0")
    ids, offs = locators(table, 0, length, block_size)
    return pool[ids, offs]


def write_kv_decode(pool_k: np.ndarray, pool_v: np.ndarray, block_tables: np.ndarray,
                    context_lens: np.ndarray, k: np.ndarray, v: np.ndarray,
                    block_size: int) -> None:
    """Decode-step write of row b at position context_lens[b]-1; rows with 0 skipped.

    Restates the graph-path write of Qwen2Adapter.decode_static,
    inference/models/qwen2.py:156-161: block = tables[b, pos // bs],
    offset = pos % bs, with context_lens = (positions + 1) * active.  The
    reference rewrites the old value for inactive rows; skipping them leaves
    the pool byte-identical.
    """
    for b, length in enumerate(np.asarray(context_lens)):
        if length <= 0:
            continue
        pos = int(length) - 1
        blk = int(block_tables[b, pos // block_size])
        pool_k[blk, pos % block_size] = k[b]
        pool_v[blk, pos % block_size] = v[b]


# ------------------------------------------------------------------------------------
# attention
# ------------------------------------------------------------------------------------


def attention_materialized(q: np.ndarray, k: np.ndarray, v: np.ndarray, positions,
                           scale: float | None = None) -> np.ndarray:
    """Causal GQA attention over gathered keys, float64, returns float64 [Q, Hq, D].

    q [Q, Hq, D]; k, v [Lk, Hkv, D]; key t is visible to query row i iff
    t <= positions[i]; query head h reads KV head h // (Hq // Hkv).
    Restates the materialized route of attention_for_request,
    inference/attention/paged.py:25-35 (repeat_interleave over heads, boolean
    mask key_pos <= position, SDPA with scale 1/sqrt(D)).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    nq, hq, d = q.shape
    hkv = k.shape[1]
    if hq % hkv:
        raise ValueError("Q heads must be a multiple of KV heads")
    ratio = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    kh = np.repeat(k, ratio, axis=1)  # [Lk, Hq, D], head h -> kv head h // ratio
    vh = np.repeat(v, ratio, axis=1)
    scores = np.einsum("qhd,thd->qht", q, kh) * scale
    key_pos = np.arange(k.shape[0])
    mask = key_pos[None, :] <= np.asarray(positions)[:, None]  # [Q, Lk]
    scores = np.where(mask[:, None, :], scores, -np.inf)
    mx = scores.max(axis=-1, keepdims=True)
    w = np.exp(scores - mx)
    w = np.where(mask[:, None, :], w, 0.0)
    w /= w.sum(axis=-1, keepdims=True)
    return np.einsum("qht,thd->qhd", w, vh)


def attention_blockwise(q: np.ndarray, pool_k: np.ndarray, pool_v: np.ndarray, table,
                        length: int, positions, block_size: int,
                        scale: float | None = None) -> np.ndarray:
    """Online softmax over physical pages, float32, returns float32 [Q, Hq, D].

    Restates the blockwise route, inference/attention/paged.py:50-70, and the
    page iteration of PagedKVCache.iter_blocks, allocator.py:136-145:
      m' = max(m, max s);  alpha = exp(m - m') (0 while m = -inf);
      acc = acc*alpha + sum p v;  l = l*alpha + sum p;  out = acc / max(l, 1e-12)
    """
    q32 = np.asarray(q, dtype=np.float32)
    nq, hq, d = q32.shape
    hkv = pool_k.shape[2]
    ratio = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    pos = np.asarray(positions)
    run_max = np.full((nq, hq), -np.inf, dtype=np.float32)
    run_sum = np.zeros((nq, hq), dtype=np.float32)
    run_val = np.zeros((nq, hq, d), dtype=np.float32)
    for j, bid in enumerate(table):
        start = j * block_size
        if start >= length:
            break
        n = min(block_size, length - start)
        kb = np.repeat(pool_k[bid, :n].astype(np.float32), ratio, axis=1)
        vb = np.repeat(pool_v[bid, :n].astype(np.float32), ratio, axis=1)
        scores = np.einsum("qhd,thd->qht", q32, kb) * np.float32(scale)
        valid = (np.arange(n) + start)[None, :] <= pos[:, None]
        scores = np.where(valid[:, None, :], scores, -np.inf).astype(np.float32)
        new_max = np.maximum(run_max, scores.max(axis=-1))
        with np.errstate(invalid="ignore"):
            alpha = np.where(np.isfinite(run_max), np.exp(run_max - new_max), 0.0).astype(np.float32)
            weights = np.where(valid[:, None, :], np.exp(scores - new_max[..., None]), 0.0)
        weights = weights.astype(np.float32)
        run_val = run_val * alpha[..., None] + np.einsum("qht,thd->qhd", weights, vb)
        run_sum = run_sum * alpha + weights.sum(-1)
        run_max = new_max
    return run_val / np.maximum(run_sum, np.float32(1e-12))[..., None]


def decode_reference(q: np.ndarray, pool_k: np.ndarray, pool_v: np.ndarray,
                     block_tables: np.ndarray, context_lens, block_size: int,
                     scale: float | None = None) -> np.ndarray:
    """Batched single-token decode with the C ABI's convention, float64 [B, Hq, D].

    Row b attends to keys 0..context_lens[b]-1 of its table (the query is the
    last of them); rows with context length 0 give exact zeros.  This is
    triton_paged_decode_batch (inference/kernels/paged_attention.py:99-155)
    with length = positions + 1 and inactive rows zeroed (:115, :131, :138),
    evaluated through the materialized route (paged.py:27-35).
    """
    q = np.asarray(q)
    out = np.zeros(q.shape, dtype=np.float64)
    for b, length in enumerate(np.asarray(context_lens)):
        length = int(length)
        if length <= 0:
            continue
        k = materialize(pool_k, block_tables[b], length, block_size)
        v = materialize(pool_v, block_tables[b], length, block_size)
        out[b] = attention_materialized(q[b:b + 1], k, v, [length - 1], scale)[0]
    return out


def paged_decode_batch(q: np.ndarray, pool_k: np.ndarray, pool_v: np.ndarray,
                       block_tables: np.ndarray, positions, active_mask, block_size: int,
                       scale: float | None = None) -> np.ndarray:
    """The reference's batched backend contract (positions + active mask).

    Restates triton_paged_decode_batch / flashinfer_paged_decode_batch's
    contract, inference/kernels/paged_attention.py:142-155 and
    inference/attention/flashinfer_backend.py:33-72: length = positions[b] + 1,
    inactive rows -> zeros.
    """
    ctx = (np.asarray(positions) + 1) * (np.asarray(active_mask) != 0)
    return decode_reference(q, pool_k, pool_v, block_tables, ctx, block_size, scale)


def prefill_reference(q: np.ndarray, q_offsets, context_lens, pool_k: np.ndarray,
                      pool_v: np.ndarray, block_tables: np.ndarray, block_size: int,
                      scale: float | None = None) -> np.ndarray:
    """Ragged chunked prefill, float64 [total_q, Hq, D].

    Sequence s owns rows q_offsets[s]..q_offsets[s+1]-1 at absolute positions
    ctx_s - n_s .. ctx_s - 1 and attends causally over its paged keys.  This
    is the per-request loop of Qwen2Adapter.forward (inference/models/
    qwen2.py:117-126) calling the materialized route (paged.py:27-35) with
    positions start..start+n-1.
    """
    q = np.asarray(q)
    out = np.zeros(q.shape, dtype=np.float64)
    q_offsets = np.asarray(q_offsets)
    for s, ctx in enumerate(np.asarray(context_lens)):
        a, b = int(q_offsets[s]), int(q_offsets[s + 1])
        n, ctx = b - a, int(ctx)
        if n <= 0:
            continue
        k = materialize(pool_k, block_tables[s], ctx, block_size)
        v = materialize(pool_v, block_tables[s], ctx, block_size)
        out[a:b] = attention_materialized(q[a:b], k, v, np.arange(ctx - n, ctx), scale)
    return out


# ------------------------------------------------------------------------------------
# split-K: partial results and the log-sum-exp merge
# ------------------------------------------------------------------------------------


def split_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, bounds,
                    scale: float | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Attention of q [R, D] over key ranges bounds[s]..bounds[s+1] of k, v [Lk, D].

    Returns part_out [S, R, D] (each normalised by its own denominator) and
    part_lse [S, R] (natural log of that denominator plus the max); an empty
    range gives lse = -inf and zeros.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    outs, lses = [], []
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        if hi <= lo:
            outs.append(np.zeros((q.shape[0], q.shape[1])))
            lses.append(np.full(q.shape[0], -np.inf))
            continue
        s = q @ k[lo:hi].T * scale
        mx = s.max(axis=1, keepdims=True)
        p = np.exp(s - mx)
        den = p.sum(axis=1, keepdims=True)
        outs.append((p @ v[lo:hi]) / den)
        lses.append((mx + np.log(den))[:, 0])
    return np.stack(outs), np.stack(lses)


def lse_merge(part_out: np.ndarray, part_lse: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """LSE = log sum_s exp(lse_s);  out = sum_s exp(lse_s - LSE) out_s.

    The combine identity of split softmax; the reference computes the same
    quantity in one pass with its running max / sum (paged.py:60-70).  Rows
    whose every split is empty give zeros and -inf.
    """
    part_out = np.asarray(part_out, dtype=np.float64)
    part_lse = np.asarray(part_lse, dtype=np.float64)
    m = part_lse.max(axis=0)
    safe = np.where(np.isfinite(m), m, 0.0)
    w = np.exp(part_lse - safe[None, :])
    den = w.sum(axis=0)
    with np.errstate(invalid="ignore", divide="ignore"):
        out = np.einsum("sr,srd->rd", w, part_out) / den[:, None]
        lse = safe + np.log(den)
    empty = ~np.isfinite(m)
    out[empty] = 0.0
    lse[empty] = -np.inf
    return out, lse


# ------------------------------------------------------------------------------------
# decode graph buckets
# ------------------------------------------------------------------------------------


def bucket_for(active_count: int, buckets=(1, 2, 4, 8)) -> int | None:
    """Smallest bucket >= active_count, None when none fits or count <= 0.

    Restates DecodeGraphManager.bucket_for, engine/execution/cuda_graph.py:31-34.
    """
    if active_count <= 0:
        return None
    return next((b for b in sorted(set(buckets)) if active_count <= b), None)


def to_fp16(x: np.ndarray) -> np.ndarray:
    """The reference returns attention in the query dtype (paged.py:70)."""
    return np.asarray(x).astype(np.float16)
