"""GPU: ragged chunked-prefill attention (fe_prefill_paged) against the oracle."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flexengine_amd import _lib, attention, ops, workloads
from flexengine_amd.kv_cache import CacheLayout, PagedKVCache
from oracle import paged_ref as R
from tests.parity import assert_attention_close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(seed, n_new, cached, hq=12, hkv=2, d=128, bs=16):
    g = torch.Generator().manual_seed(seed)
    ctx = [c + n for c, n in zip(cached, n_new)]
    pages = [math.ceil(x / bs) for x in ctx]
    nb = sum(pages) + 3
    k_pool = torch.randn(nb, bs, hkv, d, generator=g).half()
    v_pool = torch.randn(nb, bs, hkv, d, generator=g).half()
    perm = torch.randperm(nb, generator=g)
    width = max(pages)
    tables = torch.zeros(len(ctx), width, dtype=torch.int32)
    at = 0
    for i, p in enumerate(pages):
        tables[i, :p] = perm[at:at + p]
        tables[i, p:] = perm[at + p - 1] if p else 0
        at += p
    offs = np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32)
    q = torch.randn(int(offs[-1]), hq, d, generator=g).half()
    return q, torch.tensor(offs), torch.tensor(ctx, dtype=torch.int32), tables, k_pool, v_pool


def _run(q, offs, ctx, tables, kp, vp):
    n_new = (offs[1:] - offs[:-1]).tolist()
    out = ops.prefill_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), tables.to(DEV), offs.to(DEV),
                            ctx.to(DEV), max(n_new) if n_new else 0)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("n_new,cached", [([1], [0]), ([5], [0]), ([16], [0]), ([17], [3]),
                                          ([64], [0]), ([65], [100]), ([130, 7, 1], [0, 40, 999]),
                                          ([0, 33], [10, 10])])
def test_ragged_prefill_small(n_new, cached):
    q, offs, ctx, tables, kp, vp = _case(sum(n_new) + 7 * len(n_new), n_new, cached)
    got = _run(q, offs, ctx, tables, kp, vp)
    exp = R.prefill_reference(q.numpy(), offs.numpy(), ctx.numpy(), kp.numpy(), vp.numpy(),
                              tables.numpy(), 16)
    assert_attention_close(got, exp, what=f"n={n_new} c={cached}")


@pytest.mark.parametrize("hq,hkv,d,bs", [(14, 2, 64, 16), (8, 8, 64, 4), (16, 2, 128, 32)])
def test_prefill_shapes(hq, hkv, d, bs):
    q, offs, ctx, tables, kp, vp = _case(hq + d + bs, [70, 3], [25, 200], hq, hkv, d, bs)
    got = _run(q, offs, ctx, tables, kp, vp)
    exp = R.prefill_reference(q.numpy(), offs.numpy(), ctx.numpy(), kp.numpy(), vp.numpy(),
                              tables.numpy(), bs)
    assert_attention_close(got, exp)


@pytest.mark.parametrize("hq,hkv,d,q_scale", [(6, 1, 128, 16.0), (12, 2, 128, 8.0), (14, 2, 64, 16.0)])
def test_prefill_large_scores(hq, hkv, d, q_scale):
    """q scaled up so scores spread over hundreds: the running max must be the true
    max over every key of a block (all four 16-lane rows of the score tile); a max
    taken over part of them lets exp2 and the fp16 probabilities overflow."""
    q, offs, ctx, tables, kp, vp = _case(77 + hq, [40, 130, 1], [300, 20, 64], hq, hkv, d)
    q = (q.float() * q_scale).half()
    got = _run(q, offs, ctx, tables, kp, vp)
    assert np.isfinite(got).all()
    exp = R.prefill_reference(q.numpy(), offs.numpy(), ctx.numpy(), kp.numpy(), vp.numpy(),
                              tables.numpy(), 16)
    assert_attention_close(got, exp, what=f"large scores x{q_scale}")


def test_c4_prefill_chunks_full():
    w = workloads.c4_workload()
    got = _run(w.q, w.q_offsets, w.context_lens, w.block_tables, w.k_pool, w.v_pool)
    exp = R.prefill_reference(w.q.numpy(), w.q_offsets.numpy(), w.context_lens.numpy(),
                              w.k_pool.numpy(), w.v_pool.numpy(), w.block_tables.numpy(), 16)
    assert_attention_close(got, exp, what="C4 prefill")


def test_c4_decode_rows_full():
    """C4's 48 decode rows (L ~ U{256..4096}) in the same pool as the prefill chunks,
    through the decode kernel, against the float64 oracle."""
    w = workloads.c4_workload().decode
    d = w.to(DEV)
    got = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens)
    torch.cuda.synchronize()
    exp = R.decode_reference(w.q.numpy(), w.k_pool.numpy(), w.v_pool.numpy(),
                             w.block_tables.numpy(), w.context_lens.numpy(), 16)
    assert_attention_close(got.cpu().numpy(), exp, what="C4 decode rows")


def test_c4_whole_step_prefill_and_decode_share_the_pool():
    """The whole C4 step as the benchmark runs it: the prefill launch over the four
    chunks, then the decode launch over the 48 rows, back to back on one stream."""
    w = workloads.c4_workload()
    d = w.to(DEV)
    pre = ops.prefill_paged(d.q, d.k_pool, d.v_pool, d.block_tables, d.q_offsets,
                            d.context_lens, int(max(w.meta["n_new"])))
    dd = d.decode
    dec = ops.paged_decode(dd.q, d.k_pool, d.v_pool, dd.block_tables, dd.context_lens)
    torch.cuda.synchronize()
    exp_pre = R.prefill_reference(w.q.numpy(), w.q_offsets.numpy(), w.context_lens.numpy(),
                                  w.k_pool.numpy(), w.v_pool.numpy(), w.block_tables.numpy(), 16)
    exp_dec = R.decode_reference(w.decode.q.numpy(), w.k_pool.numpy(), w.v_pool.numpy(),
                                 w.decode.block_tables.numpy(), w.decode.context_lens.numpy(), 16)
    assert_attention_close(pre.cpu().numpy(), exp_pre, what="C4 step: prefill")
    assert_attention_close(dec.cpu().numpy(), exp_dec, what="C4 step: decode rows")


def test_per_request_interface_multi_token_chunk():
    """attention_for_request with Q > 1 takes the prefill kernel (the reference routes it to
    the materialized SDPA, test_triton_paged_attention.py:29-41); compare with the oracle."""
    g = torch.Generator().manual_seed(29)
    cache = PagedKVCache(CacheLayout(1, 8, 4, 1, 64), device=DEV)
    cache.reserve("r", 4)
    keys = torch.randn(4, 1, 64, generator=g).half()
    cache.write(0, "r", 0, keys.to(DEV), keys.to(DEV))
    query = torch.randn(4, 2, 64, generator=g).half()
    positions = torch.arange(4, device=DEV)
    got = attention.attention_for_request(query.to(DEV), cache, 0, "r", 4, positions)
    exp = R.attention_materialized(query.numpy(), keys.numpy(), keys.numpy(), np.arange(4))
    assert_attention_close(got.cpu().numpy(), exp)


def test_prefill_then_decode_consistency():
    """The prefill row at position p equals a decode call with context p + 1."""
    q, offs, ctx, tables, kp, vp = _case(5, [40], [60])
    got = _run(q, offs, ctx, tables, kp, vp)
    j = 23
    pos = 60 + j
    dec = ops.paged_decode(q[j:j + 1].to(DEV), kp.to(DEV), vp.to(DEV), tables.to(DEV),
                           torch.tensor([pos + 1], dtype=torch.int32, device=DEV)).cpu().numpy()
    assert np.abs(got[j] - dec[0].astype(np.float64)).max() <= 2e-3


def test_split_prefill_repeated_calls_and_shapes_share_the_workspace():
    """The key-split merge leaves its tickets at zero: repeated calls of different
    shapes on the shared workspace give the same results each time."""
    a = _case(3, [130, 7, 1], [0, 40, 999])
    b = _case(4, [65], [100])
    first_a, first_b = _run(*a), _run(*b)
    for _ in range(3):
        np.testing.assert_array_equal(_run(*a), first_a)
        np.testing.assert_array_equal(_run(*b), first_b)


def test_stream_k_merge_is_deterministic_whoever_merges():
    """A split unit is merged by whichever contributor draws the last ticket, from its
    registers or from memory: the result must not depend on which (same bits on every
    call), and must match the oracle.  C4 splits nearly every unit; 12 calls on 4
    rotating pool copies vary the timing."""
    w = workloads.c4_workload()
    d = w.to(DEV)
    max_q = int((w.q_offsets[1:] - w.q_offsets[:-1]).max())
    pools = [(d.k_pool, d.v_pool)] + [(d.k_pool.clone(), d.v_pool.clone()) for _ in range(3)]
    outs = []
    for i in range(12):
        kp, vp = pools[i % 4]
        outs.append(ops.prefill_paged(d.q, kp, vp, d.block_tables, d.q_offsets, d.context_lens,
                                      max_q))
    torch.cuda.synchronize()
    for i, o in enumerate(outs[1:], 1):
        assert torch.equal(o, outs[0]), f"call {i} differs from call 0"
    exp = R.prefill_reference(w.q.numpy(), w.q_offsets.numpy(), w.context_lens.numpy(),
                              w.k_pool.numpy(), w.v_pool.numpy(), w.block_tables.numpy(), 16)
    assert_attention_close(outs[0].cpu().numpy(), exp, what="C4 repeated")


# --------------------------------------------------------------------------------------
# prefill plan (fe_prefill_plan / fe_prefill_paged_planned): one plan per model step,
# reused by every layer; results must be bit-identical to the unplanned launch
# --------------------------------------------------------------------------------------

def _planned_prefill_cases():
    w = workloads.c4_workload()
    c4 = (w.q, w.q_offsets, w.context_lens, w.block_tables, w.k_pool, w.v_pool, 16)
    small = _case(61, [130, 7, 1], [0, 40, 999]) + (16,)
    bs32 = _case(62, [70, 3], [25, 200], 16, 2, 128, 32) + (32,)
    d64 = _case(63, [300, 1, 45], [0, 2048, 17], 14, 2, 64, 16) + (16,)
    return {"C4": c4, "small": small, "bs32": bs32, "d64-g7": d64}


@pytest.mark.parametrize("name", ["C4", "small", "bs32", "d64-g7"])
def test_planned_prefill_is_bit_identical_and_reusable(name):
    q, offs, ctx, tables, kp, vp, bs = _planned_prefill_cases()[name]
    print(f"planned prefill case {name}", flush=True)
    hq, hkv = q.shape[1], kp.shape[2]
    offs_d, ctx_d, tables_d = offs.to(DEV), ctx.to(DEV), tables.to(DEV)
    max_q = int((offs[1:] - offs[:-1]).max())
    plan = ops.prefill_paged_plan(offs_d, ctx_d, q.shape[0], hq, hkv, tables.shape[1], bs)
    assert plan is not None
    # three "layers": own pools and queries, the same offsets, lengths and tables
    for layer in range(3):
        g = torch.Generator().manual_seed(200 + layer)
        ql = torch.randn(q.shape, generator=g).half().to(DEV)
        kl = torch.randn(kp.shape, generator=g).half().to(DEV)
        vl = torch.randn(vp.shape, generator=g).half().to(DEV)
        ref = ops.prefill_paged(ql, kl, vl, tables_d, offs_d, ctx_d, max_q)
        got = ops.prefill_paged(ql, kl, vl, tables_d, offs_d, ctx_d, max_q, plan=plan)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"{name} layer {layer}: planned output differs"
    got = ops.prefill_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), tables_d, offs_d, ctx_d, max_q,
                            plan=plan)
    exp = R.prefill_reference(q.numpy(), offs.numpy(), ctx.numpy(), kp.numpy(), vp.numpy(),
                              tables.numpy(), bs)
    assert_attention_close(got.cpu().numpy(), exp, what=f"planned {name}")


def test_planned_prefill_bf16_and_refusals():
    """The bf16 planned form matches the bf16 unplanned one bit for bit; a plan for other
    tensors is refused; block sizes the stream-K kernel does not take have no plan."""
    q, offs, ctx, tables, kp, vp, bs = _planned_prefill_cases()["small"]
    qb, kb, vb = (t.float().to(torch.bfloat16).to(DEV) for t in (q, kp, vp))
    offs_d, ctx_d, tables_d = offs.to(DEV), ctx.to(DEV), tables.to(DEV)
    max_q = int((offs[1:] - offs[:-1]).max())
    plan = ops.prefill_paged_plan(offs_d, ctx_d, q.shape[0], q.shape[1], kp.shape[2],
                                  tables.shape[1], bs)
    ref = ops.prefill_paged(qb, kb, vb, tables_d, offs_d, ctx_d, max_q)
    got = ops.prefill_paged(qb, kb, vb, tables_d, offs_d, ctx_d, max_q, plan=plan)
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16 and torch.equal(got, ref)
    with pytest.raises(ValueError, match="other q_offsets"):
        ops.prefill_paged(qb, kb, vb, tables_d, offs_d, ctx_d.clone(), max_q, plan=plan)
    q4, offs4, ctx4, tables4, _, _ = _case(64, [20], [7], 8, 8, 64, 4)
    assert ops.prefill_paged_plan(offs4.to(DEV), ctx4.to(DEV), q4.shape[0], 8, 8,
                                  tables4.shape[1], 4) is None
    small = torch.empty(16, dtype=torch.uint8, device=DEV)
    rc = _lib.load().fe_prefill_plan(offs_d.data_ptr(), ctx_d.data_ptr(), ctx.shape[0],
                                     q.shape[0], q.shape[1], kp.shape[2], tables.shape[1], bs,
                                     small.data_ptr(), small.numel(), None)
    assert rc == _lib.FE_ERR_WORKSPACE


def test_planned_prefill_checks_its_plan_and_leaves_tickets_clean():
    """A plan for other tensors (a clone of context_lens, same contents) and a stale plan
    (a length changed in place after the plan call) are not used: every row NaN and the
    error word set, before any split unit's ticket is taken -- so the unplanned and
    freshly planned launches that follow are exact."""
    q, offs, ctx, tables, kp, vp, bs = _planned_prefill_cases()["small"]  # lengths 130, 47, 1000
    hq, hkv, d = q.shape[1], kp.shape[2], q.shape[2]
    qd, kd, vd = q.to(DEV), kp.to(DEV), vp.to(DEV)
    offs_d, ctx_d, tables_d = offs.to(DEV), ctx.to(DEV), tables.to(DEV)
    max_q = int((offs[1:] - offs[:-1]).max())
    plan = ops.prefill_paged_plan(offs_d, ctx_d, q.shape[0], hq, hkv, tables.shape[1], bs)
    need = int(_lib.load().fe_prefill_workspace_size(ctx.shape[0], q.shape[0], hq, hkv, d))
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    out = torch.zeros_like(qd)
    rc = _lib.load().fe_prefill_paged_planned(
        qd.data_ptr(), out.data_ptr(), kd.data_ptr(), vd.data_ptr(), kp.shape[0],
        tables_d.data_ptr(), tables.shape[1], offs_d.data_ptr(), ctx_d.clone().data_ptr(),
        ctx.shape[0], q.shape[0], max_q, hq, hkv, d, bs, 1.0 / math.sqrt(d), ws.data_ptr(),
        need, plan.buffer.data_ptr(), plan.buffer.numel(),
        torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.FE_OK
    torch.cuda.synchronize()
    assert torch.isnan(out).all() and ops.plan_error(plan) == ops.PLAN_ERR_SIZES
    ctx_d[1] += 1                                              # 47 -> 48, same page count
    got = ops.prefill_paged(qd, kd, vd, tables_d, offs_d, ctx_d, max_q, plan=plan)
    torch.cuda.synchronize()
    assert torch.isnan(got).all() and ops.plan_error(plan) == ops.PLAN_ERR_STALE
    ref = ops.prefill_paged(qd, kd, vd, tables_d, offs_d, ctx_d, max_q)
    ops.prefill_paged_plan(offs_d, ctx_d, q.shape[0], hq, hkv, tables.shape[1], bs, out=plan)
    got = ops.prefill_paged(qd, kd, vd, tables_d, offs_d, ctx_d, max_q, plan=plan)
    torch.cuda.synchronize()
    assert ops.plan_error(plan) == 0 and torch.equal(got, ref)
    ctx2 = ctx.clone()
    ctx2[1] += 1
    exp = R.prefill_reference(q.numpy(), offs.numpy(), ctx2.numpy(), kp.numpy(), vp.numpy(),
                              tables.numpy(), bs)
    assert_attention_close(got.cpu().numpy(), exp, what="after a refused plan")
