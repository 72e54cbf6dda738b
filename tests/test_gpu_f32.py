"""GPU: float32 forms -- the KV page movers, the decode, the prefill and the
shared-prefix decode -- against the oracle.

The reference's PagedKVCache defaults to float32 (allocator.py:26), the engine
builds the cache in the model's dtype, float32 among them (runtime.py:37-40,
qwen2.py:54), and its Triton decode computes in float32 (paged_attention.py:
116,126,134).  The fp32 entry points take float32 q / pools / new rows and
return float32; the oracle runs in float64 on the same values.  Inputs are fresh
float32 draws, not widened fp16 values, so a kernel that rounded q, K or V to
16 bits anywhere would fail (test_oracle.py's
test_f32_tolerance_rejects_16_bit_rounding shows the margin).

Tolerance: the fp32 unit roundoff 2^-24 times the longest chain of sequential
fp32 accumulations in the kernels -- 4096 keys in 16-key tiles, 256 steps --
is 1.5e-5: max |err| <= 2e-5, mean |err| <= 2e-6.  Page writes and gathers
are byte copies and stay bit-exact.
"""
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
F32 = torch.float32
F32_MAX_TOL = 2e-5
F32_MEAN_TOL = 2e-6


def close_f32(got: torch.Tensor, exp: np.ndarray, what: str = ""):
    assert got.dtype == F32, got.dtype
    mx, mean = assert_attention_close(got.cpu().numpy(), exp, F32_MAX_TOL, F32_MEAN_TOL, what)
    print(f"{what}: max abs {mx:.3e} mean abs {mean:.3e}", flush=True)


def to_f32(w: workloads.DecodeWorkload, seed: int) -> workloads.DecodeWorkload:
    """The workload's tables and lengths with fresh float32 q, pools and new rows."""
    g = torch.Generator().manual_seed(seed)

    def draw(t):
        return None if t is None else torch.randn(t.shape, generator=g, dtype=F32)
    return workloads.DecodeWorkload(w.name + "-f32", draw(w.q), draw(w.k_pool), draw(w.v_pool),
                                    w.block_tables, w.context_lens, draw(w.k_new), draw(w.v_new),
                                    w.unique_tokens, dict(w.meta))


def oracle_decode(w: workloads.DecodeWorkload):
    kp, vp = w.k_pool.numpy().copy(), w.v_pool.numpy().copy()
    if w.k_new is not None:
        R.write_kv_decode(kp, vp, w.block_tables.numpy(), w.context_lens.numpy(),
                          w.k_new.numpy(), w.v_new.numpy(), w.block_size)
    out = R.decode_reference(w.q.numpy(), kp, vp, w.block_tables.numpy(),
                             w.context_lens.numpy(), w.block_size)
    return out, kp, vp


def _decode_cases():
    lens = [0, 1, 15, 16, 17, 200, 0, 1023, 4096, 64]
    return [
        to_f32(workloads.c1_workload(), 301),
        to_f32(workloads.c2_workload(), 302),
        to_f32(workloads.make_decode_workload("edges", 303, len(lens), 12, 2, 128, lens,
                                              width=256, with_new_kv=True), 304),
        to_f32(workloads.make_decode_workload("d64-g7", 305, 6, 14, 2, 64,
                                              [1, 33, 700, 2049, 5, 9000], with_new_kv=True), 306),
        to_f32(workloads.make_decode_workload("bs32", 307, 5, 16, 2, 128,
                                              [3000, 17, 512, 0, 9000], block_size=32,
                                              with_new_kv=True), 308),
        to_f32(workloads.make_decode_workload("bs8-g16", 309, 4, 16, 1, 64, [9, 100, 1, 777],
                                              block_size=8, with_new_kv=True), 310),
    ]


@pytest.mark.parametrize("case", range(6))
def test_f32_decode_matches_oracle_with_page_write(case):
    w = _decode_cases()[case]
    print(f"fp32 decode case {w.name}", flush=True)
    d = w.to(DEV)
    out = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                           k_new=d.k_new, v_new=d.v_new)
    torch.cuda.synchronize()
    exp, kp, vp = oracle_decode(w)
    close_f32(out, exp, w.name)
    inactive = (w.context_lens == 0).nonzero().flatten().tolist()
    for b in inactive:
        assert torch.count_nonzero(out[b]) == 0, f"inactive row {b}"
    assert d.k_pool.cpu().numpy().tobytes() == kp.tobytes(), "page write (K)"
    assert d.v_pool.cpu().numpy().tobytes() == vp.tobytes(), "page write (V)"


def test_f32_decode_split_targets_and_repeated_calls():
    """Forced split targets (1 = no split, 512 = many pieces per row) agree with the
    oracle, and repeated calls are bit-identical."""
    w = _decode_cases()[1]
    d = w.to(DEV)
    exp, _, _ = oracle_decode(workloads.DecodeWorkload(w.name, w.q, w.k_pool, w.v_pool,
                                                       w.block_tables, w.context_lens, None,
                                                       None, w.unique_tokens, w.meta))
    first = None
    for target in (0, 1, 512, 0):
        out = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                               target_splits=target)
        torch.cuda.synchronize()
        close_f32(out, exp, f"target {target}")
        if target == 0:
            if first is None:
                first = out.clone()
            assert torch.equal(out, first), "repeated calls differ"


def _prefill_case(seed, n_new, cached, hq=12, hkv=2, d=128, bs=16):
    g = torch.Generator().manual_seed(seed)
    ctx = [c + n for c, n in zip(cached, n_new)]
    pages = [math.ceil(x / bs) for x in ctx]
    nb = sum(pages) + 3
    k_pool = torch.randn(nb, bs, hkv, d, generator=g, dtype=F32)
    v_pool = torch.randn(nb, bs, hkv, d, generator=g, dtype=F32)
    perm = torch.randperm(nb, generator=g)
    width = max(pages)
    tables = torch.zeros(len(ctx), width, dtype=torch.int32)
    at = 0
    for i, p in enumerate(pages):
        tables[i, :p] = perm[at:at + p]
        tables[i, p:] = perm[at + p - 1] if p else 0
        at += p
    offs = np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32)
    q = torch.randn(int(offs[-1]), hq, d, generator=g, dtype=F32)
    return q, torch.tensor(offs), torch.tensor(ctx, dtype=torch.int32), tables, k_pool, v_pool


@pytest.mark.parametrize("n_new,cached,shape", [
    ([1], [0], (12, 2, 128, 16)),
    ([17], [3], (12, 2, 128, 16)),
    ([130, 7, 1], [0, 40, 999], (12, 2, 128, 16)),
    ([0, 33], [10, 10], (12, 2, 128, 16)),
    ([70, 3], [25, 200], (14, 2, 64, 16)),
    ([20, 5], [7, 60], (8, 8, 64, 4)),
    ([300, 1, 45], [0, 2048, 17], (16, 2, 128, 32)),
])
def test_f32_prefill_matches_oracle(n_new, cached, shape):
    hq, hkv, d, bs = shape
    q, offs, ctx, tables, kp, vp = _prefill_case(sum(n_new) + 3 * hq + bs, n_new, cached, hq, hkv,
                                                 d, bs)
    out = ops.prefill_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), tables.to(DEV), offs.to(DEV),
                            ctx.to(DEV), max(n_new))
    torch.cuda.synchronize()
    exp = R.prefill_reference(q.numpy(), offs.numpy(), ctx.numpy(), kp.numpy(), vp.numpy(),
                              tables.numpy(), bs)
    close_f32(out, exp, f"n={n_new} c={cached} {shape}")


def test_f32_c4_prefill_chunks():
    """C4's four prefill chunks (266-434 new tokens over 1208-3012 cached) in fp32."""
    w = workloads.c4_workload()
    g = torch.Generator().manual_seed(311)
    q = torch.randn(w.q.shape, generator=g, dtype=F32)
    kp = torch.randn(w.k_pool.shape, generator=g, dtype=F32)
    vp = torch.randn(w.v_pool.shape, generator=g, dtype=F32)
    mq = int((w.q_offsets[1:] - w.q_offsets[:-1]).max())
    out = ops.prefill_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), w.block_tables.to(DEV),
                            w.q_offsets.to(DEV), w.context_lens.to(DEV), mq)
    torch.cuda.synchronize()
    exp = R.prefill_reference(q.numpy(), w.q_offsets.numpy(), w.context_lens.numpy(), kp.numpy(),
                              vp.numpy(), w.block_tables.numpy(), 16)
    close_f32(out, exp, "C4 prefill fp32")


def test_f32_kv_movers_are_byte_exact():
    """fe_write_kv_f32 (explicit slots), fe_write_kv_decode_f32, fe_write_kv_ragged_f32 and
    fe_gather_kv_f32 against the oracle's copies, with NaN payloads carried as bytes."""
    g = torch.Generator().manual_seed(312)
    nb, bs, h, d = 40, 16, 2, 128
    k_pool = torch.randn(nb, bs, h, d, generator=g, dtype=F32)
    v_pool = torch.randn(nb, bs, h, d, generator=g, dtype=F32)
    # explicit slots
    n = 45
    keys = torch.randn(n, h, d, generator=g, dtype=F32)
    vals = torch.randn(n, h, d, generator=g, dtype=F32)
    keys.view(torch.int32)[3, 1, 5] = 0x7FC0_1234  # a NaN with a payload
    table, start = [31, 4, 17], 2
    ids, offs = R.locators(table, start, n, bs)
    exp_k, exp_v = k_pool.numpy().copy(), v_pool.numpy().copy()
    R.write_kv(exp_k, exp_v, table, start, keys.numpy(), vals.numpy(), bs)
    kd, vd = k_pool.to(DEV), v_pool.to(DEV)
    ops.write_kv(keys.to(DEV), vals.to(DEV), kd, vd,
                 torch.tensor(ids, dtype=torch.int32, device=DEV),
                 torch.tensor(offs, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert kd.cpu().numpy().tobytes() == exp_k.tobytes()
    assert vd.cpu().numpy().tobytes() == exp_v.tobytes()
    # decode-step write at context_lens - 1 (0 = skipped), strided source rows
    tables = torch.tensor([[5, 6, 7], [8, 9, 10], [11, 12, 13]], dtype=torch.int32)
    lens = torch.tensor([17, 0, 48], dtype=torch.int32)
    fused = torch.randn(3, 3 * h, d, generator=g, dtype=F32)  # rows with stride 3*h*d
    kn, vn = fused[:, :h], fused[:, h:2 * h]
    R.write_kv_decode(exp_k, exp_v, tables.numpy(), lens.numpy(), kn.numpy(), vn.numpy(), bs)
    fd = fused.to(DEV)
    ops.write_kv_decode(fd[:, :h], fd[:, h:2 * h], kd, vd, tables.to(DEV), lens.to(DEV))
    torch.cuda.synchronize()
    assert kd.cpu().numpy().tobytes() == exp_k.tobytes()
    assert vd.cpu().numpy().tobytes() == exp_v.tobytes()
    # ragged chunks: rows q_offsets[s]..q_offsets[s+1]-1 are the last of context_lens[s]
    qo = torch.tensor([0, 5, 5, 12], dtype=torch.int32)
    ctx = torch.tensor([20, 3, 40], dtype=torch.int32)
    rt = torch.tensor([[20, 21, 22], [23, 24, 25], [26, 27, 28]], dtype=torch.int32)
    rk = torch.randn(12, h, d, generator=g, dtype=F32)
    rv = torch.randn(12, h, d, generator=g, dtype=F32)
    for s in range(3):
        a, e = int(qo[s]), int(qo[s + 1])
        R.write_kv(exp_k, exp_v, rt[s].tolist(), int(ctx[s]) - (e - a), rk[a:e].numpy(),
                   rv[a:e].numpy(), bs)
    ops.write_kv_ragged(rk.to(DEV), rv.to(DEV), kd, vd, rt.to(DEV), qo.to(DEV), ctx.to(DEV))
    torch.cuda.synchronize()
    assert kd.cpu().numpy().tobytes() == exp_k.tobytes()
    assert vd.cpu().numpy().tobytes() == exp_v.tobytes()
    # gather (materialize) of every row's context
    glens = torch.tensor([20, 0, 40], dtype=torch.int32)
    goffs = torch.tensor([0, 20, 20, 60], dtype=torch.int32)
    gk, gv = ops.gather_kv(kd, vd, rt.to(DEV), glens.to(DEV), goffs.to(DEV), 60)
    torch.cuda.synchronize()
    ek = np.concatenate([R.materialize(exp_k, rt[s].tolist(), int(glens[s]), bs)
                         for s in range(3) if glens[s] > 0])
    ev = np.concatenate([R.materialize(exp_v, rt[s].tolist(), int(glens[s]), bs)
                         for s in range(3) if glens[s] > 0])
    assert gk.dtype == F32 and gk.cpu().numpy().tobytes() == ek.tobytes()
    assert gv.cpu().numpy().tobytes() == ev.tobytes()


@pytest.mark.parametrize("length", [1, 17, 129, 513])
def test_f32_cache_reference_case_noncontiguous_pages(length):
    """test_triton_paged_attention.py:10-26 on the reference's default float32 cache:
    CacheLayout(1, 80, 16, 2, 64), 8 q heads, reversed page table, through the
    per-request route (a decode for one query, the prefill for the whole prompt)."""
    g = torch.Generator().manual_seed(313 + length)
    cache = PagedKVCache(CacheLayout(1, 80, 16, 2, 64), device=DEV, dtype=F32)
    cache.reserve("r", length)
    cache.tables["r"] = list(reversed(cache.tables["r"]))
    keys = torch.randn(length, 2, 64, generator=g, dtype=F32)
    values = torch.randn(length, 2, 64, generator=g, dtype=F32)
    cache.write(0, "r", 0, keys.to(DEV), values.to(DEV))
    k, v = cache.materialize(0, "r", length)
    assert k.dtype == F32 and torch.equal(k.cpu(), keys) and torch.equal(v.cpu(), values)
    query = torch.randn(1, 8, 64, generator=g, dtype=F32)
    got = attention.attention_for_request(query.to(DEV), cache, 0, "r", length,
                                          torch.tensor([length - 1], device=DEV))
    exp = R.attention_materialized(query.numpy(), keys.numpy(), values.numpy(), [length - 1])
    close_f32(got, exp, f"decode length {length}")
    prompt = torch.randn(length, 8, 64, generator=g, dtype=F32)
    got = attention.attention_for_request(prompt.to(DEV), cache, 0, "r", length,
                                          torch.arange(length, device=DEV))
    exp = R.attention_materialized(prompt.numpy(), keys.numpy(), values.numpy(),
                                   list(range(length)))
    close_f32(got, exp, f"prefill length {length}")


def test_f32_decode_plan_refuses():
    """fp32 pools have no decode plan (the C ABI has no planned fp32 entry point);
    ops refuses one before launching anything."""
    w = _decode_cases()[0]
    d = w.to(DEV)
    nb, bs, hkv = d.k_pool.shape[0], d.k_pool.shape[1], d.k_pool.shape[2]
    plan = ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs)
    with pytest.raises(ValueError, match="fp32"):
        ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens, plan=plan)


# --------------------------------------------------------------------------------------
# shared-prefix decode (fe_paged_decode_shared_prefix_f32): the prefix pass on the fp32
# prefill engine, the suffixes on the fp32 piece kernel, merged in fp32
# --------------------------------------------------------------------------------------

def _shared_prefix(w: workloads.DecodeWorkload, fuse: bool = False):
    d = w.to(DEV)
    out = ops.paged_decode_shared_prefix(
        d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
        d.meta["group_offsets"].to(DEV), d.meta["prefix_lens"].to(DEV),
        k_new=d.k_new if fuse else None, v_new=d.v_new if fuse else None)
    torch.cuda.synchronize()
    return out, d


@pytest.mark.parametrize("hq,hkv,d,bs", [(12, 2, 128, 16), (14, 2, 64, 32), (8, 1, 128, 16)])
def test_f32_shared_prefix_edge_groups(hq, hkv, d, bs):
    """Groups of 3 (prefix 40 tokens: whole blocks only), 1 and 0 members, a group of
    5 with one member ending at the prefix, one inside it and one inactive, and rows
    outside every group."""
    groups = [(3, 40), (1, 64), (0, 32), (5, 512)]
    w = to_f32(workloads.shared_prefix_workload(41 + d, groups, singles=3, hq=hq, hkv=hkv, d=d,
                                                block_size=bs,
                                                member_lens={5: 512, 6: 505, 7: 0}), 42 + d)
    got, _ = _shared_prefix(w)
    exp, _, _ = oracle_decode(w)
    close_f32(got, exp, f"fp32 cascade edges {hq}/{hkv}/{d} bs{bs}")
    assert not got[7].any(), "inactive member must give exact zeros"


def test_f32_shared_prefix_with_page_write_and_long_prefix():
    """C3-like groups with the fused page write (pools bit-exact after the call), then
    a 20000-token prefix; the cascade agrees with the plain fp32 decode."""
    w = to_f32(workloads.shared_prefix_workload(12, [(6, 256), (4, 1024)], singles=2,
                                                with_new_kv=True), 43)
    got, d = _shared_prefix(w, fuse=True)
    exp, kp, vp = oracle_decode(w)
    close_f32(got, exp, "fp32 cascade with page write")
    assert np.array_equal(d.k_pool.cpu().numpy(), kp) and np.array_equal(d.v_pool.cpu().numpy(), vp)
    w = to_f32(workloads.shared_prefix_workload(44, [(3, 20000)], singles=1, tail=(1, 200)), 45)
    got, d = _shared_prefix(w)
    exp, _, _ = oracle_decode(w)
    close_f32(got, exp, "fp32 cascade, 20000-token prefix")
    plain = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens)
    close_f32(got, plain.cpu().numpy().astype(np.float64), "fp32 cascade vs plain")