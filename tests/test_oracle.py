"""Pins the CPU oracle (oracle/paged_ref.py) before any kernel is compared with it.

Checks come from the reference's own known-answer tests (restated with the
same layouts, sequences and tolerances), from an independent library routine
(torch's float64 scaled_dot_product_attention, scipy's logsumexp) and from
closed forms.  The last block plants mistakes in the oracle and shows that
these checks catch them.
"""
from __future__ import annotations

import math
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy.special import logsumexp

from oracle import paged_ref as R
from oracle import torch_routes as TR


def sdpa_f64(q, k, v, positions, scale=None):
    """Library route: torch SDPA in float64 with the reference's boolean mask."""
    q, k, v = (torch.as_tensor(np.asarray(x, dtype=np.float64)) for x in (q, k, v))
    ratio = q.shape[1] // k.shape[1]
    kk = k.repeat_interleave(ratio, dim=1).transpose(0, 1).unsqueeze(0)
    vv = v.repeat_interleave(ratio, dim=1).transpose(0, 1).unsqueeze(0)
    qq = q.transpose(0, 1).unsqueeze(0)
    mask = (torch.arange(k.shape[0])[None, :] <= torch.as_tensor(positions)[:, None])[None, None]
    out = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=scale)
    return out.squeeze(0).transpose(0, 1).numpy()


# --------------------------------------------------------------------------------------
# KV write / gather: reference known answers and brute force
# --------------------------------------------------------------------------------------

def test_write_materialize_readback_across_block_boundary():
    """test_allocator.py:11-29: CacheLayout(2, 10, 4, 2, 3); request "a" holds blocks
    [0, 1] after reserve(3) then reserve(5); arange rows read back exactly."""
    pool_k = np.zeros((10, 4, 2, 3), dtype=np.float32)
    pool_v = np.zeros_like(pool_k)
    a = np.arange(5 * 2 * 3, dtype=np.float32).reshape(5, 2, 3)
    R.write_kv(pool_k, pool_v, [0, 1], 0, a, a + 100, 4)
    np.testing.assert_array_equal(R.materialize(pool_k, [0, 1], 5, 4), a)
    np.testing.assert_array_equal(R.materialize(pool_v, [0, 1], 5, 4), a + 100)
    # pages as iter_blocks would yield them: 4 rows then 1 row
    np.testing.assert_array_equal(pool_k[0], a[:4])
    np.testing.assert_array_equal(pool_k[1, 0], a[4])


def test_write_rejects_unreserved_slot():
    """test_allocator.py:52-56: writing slot 4 of a 4-slot table raises IndexError."""
    pool = np.zeros((10, 4, 2, 3), dtype=np.float32)
    with pytest.raises(IndexError):
        R.write_kv(pool, pool.copy(), [0], 4, np.zeros((1, 2, 3)), np.zeros((1, 2, 3)), 4)


def test_write_brute_force_bytes(rng):
    """Every written slot holds its row; every other slot is byte-identical to before."""
    nb, bs, h, d = 12, 4, 2, 8
    pool_k = rng.standard_normal((nb, bs, h, d)).astype(np.float16)
    pool_v = rng.standard_normal((nb, bs, h, d)).astype(np.float16)
    before_k, before_v = pool_k.copy(), pool_v.copy()
    table = [7, 2, 9, 0]
    start, n = 3, 9
    keys = rng.standard_normal((n, h, d)).astype(np.float16)
    vals = rng.standard_normal((n, h, d)).astype(np.float16)
    R.write_kv(pool_k, pool_v, table, start, keys, vals, bs)
    touched = set()
    for i in range(n):
        p = start + i
        blk, off = table[p // bs], p % bs
        touched.add((blk, off))
        assert pool_k[blk, off].tobytes() == keys[i].tobytes()
        assert pool_v[blk, off].tobytes() == vals[i].tobytes()
    for blk in range(nb):
        for off in range(bs):
            if (blk, off) not in touched:
                assert pool_k[blk, off].tobytes() == before_k[blk, off].tobytes()
                assert pool_v[blk, off].tobytes() == before_v[blk, off].tobytes()


def test_write_kv_decode_matches_per_row_write(rng):
    """Graph-path write (qwen2.py:156-161) == per-request write at position L-1;
    inactive rows (length 0) leave the pool untouched."""
    nb, bs, h, d = 16, 4, 2, 8
    pool_k = rng.standard_normal((nb, bs, h, d)).astype(np.float16)
    pool_v = rng.standard_normal((nb, bs, h, d)).astype(np.float16)
    tables = np.array([[3, 5, 1], [0, 2, 4], [6, 7, 8]])
    ctx = np.array([9, 0, 4])
    k = rng.standard_normal((3, h, d)).astype(np.float16)
    v = rng.standard_normal((3, h, d)).astype(np.float16)
    exp_k, exp_v = pool_k.copy(), pool_v.copy()
    for b in (0, 2):
        R.write_kv(exp_k, exp_v, list(tables[b]), int(ctx[b]) - 1, k[b:b + 1], v[b:b + 1], bs)
    R.write_kv_decode(pool_k, pool_v, tables, ctx, k, v, bs)
    assert pool_k.tobytes() == exp_k.tobytes() and pool_v.tobytes() == exp_v.tobytes()


# --------------------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------------------

@pytest.mark.parametrize("length", [1, 3, 4, 5, 15, 16, 17, 34])
@pytest.mark.parametrize("qcount", [1, 2, 3])
def test_blockwise_matches_materialized_reference_grid(length, qcount):
    """test_attention.py:8-22: CacheLayout(2, 20, 4, 2, 8), 4 q-heads, fp32,
    blockwise == materialized at atol 1e-5 for query positions length-qcount..length-1."""
    if length < qcount:
        return
    rng = np.random.default_rng(length + 17 * qcount)
    bs, nb = 4, 20
    pool_k = np.zeros((nb, bs, 2, 8), dtype=np.float32)
    pool_v = np.zeros_like(pool_k)
    table = list(range(math.ceil(length / bs)))
    keys = rng.standard_normal((length, 2, 8)).astype(np.float32)
    vals = rng.standard_normal((length, 2, 8)).astype(np.float32)
    R.write_kv(pool_k, pool_v, table, 0, keys, vals, bs)
    q = rng.standard_normal((qcount, 4, 8)).astype(np.float32)
    pos = np.arange(length - qcount, length)
    paged = R.attention_blockwise(q, pool_k, pool_v, table, length, pos, bs)
    base = R.attention_materialized(q, R.materialize(pool_k, table, length, bs),
                                    R.materialize(pool_v, table, length, bs), pos)
    np.testing.assert_allclose(paged, base, atol=1e-5, rtol=1e-5)


def test_noncontiguous_physical_pages():
    """test_attention.py:25-36: table [0, 3, 4] (block size 2), positions [3, 4]."""
    rng = np.random.default_rng(0)
    pool_k = np.zeros((8, 2, 1, 4), dtype=np.float32)
    pool_v = np.zeros_like(pool_k)
    table = [0, 3, 4]
    R.write_kv(pool_k, pool_v, table, 0, rng.standard_normal((5, 1, 4)),
               rng.standard_normal((5, 1, 4)), 2)
    q = rng.standard_normal((2, 2, 4))
    p = np.array([3, 4])
    got = R.attention_blockwise(q, pool_k, pool_v, table, 5, p, 2)
    exp = R.attention_materialized(q, R.materialize(pool_k, table, 5, 2),
                                   R.materialize(pool_v, table, 5, 2), p)
    np.testing.assert_allclose(got, exp, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("hq,hkv,d,lk,nq", [(4, 2, 8, 9, 3), (14, 2, 64, 37, 1),
                                            (12, 2, 128, 70, 5), (8, 8, 16, 5, 5)])
def test_materialized_matches_torch_sdpa_float64(hq, hkv, d, lk, nq):
    rng = np.random.default_rng(hq * 100 + lk)
    q = rng.standard_normal((nq, hq, d))
    k = rng.standard_normal((lk, hkv, d))
    v = rng.standard_normal((lk, hkv, d))
    pos = np.arange(lk - nq, lk)
    np.testing.assert_allclose(R.attention_materialized(q, k, v, pos), sdpa_f64(q, k, v, pos),
                               atol=1e-12, rtol=1e-12)


def test_closed_forms(rng):
    # one key: the output is that key's value row, for every head of the group
    q = rng.standard_normal((1, 6, 16))
    k = rng.standard_normal((1, 2, 16))
    v = rng.standard_normal((1, 2, 16))
    out = R.attention_materialized(q, k, v, [0])
    np.testing.assert_allclose(out[0, :3], np.repeat(v[0, :1], 3, 0), atol=0, rtol=0)
    np.testing.assert_allclose(out[0, 3:], np.repeat(v[0, 1:], 3, 0), atol=0, rtol=0)
    # identical keys: uniform weights, output = mean of the visible values
    k = np.repeat(rng.standard_normal((1, 2, 16)), 10, 0)
    v = rng.standard_normal((10, 2, 16))
    out = R.attention_materialized(rng.standard_normal((1, 4, 16)), k, v, [6])
    np.testing.assert_allclose(out[0, 0], v[:7, 0].mean(0), atol=1e-12)
    np.testing.assert_allclose(out[0, 3], v[:7, 1].mean(0), atol=1e-12)


def test_physical_block_permutation_invariance(rng):
    nb, bs, h, d, length = 10, 4, 2, 8, 27
    pool_k = rng.standard_normal((nb, bs, h, d))
    pool_v = rng.standard_normal((nb, bs, h, d))
    table = [4, 1, 7, 0, 9, 2, 5]
    q = rng.standard_normal((2, 4, d))
    base = R.decode_reference(q, pool_k, pool_v, np.array([table, table]), [length, 13], bs)
    perm = rng.permutation(nb)
    inv = np.argsort(perm)
    pk2, pv2 = pool_k[perm], pool_v[perm]          # block j of new pool = block perm[j]
    table2 = [int(inv[b]) for b in table]
    got = R.decode_reference(q, pk2, pv2, np.array([table2, table2]), [length, 13], bs)
    np.testing.assert_allclose(got, base, atol=1e-13)


def test_decode_inactive_rows_are_exact_zeros(rng):
    """paged_attention.py:131,138: inactive rows give exact zeros."""
    pool = rng.standard_normal((6, 4, 1, 8))
    q = rng.standard_normal((3, 2, 8))
    out = R.paged_decode_batch(q, pool, pool, np.array([[0, 1], [2, 3], [4, 5]]),
                               np.array([5, 3, 7]), np.array([1, 0, 1]), 4)
    assert (out[1] == 0).all() and np.abs(out[0]).sum() > 0 and np.abs(out[2]).sum() > 0


def test_prefill_equals_per_row_decode(rng):
    nb, bs, hkv, hq, d = 20, 4, 2, 6, 16
    pool_k = rng.standard_normal((nb, bs, hkv, d))
    pool_v = rng.standard_normal((nb, bs, hkv, d))
    tables = np.array([[3, 1, 4, 0, 5, 9], [2, 6, 8, 7, 10, 11]])
    offs = np.array([0, 5, 12])
    ctx = np.array([9, 21])
    q = rng.standard_normal((12, hq, d))
    got = R.prefill_reference(q, offs, ctx, pool_k, pool_v, tables, bs)
    for s in range(2):
        n = offs[s + 1] - offs[s]
        for j in range(n):
            row = offs[s] + j
            pos = ctx[s] - n + j
            exp = R.decode_reference(q[row:row + 1], pool_k, pool_v, tables[s:s + 1], [pos + 1], bs)
            np.testing.assert_allclose(got[row], exp[0], atol=1e-12)


def test_lse_merge_identity_and_scipy(rng):
    q = rng.standard_normal((5, 16))
    k = rng.standard_normal((40, 16))
    v = rng.standard_normal((40, 16))
    bounds = [0, 7, 7, 23, 40]   # includes an empty split
    po, pl = R.split_attention(q, k, v, bounds)
    out, lse = R.lse_merge(po, pl)
    full_o, full_l = R.split_attention(q, k, v, [0, 40])
    np.testing.assert_allclose(out, full_o[0], atol=1e-12)
    np.testing.assert_allclose(lse, full_l[0], atol=1e-12)
    np.testing.assert_allclose(lse, logsumexp(pl, axis=0), atol=1e-12)
    # all-empty row -> zeros, -inf
    out2, lse2 = R.lse_merge(np.zeros((2, 1, 3)), np.full((2, 1), -np.inf))
    assert (out2 == 0).all() and np.isneginf(lse2).all()


def test_bucket_for_matches_reference_test():
    """test_cuda_graph.py:7-12."""
    assert [R.bucket_for(n) for n in (1, 2, 3, 4, 5, 8)] == [1, 2, 4, 4, 8, 8]
    assert R.bucket_for(9) is None and R.bucket_for(0) is None


def test_torch_routes_match_oracle(rng):
    """The CPU-baseline restatements (torch, fp16 pools) agree with the float64 oracle."""
    nb, bs, hkv, hq, d = 12, 16, 2, 12, 128
    pool_k = torch.randn(nb, bs, hkv, d, generator=torch.Generator().manual_seed(5)).half()
    pool_v = torch.randn(nb, bs, hkv, d, generator=torch.Generator().manual_seed(6)).half()
    q = torch.randn(1, hq, d, generator=torch.Generator().manual_seed(7)).half()
    table = [5, 2, 9, 0, 11]
    length = 70
    pos = torch.tensor([length - 1])
    exp = R.decode_reference(q.numpy(), pool_k.numpy(), pool_v.numpy(), np.array([table]),
                             [length], bs)
    mat = TR.materialized_route(q, pool_k, pool_v, table, length, pos).float().numpy()
    blk = TR.blockwise_route(q, pool_k, pool_v, table, length, pos).float().numpy()
    np.testing.assert_allclose(mat, exp, atol=2e-3)
    np.testing.assert_allclose(blk, exp, atol=2e-3)


# --------------------------------------------------------------------------------------
# planted mistakes: each must be caught by one of the checks above
# --------------------------------------------------------------------------------------

class _NumpyProxy(types.SimpleNamespace):
    def __getattr__(self, name):
        return getattr(np, name)


def test_planted_wrong_gqa_head_map_is_caught(monkeypatch, rng):
    """q-head h must read kv-head h // G; tiling (h % Hkv) instead must fail the SDPA check."""
    proxy = _NumpyProxy(repeat=lambda a, r, axis: np.tile(a, (1, r, 1)))
    monkeypatch.setattr(R, "np", proxy)
    q = rng.standard_normal((1, 4, 8))
    k = rng.standard_normal((6, 2, 8))
    v = rng.standard_normal((6, 2, 8))
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(R.attention_materialized(q, k, v, [5]), sdpa_f64(q, k, v, [5]),
                                   atol=1e-9)


def test_planted_wrong_scale_is_caught(monkeypatch, rng):
    proxy = types.SimpleNamespace(sqrt=lambda x: math.sqrt(x) * 2.0)
    monkeypatch.setattr(R, "math", proxy)
    q = rng.standard_normal((1, 2, 8))
    k = rng.standard_normal((6, 1, 8))
    v = rng.standard_normal((6, 1, 8))
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(R.attention_materialized(q, k, v, [5]), sdpa_f64(q, k, v, [5]),
                                   atol=1e-9)


def test_planted_off_by_one_causal_mask_is_caught(monkeypatch, rng):
    """Shifting key positions by one (t < pos instead of t <= pos) breaks the L=1 closed form."""
    proxy = _NumpyProxy(arange=lambda *a, **kw: np.arange(*a, **kw) + 1)
    monkeypatch.setattr(R, "np", proxy)
    q = rng.standard_normal((1, 2, 8))
    k = rng.standard_normal((3, 1, 8))
    v = rng.standard_normal((3, 1, 8))
    with pytest.raises(AssertionError):
        out = R.attention_materialized(q, k, v, [0])
        np.testing.assert_allclose(out[0, 0], v[0, 0], atol=1e-9)


def test_planted_wrong_slot_map_is_caught(monkeypatch):
    """A locator that swaps block and offset roles fails the readback known answer."""
    def bad_locators(table, start, count, bs):
        slots = np.arange(start, start + count)
        return np.asarray(table)[slots % len(table)], slots // len(table)
    monkeypatch.setattr(R, "locators", bad_locators)
    pool_k = np.zeros((10, 4, 2, 3), dtype=np.float32)
    a = np.arange(30, dtype=np.float32).reshape(5, 2, 3)
    R.write_kv(pool_k, pool_k.copy(), [0, 1], 0, a, a, 4)
    with pytest.raises(AssertionError):
        np.testing.assert_array_equal(pool_k[0], a[:4])


def test_f32_tolerance_rejects_16_bit_rounding():
    """The fp32 GPU tests' tolerance (max |err| <= 2e-5, mean <= 2e-6) pinned from both
    sides on the oracle: a plain float32 evaluation of the same decode stays inside it,
    while rounding q, K and V to fp16 or bf16 -- what a kernel computing in 16 bits
    would do -- lands far outside it."""
    rng = np.random.default_rng(77)
    b, hq, hkv, d, bs = 3, 8, 2, 64, 16
    lens = np.array([1000, 37, 4096])
    width = 4096 // bs
    tables = np.stack([rng.permutation(3 * width)[:width] for _ in range(b)]).astype(np.int32)
    kp = rng.standard_normal((3 * width, bs, hkv, d)).astype(np.float32)
    vp = rng.standard_normal((3 * width, bs, hkv, d)).astype(np.float32)
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    exact = R.decode_reference(q, kp, vp, tables, lens, bs)
    # float32 arithmetic throughout (numpy float32 matmuls and softmax)
    g = hq // hkv
    f32 = np.zeros_like(q)
    for i in range(b):
        k = R.materialize(kp, tables[i], int(lens[i]), bs)
        v = R.materialize(vp, tables[i], int(lens[i]), bs)
        for h in range(hq):
            s = (k[:, h // g] @ q[i, h]) * np.float32(1 / math.sqrt(d))
            p = np.exp(s - s.max())
            f32[i, h] = (p @ v[:, h // g]) / p.sum()
    err = np.abs(f32 - exact)
    assert err.max() <= 2e-5 and err.mean() <= 2e-6, (err.max(), err.mean())
    for rnd in (lambda x: x.astype(np.float16).astype(np.float32),
                lambda x: torch.from_numpy(x).to(torch.bfloat16).float().numpy()):
        r = R.decode_reference(rnd(q), rnd(kp), rnd(vp), tables, lens, bs)
        err = np.abs(r - exact)
        assert err.max() > 10 * 2e-5 and err.mean() > 10 * 2e-6, (err.max(), err.mean())
