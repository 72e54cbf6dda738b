"""GPU: fused paged decode (fe_paged_decode + split-K LSE merge) against the oracle.

Tolerance (hot-path contract): max |err| <= 2e-3 and mean |err| <= 2e-4 of the
fp16 output against the float64 oracle.  Page writes fused into the decode call
must be bit-exact.
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


def run_decode(w: workloads.DecodeWorkload, target_splits: int = 0, fuse: bool = True):
    d = w.to(DEV)
    kn = d.k_new if fuse else None
    vn = d.v_new if fuse else None
    out = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                           k_new=kn, v_new=vn, target_splits=target_splits)
    torch.cuda.synchronize()
    return out.cpu(), d


def oracle_decode(w: workloads.DecodeWorkload):
    kp, vp = w.k_pool.numpy().copy(), w.v_pool.numpy().copy()
    if w.k_new is not None:
        R.write_kv_decode(kp, vp, w.block_tables.numpy(), w.context_lens.numpy(),
                          w.k_new.numpy(), w.v_new.numpy(), w.block_size)
    out = R.decode_reference(w.q.numpy(), kp, vp, w.block_tables.numpy(),
                             w.context_lens.numpy(), w.block_size)
    return out, kp, vp


# --------------------------------------------------------------------------------------
# the reference's own GPU test cases, through the per-request interface
# --------------------------------------------------------------------------------------

@pytest.mark.parametrize("length", [1, 17, 129, 513])
def test_reference_case_noncontiguous_pages(length):
    """test_triton_paged_attention.py:10-26: CacheLayout(1, 80, 16, 2, 64), 8 q-heads,
    reversed page table, fp16; here held to the tighter contract tolerance."""
    g = torch.Generator().manual_seed(7 + length)
    cache = PagedKVCache(CacheLayout(1, 80, 16, 2, 64), device=DEV)
    cache.reserve("r", length)
    cache.tables["r"] = list(reversed(cache.tables["r"]))
    keys = torch.randn(length, 2, 64, generator=g).half()
    values = torch.randn(length, 2, 64, generator=g).half()
    cache.write(0, "r", 0, keys.to(DEV), values.to(DEV))
    query = torch.randn(1, 8, 64, generator=g).half()
    position = torch.tensor([length - 1], device=DEV)
    got = attention.attention_for_request(query.to(DEV), cache, 0, "r", length, position)
    exp = R.attention_materialized(query.numpy(), keys.numpy(), values.numpy(), [length - 1])
    assert got.dtype == torch.float16 and got.shape == (1, 8, 64)
    assert_attention_close(got.cpu().numpy(), exp, what=f"length {length}")


def test_reference_case_group_size_seven():
    """test_flashinfer_attention.py:36-49: Qwen2.5-0.5B heads (14 q / 2 kv / D 64), length 17."""
    g = torch.Generator().manual_seed(36)
    length = 17
    cache = PagedKVCache(CacheLayout(1, 8, 16, 2, 64), device=DEV)
    cache.reserve("r", length)
    keys = torch.randn(length, 2, 64, generator=g).half()
    cache.write(0, "r", 0, keys.to(DEV), keys.to(DEV))
    query = torch.randn(1, 14, 64, generator=g).half()
    pos = torch.tensor([length - 1], device=DEV)
    got = attention.attention_for_request(query.to(DEV), cache, 0, "r", length, pos)
    exp = R.attention_materialized(query.numpy(), keys.numpy(), keys.numpy(), [length - 1])
    assert_attention_close(got.cpu().numpy(), exp)


# --------------------------------------------------------------------------------------
# benchmark configurations at full size
# --------------------------------------------------------------------------------------

def test_c1_full():
    w = workloads.c1_workload()
    got, _ = run_decode(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="C1")


def test_c2_full_with_fused_page_write():
    w = workloads.c2_workload()
    got, d = run_decode(w)
    exp, kp, vp = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="C2")
    # fused page write: pools byte-identical to the oracle's write
    assert d.k_pool.cpu().numpy().tobytes() == kp.tobytes()
    assert d.v_pool.cpu().numpy().tobytes() == vp.tobytes()


def test_c2_split_count_invariance():
    """One piece per sequence vs. the finest split give the same result (to tolerance)."""
    w = workloads.c2_workload()
    exp, _, _ = oracle_decode(w)
    outs = []
    for target in (1, 64, 4096):
        got, _ = run_decode(w, target_splits=target)
        assert_attention_close(got.numpy(), exp, what=f"target_splits={target}")
        outs.append(got.float().numpy())
    assert np.abs(outs[0] - outs[2]).max() <= 2e-3


def test_c3_shared_prefix_split_k():
    w = workloads.c3_workload(groups=2, per_group=8)
    got, _ = run_decode(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="C3 (2x8)")


# --------------------------------------------------------------------------------------
# shapes and edge cases
# --------------------------------------------------------------------------------------

@pytest.mark.parametrize("hq,hkv,d", [(12, 2, 128), (14, 2, 64), (16, 1, 128), (8, 8, 64),
                                      (16, 2, 128), (5, 5, 128), (28, 4, 128)])
def test_head_configurations(hq, hkv, d):
    lengths = [1, 2, 15, 16, 17, 63, 64, 65, 200, 1000]
    w = workloads.make_decode_workload("shape", hq * 31 + d, len(lengths), hq, hkv, d, lengths)
    got, _ = run_decode(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what=f"{hq}/{hkv}/{d}")


@pytest.mark.parametrize("bs", [1, 2, 4, 8, 32, 64])
def test_block_sizes(bs):
    lengths = [1, 3, 33, 100, 257, 700]
    w = workloads.make_decode_workload("bs", 500 + bs, len(lengths), 12, 2, 128, lengths,
                                       block_size=bs, with_new_kv=True)
    got, d = run_decode(w)
    exp, kp, vp = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what=f"block_size {bs}")
    assert d.k_pool.cpu().numpy().tobytes() == kp.tobytes()


def test_inactive_rows_give_exact_zeros():
    lengths = [40, 0, 300, 0, 1]
    w = workloads.make_decode_workload("inactive", 77, 5, 12, 2, 128, [max(n, 1) for n in lengths])
    w.context_lens = torch.tensor(lengths, dtype=torch.int32)
    d = w.to(DEV)
    out = torch.full_like(d.q, 7.0)
    ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens, out=out)
    got = out.cpu()
    assert torch.count_nonzero(got[1]) == 0 and torch.count_nonzero(got[3]) == 0
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp)


def test_batched_backend_signature_positions_and_active_mask():
    """The reference's batched contract: (q, cache, layer, tables(int64), positions, active)."""
    g = torch.Generator().manual_seed(99)
    cache = PagedKVCache(CacheLayout(2, 64, 16, 2, 128), device=DEV)
    rows = ["a", "b", "c"]
    lens = [50, 130, 7]
    for r, n in zip(rows, lens):
        cache.reserve(r, n)
        kv = torch.randn(n, 2, 128, generator=g).half().to(DEV)
        cache.write(1, r, 0, kv, kv * 0.5)
    tables = cache.block_table(rows).to(torch.long)
    positions = torch.tensor([n - 1 for n in lens], device=DEV)
    active = torch.tensor([1.0, 0.0, 1.0], device=DEV)
    q = torch.randn(3, 12, 128, generator=g).half().to(DEV)
    got = attention.paged_decode_batch(q, cache, 1, tables, positions, active).cpu().numpy()
    exp = R.paged_decode_batch(q.cpu().numpy(), cache.k[1].cpu().numpy(), cache.v[1].cpu().numpy(),
                               tables.cpu().numpy(), positions.cpu().numpy(),
                               active.cpu().numpy(), 16)
    assert_attention_close(got, exp)
    assert (got[1] == 0).all()


def test_stale_nan_beyond_context_is_ignored():
    """Pool slots past the context (same block) hold NaN; outputs must stay finite."""
    lengths = [5, 21, 40]
    w = workloads.make_decode_workload("nan", 5, 3, 12, 2, 128, lengths)
    kp, vp = w.k_pool.clone(), w.v_pool.clone()
    for b, n in enumerate(lengths):
        for t in range(n, ((n + 15) // 16) * 16):
            blk = int(w.block_tables[b, t // 16])
            kp[blk, t % 16] = float("nan")
            vp[blk, t % 16] = float("nan")
    w.k_pool, w.v_pool = kp, vp
    got, _ = run_decode(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp)


def test_long_single_sequence_many_splits():
    w = workloads.make_decode_workload("long", 8, 1, 12, 2, 128, [20000])
    got, _ = run_decode(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="L=20000")


def test_strided_query_rows():
    """q as a view into a fused QKV projection output (row stride > Hq*D)."""
    lengths = [33, 90]
    w = workloads.make_decode_workload("stride", 12, 2, 12, 2, 128, lengths)
    d = w.to(DEV)
    big = torch.zeros(2, 16 * 128, dtype=torch.float16, device=DEV)
    big[:, : 12 * 128] = d.q.reshape(2, -1)
    qv = big[:, : 12 * 128].view(2, 12, 128)
    got = ops.paged_decode(qv, d.k_pool, d.v_pool, d.block_tables, d.context_lens).cpu()
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp)


def test_out_of_range_table_entries_do_not_fault():
    """Garbage block ids are clamped into the pool (no fault); valid rows are unaffected."""
    lengths = [40, 40]
    w = workloads.make_decode_workload("clamp", 21, 2, 12, 2, 128, lengths)
    w.block_tables = w.block_tables.clone()
    w.block_tables[1, :] = 10 ** 6
    got, _ = run_decode(w)
    exp, _, _ = oracle_decode(workloads.make_decode_workload("clamp", 21, 2, 12, 2, 128, lengths))
    assert_attention_close(got[:1].numpy(), exp[:1])
    assert torch.isfinite(got[1].float()).all()


def test_lse_merge_entry_point():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((6, 128))
    k = rng.standard_normal((300, 128))
    v = rng.standard_normal((300, 128))
    po, pl = R.split_attention(q, k, v, [0, 50, 50, 170, 300])
    out, lse = ops.lse_merge(torch.tensor(po, dtype=torch.float32, device=DEV),
                             torch.tensor(pl, dtype=torch.float32, device=DEV), with_lse=True)
    exp_o, exp_l = R.lse_merge(po, pl)
    assert_attention_close(out.cpu().numpy(), exp_o)
    np.testing.assert_allclose(lse.cpu().numpy(), exp_l, atol=1e-4)


def test_error_codes_surface_as_exceptions():
    q = torch.zeros(1, 12, 1024, dtype=torch.float16, device=DEV)
    pool = torch.zeros(4, 16, 2, 1024, dtype=torch.float16, device=DEV)
    t = torch.zeros(1, 1, dtype=torch.int32, device=DEV)
    c = torch.ones(1, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported"):
        ops.paged_decode(q, pool, pool, t, c)


@pytest.mark.parametrize("bs", [16, 32])
def test_fused_write_short_contexts(bs):
    """The decoded token's row is stored and re-read inside the kernel; at L=1 the output
    must equal v_new exactly for every query head of the group."""
    lengths = [1, 2, 15, 16, 17, 63, 64, 65, 130]
    w = workloads.make_decode_workload("fused", 40 + bs, len(lengths), 12, 2, 128, lengths,
                                       block_size=bs, with_new_kv=True)
    got, d = run_decode(w)
    exp, kp, vp = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="fused short")
    v_new = w.v_new.numpy()
    for h in range(12):
        assert (got[0, h].numpy() == v_new[0, h // 6]).all()
    assert d.k_pool.cpu().numpy().tobytes() == kp.tobytes()
    assert d.v_pool.cpu().numpy().tobytes() == vp.tobytes()


def test_workspace_reuse_across_shapes():
    """One workspace serves calls of different shapes and split counts in a row (the split
    tickets it holds return to zero after every call)."""
    big = workloads.c2_workload(batch=32)
    small = workloads.make_decode_workload("small", 3, 3, 12, 2, 128, [700, 5, 2000])
    exp_big, _, _ = oracle_decode(big)
    exp_small, _, _ = oracle_decode(small)
    ws = torch.zeros((ops.decode_workspace_bytes(32, 12, 128, 4096, 2048),),
                     dtype=torch.uint8, device=DEV)
    db, dsm = big.to(DEV), small.to(DEV)
    for target in (2048, 7, 512, 64):
        ob = ops.paged_decode(db.q, db.k_pool, db.v_pool, db.block_tables, db.context_lens,
                              k_new=db.k_new, v_new=db.v_new, workspace=ws, target_splits=target)
        osm = ops.paged_decode(dsm.q, dsm.k_pool, dsm.v_pool, dsm.block_tables, dsm.context_lens,
                               workspace=ws, target_splits=target)
        assert_attention_close(ob.cpu().numpy(), exp_big, what=f"big t={target}")
        assert_attention_close(osm.cpu().numpy(), exp_small, what=f"small t={target}")


def test_split_merge_repeated_calls_are_stable():
    """The in-kernel split-K merge (coherent partials + ticket) gives the same, correct
    result on every one of many back-to-back calls, for several split counts."""
    w = workloads.c2_workload()
    exp, _, _ = oracle_decode(w)
    d = w.to(DEV)
    outs = []
    for rep in range(8):
        for target in (96, 256, 777, 2048):
            outs.append((target, ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables,
                                                  d.context_lens, k_new=d.k_new, v_new=d.v_new,
                                                  target_splits=target)))
    torch.cuda.synchronize()
    first = {}
    for target, o in outs:
        got = o.cpu().numpy()
        assert_attention_close(got, exp, what=f"target={target}")
        if target in first:
            assert (first[target] == got).all(), "results differ between identical calls"
        else:
            first[target] = got


@pytest.mark.parametrize("hq,hkv,d", [(12, 2, 128), (6, 1, 128), (14, 2, 64)])
def test_decode_large_scores(hq, hkv, d):
    """q scaled by 16: scores spread over hundreds, so every running max (per tile,
    per wave, per piece, across the split merge) must be exact or exp2 overflows."""
    w = workloads.make_decode_workload("large", 9 + hq, 6, hq, hkv, d, [700, 5, 2000, 33, 4096, 129])
    w.q = (w.q.float() * 16).half()
    got, _ = run_decode(w, fuse=False)
    assert np.isfinite(got.numpy()).all()
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what=f"large scores {hq}/{hkv}/{d}")


# --------------------------------------------------------------------------------------
# shared-prefix (cascade) decode: same results as the plain decode on the same tables
# --------------------------------------------------------------------------------------

def run_shared_prefix(w: workloads.DecodeWorkload, fuse: bool = False, target_splits: int = 0):
    d = w.to(DEV)
    out = ops.paged_decode_shared_prefix(
        d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
        d.meta["group_offsets"].to(DEV), d.meta["prefix_lens"].to(DEV),
        k_new=d.k_new if fuse else None, v_new=d.v_new if fuse else None,
        target_splits=target_splits)
    torch.cuda.synchronize()
    return out.cpu(), d


def test_shared_prefix_c3_shape_matches_oracle_and_plain_decode():
    w = workloads.c3_workload(groups=2, per_group=8)
    got, _ = run_shared_prefix(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="cascade C3 (2x8)")
    plain, _ = run_decode(w)
    assert_attention_close(got.numpy(), plain.numpy().astype(np.float64), what="cascade vs plain")


@pytest.mark.parametrize("hq,hkv,d,bs", [(12, 2, 128, 16), (14, 2, 64, 16), (8, 1, 128, 32),
                                          (16, 4, 64, 16)])
def test_shared_prefix_edge_cases(hq, hkv, d, bs):
    """Groups of 3 (prefix 40 tokens: only whole blocks are shared), 1 and 0
    members, a group of 5 in which one member's context ends exactly at the
    prefix, one inside it and one is inactive, and rows outside every group."""
    groups = [(3, 40), (1, 64), (0, 32), (5, 512)]
    w = workloads.shared_prefix_workload(11, groups, singles=3, hq=hq, hkv=hkv, d=d,
                                         block_size=bs, member_lens={5: 512, 6: 505, 7: 0})
    got, _ = run_shared_prefix(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what=f"edge cases {hq}/{hkv}/{d} bs{bs}")
    assert not got[7].any(), "inactive member must give exact zeros"


def test_shared_prefix_fused_page_write_is_bit_exact():
    """The decoded token lies past the shared prefix: written into the member's
    private block in the same call, byte-exact, and attended."""
    w = workloads.shared_prefix_workload(12, [(6, 256), (4, 1024)], singles=2, with_new_kv=True,
                                         tail=(1, 200))
    got, d = run_shared_prefix(w, fuse=True)
    exp, kp, vp = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="cascade + fused write")
    assert np.array_equal(d.k_pool.cpu().numpy().view(np.int16), kp.view(np.int16))
    assert np.array_equal(d.v_pool.cpu().numpy().view(np.int16), vp.view(np.int16))


def test_shared_prefix_without_groups_is_the_plain_decode():
    w = workloads.c2_workload(batch=16)
    d = w.to(DEV)
    empty = torch.zeros(1, dtype=torch.int32, device=DEV)
    got = ops.paged_decode_shared_prefix(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                                         empty, empty[:0])
    plain = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens)
    assert torch.equal(got, plain)


def test_c3_full_plain_and_cascade_against_oracle():
    """Full C3 (8 groups x 32 rows sharing 2048 tokens, private tails U{16..2048}):
    the plain decode and the shared-prefix decode each against the float64 oracle."""
    w = workloads.c3_workload()
    exp, _, _ = oracle_decode(w)
    plain, _ = run_decode(w)
    assert_attention_close(plain.numpy(), exp, what="full C3 plain decode")
    cascade, _ = run_shared_prefix(w)
    assert_attention_close(cascade.numpy(), exp, what="full C3 cascade decode")


def test_shared_prefix_full_c3_against_plain_decode_and_repeatable():
    """Full C3 (8 groups x 32 sharing 2048 tokens): the cascade agrees with the
    plain decode to the contract tolerance and is bit-identical across calls."""
    w = workloads.c3_workload()
    d = w.to(DEV)
    go, pl = d.meta["group_offsets"].to(DEV), d.meta["prefix_lens"].to(DEV)
    outs = [ops.paged_decode_shared_prefix(d.q, d.k_pool, d.v_pool, d.block_tables,
                                           d.context_lens, go, pl) for _ in range(3)]
    plain = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens)
    torch.cuda.synchronize()
    assert_attention_close(outs[0].cpu().numpy(), plain.cpu().numpy().astype(np.float64),
                           what="full C3 cascade vs plain")
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("hq,hkv,d,bs", [(12, 2, 128, 16), (8, 1, 64, 32)])
def test_shared_prefix_long_prefixes_cross_the_block_id_reload(hq, hkv, d, bs):
    """Prefixes of 20000 and 17000 tokens: each of the prefix pass's four key
    splits holds more than 61 blocks of 64 keys, so every wave reloads its
    block ids in mid-pipeline (the next 64 blocks' ids); one member's context
    ends inside its prefix and one row has none."""
    groups = [(3, 20000), (2, 17000)]
    w = workloads.shared_prefix_workload(31 + d, groups, singles=1, hq=hq, hkv=hkv, d=d,
                                         block_size=bs, tail=(1, 200), member_lens={4: 9000})
    got, _ = run_shared_prefix(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what=f"long prefixes {hq}/{hkv}/{d} bs{bs}")


# --------------------------------------------------------------------------------------
# large batches: the plain decode (piece kernel) at 160 and 2048 rows, and the
# shared-prefix decode, whose suffix pass runs the balanced kernel from 128 rows
# (equal tile ranges per workgroup, whatever the context-length mix)
# --------------------------------------------------------------------------------------

def _with_lengths(seed, lengths, hq, hkv, d, bs=16, fuse=True):
    """A decode workload whose rows have exactly `lengths` (0 = inactive row)."""
    w = workloads.make_decode_workload("balanced", seed, len(lengths), hq, hkv, d,
                                       [max(n, 1) for n in lengths], block_size=bs,
                                       with_new_kv=fuse)
    w.context_lens = torch.tensor(lengths, dtype=torch.int32)
    return w


def _random_lengths(seed, batch, lo, hi):
    return np.random.default_rng(seed).integers(lo, hi + 1, size=batch).tolist()


LARGE_SHAPES = [(12, 2, 128, 16), (14, 2, 64, 16), (16, 1, 128, 32), (8, 8, 64, 64),
                (28, 4, 128, 16), (16, 2, 64, 32)]


@pytest.mark.parametrize("hq,hkv,d,bs", LARGE_SHAPES)
def test_large_ragged_batch_with_inactive_rows_and_page_write(hq, hkv, d, bs):
    lengths = _random_lengths(hq * 13 + d + bs, 160, 1, 700)
    lengths[1:5] = [1, 16, 17, 3000]
    for b in range(0, 160, 17):
        lengths[b] = 0
    w = _with_lengths(hq + d + bs, lengths, hq, hkv, d, bs)
    got, dv = run_decode(w)
    exp, kp, vp = oracle_decode(w)
    assert torch.count_nonzero(got[0]) == 0 and torch.count_nonzero(got[17]) == 0
    assert_attention_close(got.numpy(), exp, what=f"large {hq}/{hkv}/{d} bs {bs}")
    assert dv.k_pool.cpu().numpy().tobytes() == kp.tobytes()
    assert dv.v_pool.cpu().numpy().tobytes() == vp.tobytes()


def test_large_batch_of_tiny_sequences():
    w = _with_lengths(2048, _random_lengths(2048, 2048, 0, 40), 8, 1, 128, fuse=False)
    got, _ = run_decode(w, fuse=False)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="2048 tiny rows")


@pytest.mark.parametrize("hq,hkv,d,bs", LARGE_SHAPES)
def test_balanced_cascade_ragged_batch_with_inactive_rows_and_page_write(hq, hkv, d, bs):
    """160 rows: groups of 48, 32, 24 and 1 members (prefixes of 256, 64, 1000 and
    512 tokens; whole blocks shared), then 55 rows of their own.  Inactive rows in a
    group, as its only member, and outside; rows of 1, 16, 17 and 3000 tokens.  The
    decoded token is written past each member's prefix, into its private block."""
    groups = [(48, 256), (32, 64), (24, 1000), (1, 512)]
    lens = {50: 0, 104: 0, 130: 0, 105: 1, 106: 16, 107: 17, 108: 3000}
    w = workloads.shared_prefix_workload(hq * 13 + d + bs, groups, singles=55, hq=hq, hkv=hkv,
                                         d=d, block_size=bs, tail=(1, 700), member_lens=lens,
                                         with_new_kv=True)
    assert w.batch == 160
    got, dv = run_shared_prefix(w, fuse=True)
    exp, kp, vp = oracle_decode(w)
    for b in (50, 104, 130):
        assert torch.count_nonzero(got[b]) == 0, f"inactive row {b}"
    assert_attention_close(got.numpy(), exp, what=f"balanced cascade {hq}/{hkv}/{d} bs {bs}")
    assert dv.k_pool.cpu().numpy().tobytes() == kp.tobytes()
    assert dv.v_pool.cpu().numpy().tobytes() == vp.tobytes()


def test_balanced_cascade_many_tiny_sequences():
    """2048 rows, group size 8: 200 groups of 4 sharing one 16-token block with
    suffixes of 0..40 tokens (members ending at or inside the prefix included), and
    1248 rows of 0..40 tokens: workgroup ranges hold many short segments (the
    per-segment barrier path when their states outnumber the slots)."""
    w = workloads.shared_prefix_workload(2048, [(4, 16)] * 200, singles=1248, hq=8, hkv=1,
                                         d=128, tail=(0, 40), member_lens={1: 5, 2: 0, 9: 16})
    assert w.batch == 2048
    got, _ = run_shared_prefix(w)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(got.numpy(), exp, what="2048 tiny rows, cascade")
    assert torch.count_nonzero(got[2]) == 0


def test_balanced_cascade_repeated_calls_are_identical_and_share_the_workspace():
    """The cascade at 200 rows and a 3-row plain decode alternate on one workspace
    (its split tickets are shared): every call is right and the large one is
    bit-identical from call to call."""
    w = workloads.shared_prefix_workload(99, [(50, 512), (50, 1024)], singles=100,
                                         tail=(100, 3000))
    small = workloads.make_decode_workload("small", 5, 3, 12, 2, 128, [700, 5, 2000])
    exp, _, _ = oracle_decode(w)
    exp_small, _, _ = oracle_decode(small)
    d, ds = w.to(DEV), small.to(DEV)
    go, pl = d.meta["group_offsets"].to(DEV), d.meta["prefix_lens"].to(DEV)
    need = _lib.load().fe_paged_decode_shared_prefix_workspace_size(
        w.batch, 12, 2, 128, w.block_tables.shape[1] * 16, 2, 0)
    ws = torch.zeros((need,), dtype=torch.uint8, device=DEV)
    first = None
    for rep in range(6):
        o = ops.paged_decode_shared_prefix(d.q, d.k_pool, d.v_pool, d.block_tables,
                                           d.context_lens, go, pl, workspace=ws)
        os_ = ops.paged_decode(ds.q, ds.k_pool, ds.v_pool, ds.block_tables, ds.context_lens,
                               workspace=ws)
        got = o.cpu().numpy()
        assert_attention_close(got, exp, what=f"rep {rep}")
        assert_attention_close(os_.cpu().numpy(), exp_small, what=f"small rep {rep}")
        if first is None:
            first = got
        assert (first == got).all(), "results differ between identical calls"


# --------------------------------------------------------------------------------------
# decode plan (fe_paged_decode_plan / fe_paged_decode_planned): one plan per decode step,
# reused by every layer; results must be bit-identical to the unplanned launch
# --------------------------------------------------------------------------------------

def _planned_cases():
    c2 = workloads.c2_workload()
    lens = [0, 1, 15, 16, 17, 200, 0, 1023, 4096, 64]  # inactive rows, tile and piece edges
    edge = workloads.make_decode_workload("edges", 91, len(lens), 12, 2, 128, lens,
                                          width=256, with_new_kv=True)
    c1 = workloads.c1_workload()
    big = workloads.make_decode_workload("bs32", 93, 5, 16, 2, 128, [3000, 17, 512, 0, 9000],
                                         block_size=32, with_new_kv=True)
    return [c2, edge, c1, big]


@pytest.mark.parametrize("case", range(4))
def test_planned_decode_is_bit_identical_and_reusable(case):
    w = _planned_cases()[case]
    print(f"planned decode case {w.name}", flush=True)
    d = w.to(DEV)
    nb, bs, hkv = d.k_pool.shape[0], d.k_pool.shape[1], d.k_pool.shape[2]
    plan = ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs)
    # three "layers": own pools and queries, the same tables and lengths
    for layer in range(3):
        g = torch.Generator().manual_seed(100 * case + layer)
        kp = torch.randn(d.k_pool.shape, generator=g).half().to(DEV)
        vp = torch.randn(d.v_pool.shape, generator=g).half().to(DEV)
        q = torch.randn(d.q.shape, generator=g).half().to(DEV)
        kn = vn = None
        if d.k_new is not None:
            kn = torch.randn(d.k_new.shape, generator=g).half().to(DEV)
            vn = torch.randn(d.v_new.shape, generator=g).half().to(DEV)
        kp2, vp2 = kp.clone(), vp.clone()
        ref = ops.paged_decode(q, kp, vp, d.block_tables, d.context_lens, k_new=kn, v_new=vn)
        got = ops.paged_decode(q, kp2, vp2, d.block_tables, d.context_lens, k_new=kn, v_new=vn,
                               plan=plan)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"{w.name} layer {layer}: planned output differs"
        assert torch.equal(kp2, kp) and torch.equal(vp2, vp), f"{w.name}: page write differs"
    # and against the oracle for the workload's own pools
    out = ops.paged_decode(d.q, d.k_pool.clone(), d.v_pool.clone(), d.block_tables,
                           d.context_lens, k_new=d.k_new, v_new=d.v_new, plan=plan)
    exp, _, _ = oracle_decode(w)
    assert_attention_close(out.cpu().numpy(), exp, what=f"planned {w.name}")


def test_planned_decode_rejects_a_foreign_plan():
    w = workloads.c1_workload()
    d = w.to(DEV)
    nb, bs, hkv = d.k_pool.shape[0], d.k_pool.shape[1], d.k_pool.shape[2]
    plan = ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs)
    other = d.context_lens.clone()
    with pytest.raises(ValueError, match="other block_tables"):
        ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, other, plan=plan)
    small = torch.empty(16, dtype=torch.uint8, device=DEV)
    lib = _lib.load()
    rc = lib.fe_paged_decode_plan(d.block_tables.data_ptr(), d.block_tables.shape[1],
                                  d.context_lens.data_ptr(), nb, d.q.shape[0], hkv, bs, 0,
                                  small.data_ptr(), small.numel(), None)
    assert rc == _lib.FE_ERR_WORKSPACE


def _planned_call(d, out, plan, tables):
    """fe_paged_decode_planned through the C ABI (ops refuses a plan for other tensors
    before launching; the library's own check is what is tested here)."""
    nb, bs, hkv, hd = d.k_pool.shape
    need = ops.decode_workspace_bytes(d.q.shape[0], d.q.shape[1], hd, tables.shape[1] * bs)
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    rc = _lib.load().fe_paged_decode_planned(
        d.q.data_ptr(), d.q.stride(0), out.data_ptr(), d.k_new.data_ptr(), d.v_new.data_ptr(),
        d.k_new.stride(0), d.k_pool.data_ptr(), d.v_pool.data_ptr(), nb, tables.data_ptr(),
        tables.shape[1], d.context_lens.data_ptr(), ws.data_ptr(), need, d.q.shape[0],
        d.q.shape[1], hkv, hd, bs, 1.0 / math.sqrt(hd), 0, plan.buffer.data_ptr(),
        plan.buffer.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.FE_OK, _lib.error_string(rc)
    torch.cuda.synchronize()


def test_planned_decode_refuses_a_plan_recorded_for_other_tables():
    """A plan whose record of the tables' address is not the call's: NaN in every row,
    no page write, error word FE_PLAN_ERR_SIZES; the next plan call clears the word."""
    w = _planned_cases()[1]
    d = w.to(DEV)
    nb, bs, hkv = d.k_pool.shape[0], d.k_pool.shape[1], d.k_pool.shape[2]
    plan = ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs)
    k0, v0 = d.k_pool.clone(), d.v_pool.clone()
    out = torch.zeros_like(d.q)
    _planned_call(d, out, plan, d.block_tables.clone())
    assert torch.isnan(out).all(), "rows computed from a plan for other tables"
    assert ops.plan_error(plan) == ops.PLAN_ERR_SIZES
    assert torch.equal(d.k_pool, k0) and torch.equal(d.v_pool, v0), "page written"
    ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs, out=plan)
    assert ops.plan_error(plan) == 0
    kp, vp = d.k_pool.clone(), d.v_pool.clone()
    ref = ops.paged_decode(d.q, kp, vp, d.block_tables, d.context_lens, k_new=d.k_new,
                           v_new=d.v_new)
    _planned_call(d, out, plan, d.block_tables)
    assert torch.equal(out, ref) and ops.plan_error(plan) == 0
    assert torch.equal(d.k_pool, kp) and torch.equal(d.v_pool, vp)


def test_stale_plan_rows_are_nan_and_write_no_page():
    """Lengths changed in place after the plan call (a plan of the previous step):
    those rows give NaN and write nothing to the pools, the error word is
    FE_PLAN_ERR_STALE, and every other row is what an unplanned call gives."""
    w = _planned_cases()[1]                  # lengths [0, 1, 15, 16, 17, 200, 0, 1023, 4096, 64]
    d = w.to(DEV)
    nb, bs, hkv = d.k_pool.shape[0], d.k_pool.shape[1], d.k_pool.shape[2]
    plan = ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs)
    stale = [2, 5]                           # 15 -> 16 and 200 -> 201: tile and piece edges
    d.context_lens[stale] += 1
    k0, v0 = d.k_pool.clone(), d.v_pool.clone()
    got = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                           k_new=d.k_new, v_new=d.v_new, plan=plan)
    torch.cuda.synchronize()
    assert ops.plan_error(plan) == ops.PLAN_ERR_STALE
    assert torch.isnan(got[stale]).all()
    keep = [b for b in range(w.batch) if b not in stale]
    # the same call without the stale rows (inactive: no output, no page write)
    lens = d.context_lens.clone()
    lens[stale] = 0
    kp, vp = k0.clone(), v0.clone()
    ref = ops.paged_decode(d.q, kp, vp, d.block_tables, lens, k_new=d.k_new, v_new=d.v_new)
    torch.cuda.synchronize()
    assert torch.isfinite(got[keep]).all()
    diff = (got[keep].float() - ref[keep].float()).abs().max().item()
    assert diff <= 2e-3, f"kept rows differ from the unplanned call by {diff}"
    assert torch.equal(d.k_pool, kp) and torch.equal(d.v_pool, vp), "stale rows wrote a page"
