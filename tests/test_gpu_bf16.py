"""GPU: bfloat16 forms of the paged decode and prefill against the oracle.

The reference builds its models and KV caches in bfloat16 as well as float16
(inference/models/qwen2.py:54, engine/kv_cache/allocator.py:24).  The bf16
entry points take bf16 q / pools / new rows and return bf16; the oracle runs in
float64 on the same bf16 values (converted exactly to float32 first).

Tolerance: the fp16 contract (max |err| <= 2e-3, mean <= 2e-4) scaled by the
ratio of the two formats' unit roundoffs, 2^-8 / 2^-11 = 8: max |err| <= 1.6e-2,
mean |err| <= 1.6e-3.  The kernel rounds twice to bf16 (the probabilities before
the PV product and the output), where the fp16 kernel rounds the same two values
to fp16.  Page writes are byte copies and stay bit-exact.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flexengine_amd import _lib, attention, ops, workloads
from flexengine_amd.kv_cache import CacheLayout, PagedKVCache
from oracle import paged_ref as R
from tests.parity import MAX_ABS_TOL, MEAN_ABS_TOL, assert_attention_close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF16 = torch.bfloat16
ULP_RATIO = 2.0 ** -8 / 2.0 ** -11
BF16_MAX_TOL = MAX_ABS_TOL * ULP_RATIO
BF16_MEAN_TOL = MEAN_ABS_TOL * ULP_RATIO


def close_bf16(got: torch.Tensor, exp: np.ndarray, what: str = ""):
    assert got.dtype == BF16, got.dtype
    mx, mean = assert_attention_close(got.float().cpu().numpy(), exp, BF16_MAX_TOL,
                                      BF16_MEAN_TOL, what)
    print(f"{what}: max abs {mx:.3e} mean abs {mean:.3e}", flush=True)


def f32(t: torch.Tensor | None) -> np.ndarray | None:
    """bf16 -> float32 numpy (exact)."""
    return None if t is None else t.float().numpy()


def to_bf16(w: workloads.DecodeWorkload) -> workloads.DecodeWorkload:
    def cv(t):
        return None if t is None else t.float().to(BF16)
    return workloads.DecodeWorkload(w.name + "-bf16", cv(w.q), cv(w.k_pool), cv(w.v_pool),
                                    w.block_tables, w.context_lens, cv(w.k_new), cv(w.v_new),
                                    w.unique_tokens, dict(w.meta))


def oracle_decode(w: workloads.DecodeWorkload):
    """float64 decode of a bf16 workload, and its pools after the page write as int16 bits."""
    kp = w.k_pool.view(torch.int16).numpy().copy()
    vp = w.v_pool.view(torch.int16).numpy().copy()
    if w.k_new is not None:
        R.write_kv_decode(kp, vp, w.block_tables.numpy(), w.context_lens.numpy(),
                          w.k_new.view(torch.int16).numpy(), w.v_new.view(torch.int16).numpy(),
                          w.block_size)
    kf = torch.from_numpy(kp).view(BF16).float().numpy()
    vf = torch.from_numpy(vp).view(BF16).float().numpy()
    out = R.decode_reference(f32(w.q), kf, vf, w.block_tables.numpy(), w.context_lens.numpy(),
                             w.block_size)
    return out, kp, vp


def _decode_cases():
    lens = [0, 1, 15, 16, 17, 200, 0, 1023, 4096, 64]
    return [
        to_bf16(workloads.c1_workload()),
        to_bf16(workloads.c2_workload()),
        to_bf16(workloads.make_decode_workload("edges", 191, len(lens), 12, 2, 128, lens,
                                               width=256, with_new_kv=True)),
        to_bf16(workloads.make_decode_workload("d64-g7", 192, 6, 14, 2, 64,
                                               [1, 33, 700, 2049, 5, 9000], with_new_kv=True)),
        to_bf16(workloads.make_decode_workload("bs32", 193, 5, 16, 2, 128,
                                               [3000, 17, 512, 0, 9000], block_size=32,
                                               with_new_kv=True)),
    ]


@pytest.mark.parametrize("case", range(5))
def test_bf16_decode_against_oracle_with_fused_page_write(case):
    w = _decode_cases()[case]
    print(f"bf16 decode case {w.name}", flush=True)
    d = w.to(DEV)
    got = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                           k_new=d.k_new, v_new=d.v_new)
    torch.cuda.synchronize()
    exp, kp, vp = oracle_decode(w)
    close_bf16(got, exp, w.name)
    assert d.k_pool.cpu().view(torch.int16).numpy().tobytes() == kp.tobytes()
    assert d.v_pool.cpu().view(torch.int16).numpy().tobytes() == vp.tobytes()


@pytest.mark.parametrize("case", [1, 2, 4])
def test_bf16_planned_decode_is_bit_identical(case):
    w = _decode_cases()[case]
    print(f"bf16 planned decode case {w.name}", flush=True)
    d = w.to(DEV)
    nb, bs, hkv = d.k_pool.shape[0], d.k_pool.shape[1], d.k_pool.shape[2]
    plan = ops.paged_decode_plan(d.block_tables, d.context_lens, nb, hkv, bs)
    kp, vp = d.k_pool.clone(), d.v_pool.clone()
    ref = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                           k_new=d.k_new, v_new=d.v_new)
    got = ops.paged_decode(d.q, kp, vp, d.block_tables, d.context_lens, k_new=d.k_new,
                           v_new=d.v_new, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), f"{w.name}: planned bf16 output differs"
    assert torch.equal(kp, d.k_pool) and torch.equal(vp, d.v_pool)


def test_bf16_and_fp16_decode_agree_on_shared_values():
    """Values exactly representable in both formats: the two kernels differ only by the
    roundings of P and of the output, so they agree to the bf16 tolerance."""
    w = to_bf16(workloads.c2_workload())
    w.k_new = w.v_new = None
    d = w.to(DEV)
    out_b = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens)
    out_h = ops.paged_decode(d.q.half(), d.k_pool.half(), d.v_pool.half(), d.block_tables,
                             d.context_lens)
    torch.cuda.synchronize()
    exp, _, _ = oracle_decode(w)
    assert_attention_close(out_h.cpu().numpy(), exp, what="fp16 kernel on bf16 values")
    close_bf16(out_b, exp, "bf16 kernel")


# --------------------------------------------------------------------------------------
# prefill
# --------------------------------------------------------------------------------------

def _prefill_case(seed, n_new, cached, hq=12, hkv=2, d=128, bs=16, q_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    ctx = [c + n for c, n in zip(cached, n_new)]
    pages = [math.ceil(x / bs) for x in ctx]
    nb = sum(pages) + 3
    k_pool = torch.randn(nb, bs, hkv, d, generator=g).to(BF16)
    v_pool = torch.randn(nb, bs, hkv, d, generator=g).to(BF16)
    perm = torch.randperm(nb, generator=g)
    tables = torch.zeros(len(ctx), max(pages), dtype=torch.int32)
    at = 0
    for i, p in enumerate(pages):
        tables[i, :p] = perm[at:at + p]
        tables[i, p:] = perm[at + p - 1] if p else 0
        at += p
    offs = torch.tensor(np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32))
    q = (torch.randn(int(offs[-1]), hq, d, generator=g) * q_scale).to(BF16)
    return q, offs, torch.tensor(ctx, dtype=torch.int32), tables, k_pool, v_pool


def _prefill(q, offs, ctx, tables, kp, vp):
    n_new = (offs[1:] - offs[:-1]).tolist()
    out = ops.prefill_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), tables.to(DEV), offs.to(DEV),
                            ctx.to(DEV), max(n_new) if n_new else 0)
    torch.cuda.synchronize()
    return out


def _prefill_oracle(q, offs, ctx, tables, kp, vp, bs):
    return R.prefill_reference(f32(q), offs.numpy(), ctx.numpy(), f32(kp), f32(vp),
                               tables.numpy(), bs)


@pytest.mark.parametrize("n_new,cached", [([1], [0]), ([16], [0]), ([17], [3]), ([65], [100]),
                                          ([130, 7, 1], [0, 40, 999]), ([0, 33], [10, 10])])
def test_bf16_ragged_prefill(n_new, cached):
    case = _prefill_case(sum(n_new) + 5 * len(n_new), n_new, cached)
    print(f"bf16 prefill n={n_new} c={cached}", flush=True)
    close_bf16(_prefill(*case), _prefill_oracle(*case, 16), f"bf16 prefill n={n_new}")


@pytest.mark.parametrize("hq,hkv,d,bs", [(14, 2, 64, 16), (16, 2, 128, 32), (8, 8, 64, 16)])
def test_bf16_prefill_shapes(hq, hkv, d, bs):
    case = _prefill_case(hq + d + bs, [70, 3], [25, 200], hq, hkv, d, bs)
    print(f"bf16 prefill shape {hq}/{hkv}/{d}/{bs}", flush=True)
    close_bf16(_prefill(*case), _prefill_oracle(*case, bs), f"bf16 prefill {hq}/{hkv}/{d}/{bs}")


def test_bf16_prefill_large_scores():
    """Scores spread over hundreds: the running max and the bf16 probabilities stay finite."""
    case = _prefill_case(83, [40, 130, 1], [300, 20, 64], 12, 2, 128, q_scale=8.0)
    got = _prefill(*case)
    assert torch.isfinite(got.float()).all()
    close_bf16(got, _prefill_oracle(*case, 16), "bf16 prefill large scores")


def test_bf16_c4_prefill_chunks_full():
    w = workloads.c4_workload()
    q, kp, vp = w.q.float().to(BF16), w.k_pool.float().to(BF16), w.v_pool.float().to(BF16)
    got = _prefill(q, w.q_offsets, w.context_lens, w.block_tables, kp, vp)
    exp = _prefill_oracle(q, w.q_offsets, w.context_lens, w.block_tables, kp, vp, 16)
    close_bf16(got, exp, "bf16 C4 prefill")


def test_bf16_per_request_interface():
    """A bf16 PagedKVCache through attention_for_request: multi-token chunk (prefill
    kernel) then one-token query (decode kernel)."""
    g = torch.Generator().manual_seed(404)
    cache = PagedKVCache(CacheLayout(1, 64, 16, 2, 64), device=DEV, dtype=BF16)
    length = 300
    cache.reserve("r", length)
    keys = torch.randn(length, 2, 64, generator=g).to(BF16)
    values = torch.randn(length, 2, 64, generator=g).to(BF16)
    cache.write(0, "r", 0, keys.to(DEV), values.to(DEV))
    q = torch.randn(37, 14, 64, generator=g).to(BF16)
    pos = torch.arange(length - 37, length)
    got = attention.attention_for_request(q.to(DEV), cache, 0, "r", length, pos.to(DEV))
    exp = R.attention_materialized(f32(q), f32(keys), f32(values), pos.numpy())
    close_bf16(got, exp, "bf16 per-request chunk")
    got1 = attention.attention_for_request(q[-1:].to(DEV), cache, 0, "r", length,
                                           pos[-1:].to(DEV))
    close_bf16(got1, exp[-1:], "bf16 per-request decode")
    k_back, _ = cache.materialize(0, "r", length)
    assert torch.equal(k_back.cpu(), keys)


@pytest.mark.parametrize("hq,hkv,d,bs,n_new,cached", [
    (8, 8, 64, 4, [20], [7]),               # the tile kernel, one row tile per wave
    (14, 2, 64, 1, [37, 5], [0, 300]),       # block size 1
    (12, 2, 128, 8, [3], [900]),             # few row blocks: key splits merged by ticket
    (12, 2, 128, 8, [150, 90], [60, 500]),   # many rows: two row tiles per wave
])
def test_bf16_prefill_small_blocks(hq, hkv, d, bs, n_new, cached):
    """Block sizes below 16 run the tile kernel (prefill_kernel) in its bf16 form."""
    case = _prefill_case(hq * bs + d + sum(n_new), n_new, cached, hq, hkv, d, bs)
    print(f"bf16 prefill bs={bs} {hq}/{hkv}/{d} n={n_new} c={cached}", flush=True)
    close_bf16(_prefill(*case), _prefill_oracle(*case, bs), f"bf16 prefill bs={bs} n={n_new}")


# --------------------------------------------------------------------------------------
# shared-prefix (cascade) decode
# --------------------------------------------------------------------------------------

def _shared_prefix(w: workloads.DecodeWorkload, fuse: bool):
    d = w.to(DEV)
    out = ops.paged_decode_shared_prefix(
        d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
        d.meta["group_offsets"].to(DEV), d.meta["prefix_lens"].to(DEV),
        k_new=d.k_new if fuse else None, v_new=d.v_new if fuse else None)
    torch.cuda.synchronize()
    return out, d


def test_bf16_shared_prefix_c3_shape():
    """C3's shape at 2 groups x 8 (the piece kernel runs the suffixes below 128 rows)."""
    w = to_bf16(workloads.c3_workload(groups=2, per_group=8))
    got, _ = _shared_prefix(w, fuse=False)
    exp, _, _ = oracle_decode(w)
    close_bf16(got, exp, "bf16 cascade C3 (2x8)")


def test_bf16_shared_prefix_long_prefix():
    """A 20000-token prefix in bf16: the prefix pass's splits cross the
    mid-pipeline block-id reload."""
    w = to_bf16(workloads.shared_prefix_workload(23, [(3, 20000)], singles=1, hq=12, hkv=2,
                                                 d=128, tail=(1, 200)))
    got, _ = _shared_prefix(w, fuse=False)
    exp, _, _ = oracle_decode(w)
    close_bf16(got, exp, "bf16 cascade, 20000-token prefix")


@pytest.mark.parametrize("hq,hkv,d,bs", [(12, 2, 128, 16), (14, 2, 64, 32)])
def test_bf16_shared_prefix_edge_groups(hq, hkv, d, bs):
    """Groups of 3 (prefix of 40 tokens: whole blocks only), 1 and 0 members and one of
    5 whose members end at the prefix, inside it and inactive; rows outside every group.
    No decode-step write: a member ending at the prefix would write its token into a
    shared block, which the caller must not ask for (the reference refuses it)."""
    groups = [(3, 40), (1, 64), (0, 32), (5, 512)]
    w = to_bf16(workloads.shared_prefix_workload(21, groups, singles=3, hq=hq, hkv=hkv, d=d,
                                                 block_size=bs,
                                                 member_lens={5: 512, 6: 505, 7: 0}))
    print(f"bf16 cascade edges {hq}/{hkv}/{d}/{bs}", flush=True)
    got, _ = _shared_prefix(w, fuse=False)
    exp, _, _ = oracle_decode(w)
    close_bf16(got, exp, f"bf16 cascade edges {hq}/{hkv}/{d}/{bs}")
    assert not got[7].any(), "inactive member must give exact zeros"


def test_bf16_balanced_cascade_with_page_write():
    """160 rows: the suffixes run on the balanced kernel in its bf16 form."""
    groups = [(48, 256), (32, 64), (24, 1000), (1, 512)]
    lens = {50: 0, 105: 1, 106: 16, 107: 17, 108: 3000}
    w = to_bf16(workloads.shared_prefix_workload(77, groups, singles=55, hq=12, hkv=2, d=128,
                                                 block_size=16, tail=(1, 700), member_lens=lens,
                                                 with_new_kv=True))
    assert w.batch == 160
    got, dv = _shared_prefix(w, fuse=True)
    exp, kp, vp = oracle_decode(w)
    assert torch.count_nonzero(got[50]) == 0
    close_bf16(got, exp, "bf16 balanced cascade")
    assert dv.k_pool.cpu().view(torch.int16).numpy().tobytes() == kp.tobytes()
    assert dv.v_pool.cpu().view(torch.int16).numpy().tobytes() == vp.tobytes()


def test_bf16_lse_merge():
    """fe_lse_merge_bf16 on fp32 partials of a split attention (zero-length splits
    included) against the oracle's merge, output rounded to bf16."""
    rng = np.random.default_rng(8)
    q = rng.standard_normal((6, 128))
    k = rng.standard_normal((300, 128))
    v = rng.standard_normal((300, 128))
    po, pl = R.split_attention(q, k, v, [0, 50, 50, 170, 300])
    out, lse = ops.lse_merge(torch.tensor(po, dtype=torch.float32, device=DEV),
                             torch.tensor(pl, dtype=torch.float32, device=DEV), with_lse=True,
                             dtype=BF16)
    exp_o, exp_l = R.lse_merge(po, pl)
    close_bf16(out, exp_o, "bf16 lse merge")
    np.testing.assert_allclose(lse.cpu().numpy(), exp_l, atol=1e-4)


def test_bf16_unsupported_forms_are_refused():
    """Mixed dtypes are refused before any launch."""
    w = to_bf16(workloads.c1_workload()).to(DEV)
    with pytest.raises(ValueError, match="pools' dtype"):
        ops.paged_decode(w.q.half(), w.k_pool, w.v_pool, w.block_tables, w.context_lens)
    with pytest.raises(ValueError, match="same"):
        ops.paged_decode(w.q, w.k_pool, w.v_pool.half(), w.block_tables, w.context_lens)


def test_bf16_page_writes_and_gather_are_byte_copies():
    """fe_write_kv, fe_write_kv_decode and fe_gather_kv move 16-bit words: with bf16 pools
    they are bit-exact against the oracle's copies of the int16 bits; a new-row dtype that
    differs from the pools' is refused."""
    g = torch.Generator().manual_seed(505)
    nb, bs, h, d, b = 48, 16, 2, 128, 5
    kp = torch.randn(nb, bs, h, d, generator=g).to(BF16)
    vp = torch.randn(nb, bs, h, d, generator=g).to(BF16)
    tables = torch.randperm(nb, generator=g)[: b * 8].view(b, 8).to(torch.int32)
    ctx = torch.tensor([1, 0, 16, 17, 128], dtype=torch.int32)
    kn = torch.randn(b, h, d, generator=g).to(BF16)
    vn = torch.randn(b, h, d, generator=g).to(BF16)
    ek, ev = kp.view(torch.int16).numpy().copy(), vp.view(torch.int16).numpy().copy()
    R.write_kv_decode(ek, ev, tables.numpy(), ctx.numpy(), kn.view(torch.int16).numpy(),
                      vn.view(torch.int16).numpy(), bs)
    kd, vd = kp.to(DEV), vp.to(DEV)
    ops.write_kv_decode(kn.to(DEV), vn.to(DEV), kd, vd, tables.to(DEV), ctx.to(DEV))
    torch.cuda.synchronize()
    assert kd.cpu().view(torch.int16).numpy().tobytes() == ek.tobytes()
    assert vd.cpu().view(torch.int16).numpy().tobytes() == ev.tobytes()
    # slot writes of 3 rows, then the gather of every row of sequence 3
    rows_k = torch.randn(3, h, d, generator=g).to(BF16)
    blocks = tables[3, :1].repeat(3)
    offs = torch.tensor([2, 3, 4], dtype=torch.int32)
    ops.write_kv(rows_k.to(DEV), rows_k.to(DEV), kd, vd, blocks.to(DEV), offs.to(DEV))
    R.write_kv(ek, ev, tables[3].tolist(), 2, rows_k.view(torch.int16).numpy(),
               rows_k.view(torch.int16).numpy(), bs)
    n = int(ctx[3])
    ko, vo = ops.gather_kv(kd, vd, tables[3:4].to(DEV), ctx[3:4].to(DEV),
                           torch.tensor([0, n], dtype=torch.int32, device=DEV), n)
    torch.cuda.synchronize()
    assert ko.dtype == BF16
    assert ko.cpu().view(torch.int16).numpy().tobytes() == \
        R.materialize(ek, tables[3].tolist(), n, bs).tobytes()
    assert vo.cpu().view(torch.int16).numpy().tobytes() == \
        R.materialize(ev, tables[3].tolist(), n, bs).tobytes()
    with pytest.raises(ValueError, match="wrong KV dtype"):
        ops.write_kv_decode(kn.half().to(DEV), vn.half().to(DEV), kd, vd, tables.to(DEV),
                            ctx.to(DEV))
