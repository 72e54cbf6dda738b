"""GPU: KV page write and block-table gather are bit-exact against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from flexengine_amd import ops
from flexengine_amd.kv_cache import CacheLayout, PagedKVCache
from oracle import paged_ref as R

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy()


def test_write_kv_slots_bit_exact_and_untouched_rows():
    g = torch.Generator().manual_seed(11)
    nb, bs, h, d = 40, 16, 2, 128
    k_pool = torch.randn(nb, bs, h, d, generator=g).half()
    v_pool = torch.randn(nb, bs, h, d, generator=g).half()
    n = 45
    keys = torch.randn(n, h, d, generator=g).half()
    vals = torch.randn(n, h, d, generator=g).half()
    table = [31, 4, 17]
    start = 2
    ids, offs = R.locators(table, start, n, bs)
    exp_k, exp_v = k_pool.numpy().copy(), v_pool.numpy().copy()
    R.write_kv(exp_k, exp_v, table, start, keys.numpy(), vals.numpy(), bs)
    kd, vd = k_pool.to(DEV), v_pool.to(DEV)
    ops.write_kv(keys.to(DEV), vals.to(DEV), kd, vd,
                 torch.tensor(ids, dtype=torch.int32, device=DEV),
                 torch.tensor(offs, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert (_bits(kd) == exp_k.view(np.int16)).all()
    assert (_bits(vd) == exp_v.view(np.int16)).all()


def test_write_kv_skips_negative_slots_and_keeps_nan_payloads():
    nb, bs, h, d = 8, 4, 1, 64
    k_pool = torch.zeros(nb, bs, h, d, dtype=torch.float16, device=DEV)
    v_pool = torch.zeros_like(k_pool)
    keys = torch.full((3, h, d), float("nan"), dtype=torch.float16)
    keys.view(torch.int16)[1] = 0x7E01  # a NaN with a payload: must be copied as bytes
    keys[2] = 1.5
    vals = keys.clone()
    blocks = torch.tensor([5, -1, 2], dtype=torch.int32, device=DEV)
    offs = torch.tensor([3, 0, 1], dtype=torch.int32, device=DEV)
    ops.write_kv(keys.to(DEV), vals.to(DEV), k_pool, v_pool, blocks, offs)
    torch.cuda.synchronize()
    kp = _bits(k_pool)
    assert (kp[5, 3] == keys.view(torch.int16).numpy()[0]).all()
    assert (kp[2, 1] == keys.view(torch.int16).numpy()[2]).all()
    mask = np.ones(kp.shape[:2], dtype=bool)
    mask[5, 3] = mask[2, 1] = False
    assert (kp[mask] == 0).all(), "skipped / untouched slots must stay zero"


def test_write_kv_strided_source_rows():
    """k/v as views into a fused [T, (Hq+2Hkv)*D] projection (row stride > Hkv*D)."""
    g = torch.Generator().manual_seed(3)
    t, hq, hkv, d, bs, nb = 9, 6, 2, 64, 16, 4
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).half().to(DEV)
    k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    k_pool = torch.zeros(nb, bs, hkv, d, dtype=torch.float16, device=DEV)
    v_pool = torch.zeros_like(k_pool)
    ids, offs = R.locators([2, 0], 5, t, bs)
    ops.write_kv(k, v, k_pool, v_pool, torch.tensor(ids, dtype=torch.int32, device=DEV),
                 torch.tensor(offs, dtype=torch.int32, device=DEV))
    exp_k = np.zeros((nb, bs, hkv, d), dtype=np.float16)
    exp_v = exp_k.copy()
    R.write_kv(exp_k, exp_v, [2, 0], 5, k.cpu().numpy(), v.cpu().numpy(), bs)
    assert (_bits(k_pool) == exp_k.view(np.int16)).all()
    assert (_bits(v_pool) == exp_v.view(np.int16)).all()


@pytest.mark.parametrize("bs", [4, 16, 32])
def test_write_kv_decode_bit_exact(bs):
    g = torch.Generator().manual_seed(bs)
    nb, h, d, b = 64, 2, 128, 5
    k_pool = torch.randn(nb, bs, h, d, generator=g).half()
    v_pool = torch.randn(nb, bs, h, d, generator=g).half()
    perm = torch.randperm(nb, generator=g)
    width = 10
    tables = perm[: b * width].view(b, width).to(torch.int32)
    ctx = torch.tensor([1, 0, bs, bs + 1, width * bs], dtype=torch.int32)
    kn = torch.randn(b, h, d, generator=g).half()
    vn = torch.randn(b, h, d, generator=g).half()
    exp_k, exp_v = k_pool.numpy().copy(), v_pool.numpy().copy()
    R.write_kv_decode(exp_k, exp_v, tables.numpy(), ctx.numpy(), kn.numpy(), vn.numpy(), bs)
    kd, vd = k_pool.to(DEV), v_pool.to(DEV)
    ops.write_kv_decode(kn.to(DEV), vn.to(DEV), kd, vd, tables.to(DEV), ctx.to(DEV))
    assert (_bits(kd) == exp_k.view(np.int16)).all()
    assert (_bits(vd) == exp_v.view(np.int16)).all()


@pytest.mark.parametrize("bs", [2, 16])
def test_gather_bit_exact_reversed_tables(bs):
    g = torch.Generator().manual_seed(7 + bs)
    nb, h, d = 96, 2, 64
    k_pool = torch.randn(nb, bs, h, d, generator=g).half()
    v_pool = torch.randn(nb, bs, h, d, generator=g).half()
    lengths = [1, 17, 40, 0, 33]
    width = max((n + bs - 1) // bs for n in lengths)
    perm = torch.randperm(nb, generator=g)
    tables = torch.zeros(len(lengths), width, dtype=torch.int32)
    at = 0
    for i, n in enumerate(lengths):
        pages = (n + bs - 1) // bs
        row = perm[at:at + pages].flip(0)  # reversed tables, as test_triton_paged_attention.py:15
        at += pages
        tables[i, :pages] = row
    offs = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    total = int(offs[-1])
    ko, vo = ops.gather_kv(k_pool.to(DEV), v_pool.to(DEV), tables.to(DEV),
                           torch.tensor(lengths, dtype=torch.int32, device=DEV),
                           torch.tensor(offs, device=DEV), total)
    ko, vo = ko.cpu().numpy(), vo.cpu().numpy()
    for i, n in enumerate(lengths):
        if n == 0:
            continue
        ek = R.materialize(k_pool.numpy(), tables[i].tolist(), n, bs)
        ev = R.materialize(v_pool.numpy(), tables[i].tolist(), n, bs)
        assert ko[offs[i]:offs[i + 1]].tobytes() == ek.tobytes()
        assert vo[offs[i]:offs[i + 1]].tobytes() == ev.tobytes()


def test_paged_cache_write_materialize_roundtrip():
    """The reference's readback test (test_allocator.py:11-29) through the device cache."""
    c = PagedKVCache(CacheLayout(2, 10, 4, 2, 8), device=DEV, fill=0.0)
    c.reserve("a", 3)
    c.reserve("a", 5)
    c.reserve("b", 7)
    assert c.tables["a"] == [0, 1] and c.tables["b"] == [2, 3]
    a = torch.arange(5 * 2 * 8).reshape(5, 2, 8).half().to(DEV)
    c.write(0, "a", 0, a, a + 100)
    ka, va = c.materialize(0, "a", 5)
    assert torch.equal(ka, a) and torch.equal(va, a + 100)
    assert [len(k) for _, k, _ in c.iter_blocks(0, "a", 5)] == [4, 1]
    assert torch.count_nonzero(c.k[1]) == 0, "layer 1 untouched"
    c.assert_invariants()
    c.attach_prefix("p", [0])
    with pytest.raises(RuntimeError, match="shared immutable"):
        c.write(0, "a", 0, a[:1], a[:1])


# --------------------------------------------------------------------------------------
# device-side slot mapping of the ragged write and device-built block tables
# --------------------------------------------------------------------------------------

@pytest.mark.parametrize("bs,h,d", [(16, 2, 128), (1, 2, 64), (4, 1, 64), (32, 4, 128)])
def test_write_kv_ragged_matches_the_per_request_write(bs, h, d):
    """Chunks of 1..70 new tokens after 0..100 cached ones (crossing block edges),
    through fe_write_kv_ragged, byte-for-byte equal to the oracle's per-request
    write (allocator.py:107-127) into a pool with stale contents elsewhere."""
    g = torch.Generator().manual_seed(bs + h + d)
    news, cached = [1, 17, 70, 5, 33], [0, 100, 3, 16 * 3, 7]
    nb = sum(-(-(c + n) // bs) for c, n in zip(cached, news)) + 5
    perm = torch.randperm(nb, generator=g).tolist()
    tables, at = [], 0
    for c, n in zip(cached, news):
        p = -(-(c + n) // bs)
        tables.append(perm[at:at + p])
        at += p
    width = max(len(t) for t in tables)
    tab = torch.tensor([t + [t[-1]] * (width - len(t)) for t in tables], dtype=torch.int32)
    k_pool = torch.randn(nb, bs, h, d, generator=g).half()
    v_pool = torch.randn(nb, bs, h, d, generator=g).half()
    keys = torch.randn(sum(news), h, d, generator=g).half()
    vals = torch.randn(sum(news), h, d, generator=g).half()
    offs = np.concatenate([[0], np.cumsum(news)]).astype(np.int32)
    ctx = torch.tensor([c + n for c, n in zip(cached, news)], dtype=torch.int32)
    ek, ev = k_pool.numpy().copy(), v_pool.numpy().copy()
    for s, (c, n) in enumerate(zip(cached, news)):
        R.write_kv(ek, ev, tables[s], c, keys[offs[s]:offs[s + 1]].numpy(),
                   vals[offs[s]:offs[s + 1]].numpy(), bs)
    kd, vd = k_pool.to(DEV), v_pool.to(DEV)
    ops.write_kv_ragged(keys.to(DEV), vals.to(DEV), kd, vd, tab.to(DEV),
                        torch.tensor(offs).to(DEV), ctx.to(DEV))
    assert kd.cpu().numpy().tobytes() == ek.tobytes()
    assert vd.cpu().numpy().tobytes() == ev.tobytes()


def test_device_tables_follow_the_allocator():
    """The device mirror tracks reserve (growth past the mirror's first width),
    attach_prefix, free_request and the reuse of freed rows; device_tables equals
    the host-built block_table for every padding choice, and None rows are pads."""
    c = PagedKVCache(CacheLayout(1, 400, 4, 1, 8), device=DEV)
    c.reserve("a", 9)
    c.reserve("b", 1)
    c.reserve("c", 0)
    c.attach_prefix("p", c.tables["a"][:2])
    c.reserve("a", 4 * 90)                      # 90 blocks: wider than the initial mirror
    c.free_request("b")
    c.reserve("d", 20)                          # reuses b's mirror row
    c.reserve("p", 14)
    ids = ["a", "c", "p", "d"]
    width = max(len(c.tables[r]) for r in ids)
    for pad in (None, 7):
        want = c.block_table(ids, width, pad_block=pad)
        got = c.device_tables(ids, width, pad_block=pad)
        assert torch.equal(got, want), pad
    got = c.device_tables(["d", None, "p"], 100, pad_block=3)
    assert got[1].tolist() == [3] * 100
    assert got[0, :5].tolist() == c.tables["d"] and got[0, 5:].tolist() == [3] * 95
    c.tables["d"] = list(reversed(c.tables["d"]))   # a reorder re-copies the row itself
    assert c.device_tables(["d"])[0].tolist() == c.tables["d"]
    c.assert_invariants()                           # device tables == host tables
    with pytest.raises(ValueError):
        c.device_tables(["a"], 10)


def test_graph_inputs_pad_rows_with_a_scratch_block():
    """runtime.py:201-213: active rows carry token, position and table; padded rows
    and the table tails hold a scratch block."""
    from flexengine_amd.decode_step import SCRATCH_ID, GraphDecodeStep
    from flexengine_amd.model import Chunk
    cache = PagedKVCache(CacheLayout(1, 40, 4, 2, 8), device=DEV)
    cache.reserve("a", 6)
    step = GraphDecodeStep(model=None, cache=cache, max_model_len=16)
    assert len(cache.tables[SCRATCH_ID]) == 8 * 4 // 4
    inp = step.graph_inputs([Chunk("a", [42], 5)], 4)
    assert inp["input_ids"].tolist() == [42, 0, 0, 0]
    assert inp["positions"].tolist() == [5, 0, 0, 0]
    assert inp["block_tables"].dtype == torch.int32
    scratch = step.scratch_blocks[0]
    assert inp["block_tables"][0].tolist() == cache.tables["a"] + [scratch] * 2
    for row in range(1, 4):
        assert inp["block_tables"][row].tolist() == [scratch] * 4
    with pytest.raises(ValueError):
        step.graph_inputs([Chunk("a", [1], 0)] * 5, 4)
