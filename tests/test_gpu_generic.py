"""GPU: head dims other than 64 / 128 and decode groups of 17-128 query heads per KV
head -- the generic attention kernel; at head_dim 256 in 16 bits the matrix-core
decode (groups <= 16) and prefill instantiated at 256; and groups above 16 with a
divisor in 8..16 (24, 32, 48, 64 below) split into virtual KV heads on the matrix-core
decode; and 16-bit decodes at other multiples of 8 below 256 over pages of 16k
tokens, on the matrix-core decode padded to the next of 64 / 128 / 256 (fp32 up to 64
and from 96 to 120 at any block size, on the fp32 engine padded to 64 / 128; the
prefills alike, fp32 at every multiple of 8 below 128)
-- against the oracle, in fp16, bf16 and fp32.  (The matrix-core prefill takes any group size: the group-24 / 32 cases at
head_dim 64 / 128 below run there.)

The reference's Triton decode takes any head_dim (BLOCK_D = next_power_of_2
with a dim mask, inference/kernels/paged_attention.py:106,112,152), and its
synthetic-model test runs head_dim 8 over a float32 cache of 4-token blocks
(tests/unit/test_synthetic_qwen.py:55,91: CacheLayout(2, 40, 4, 2, 8), 4 query
heads over 2 KV heads).  Those shapes reach fe_paged_decode / fe_prefill_paged
(and their _bf16 / _f32 forms) and run on the generic kernel; the decode's
fused page write is bit-exact as everywhere else.

Tolerances: fp16 the hot-path contract (max 2e-3, mean 2e-4), bf16 that scaled
by the bf16 / fp16 unit-roundoff ratio (2^-8 / 2^-11), fp32 max 2e-5, mean 2e-6
(the kernel accumulates in fp32: at most 512 sequential products per score and
64 keys per chunk between rescales).
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
FP16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32
TOL = {
    FP16: (MAX_ABS_TOL, MEAN_ABS_TOL),
    BF16: (MAX_ABS_TOL * 8.0, MEAN_ABS_TOL * 8.0),
    F32: (2e-5, 2e-6),
}

# (head_dim, Hq, Hkv, block size, dtype)
SHAPES = [
    (8, 4, 2, 4, F32),      # the reference's synthetic model
    (8, 4, 2, 4, FP16),
    (32, 8, 2, 16, FP16),
    (40, 10, 5, 8, BF16),
    (80, 12, 2, 16, FP16),
    (96, 12, 2, 16, BF16),
    (96, 12, 4, 32, F32),
    (256, 8, 1, 16, FP16),   # 16-bit D 256, groups <= 16: the matrix-core decode
    (256, 12, 2, 8, BF16),
    (256, 32, 2, 32, FP16),
    (256, 16, 2, 32, F32),
    (512, 4, 1, 16, FP16),
    (64, 32, 1, 16, FP16),   # group 32: past the matrix-core kernels' 16
    (128, 32, 1, 16, BF16),
    (128, 24, 1, 8, F32),
    (64, 71, 1, 16, FP16),   # 71 query heads over one KV head
    (128, 48, 1, 16, BF16),  # 48 over one
    (128, 64, 1, 32, F32),   # group 64 x 128: the generic kernel's largest item
    (112, 16, 2, 16, BF16),  # multiples of 8 in 16 bits, pages of 16k tokens: the
    (192, 8, 1, 32, FP16),   # matrix-core decode padded to 64 / 128 / 256
    (48, 8, 8, 16, FP16),
    (160, 20, 4, 64, BF16),
    (96, 32, 1, 16, FP16),   # padded, and group 32 as two virtual KV heads
    (24, 4, 4, 16, FP16),
    (8, 4, 2, 16, BF16),
    (48, 8, 2, 16, F32),     # fp32 multiples of 8 up to 64, and 96 / 104 / 112: the
    (112, 16, 4, 8, F32),    # fp32 engine padded to 64 / 128 at any block size (the
    (40, 32, 1, 16, F32),    # synthetic model's D 8 above too); group 32 as two
    (80, 8, 2, 16, F32),     # virtual heads; D 80 stays on the generic kernel
    (36, 6, 2, 16, FP16),    # head dims off the 16-byte vector: element loads
    (6, 4, 1, 4, F32),
    (20, 4, 2, 32, BF16),
]


def _ids(s):
    d, hq, hkv, bs, dt = s
    return f"d{d}-{hq}x{hkv}-bs{bs}-{str(dt).split('.')[-1]}"


def _draw(gen: torch.Generator, shape, dtype) -> torch.Tensor:
    return torch.randn(shape, generator=gen, dtype=F32).to(dtype)


def _np64(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy().astype(np.float64)


def _close(got: torch.Tensor, exp: np.ndarray, dtype, what: str):
    mx_tol, mean_tol = TOL[dtype]
    assert got.dtype == dtype, got.dtype
    mx, mean = assert_attention_close(_np64(got.cpu()), exp, mx_tol, mean_tol, what)
    print(f"{what}: max abs {mx:.3e} mean abs {mean:.3e}", flush=True)


def _decode_workload(shape, seed, lengths):
    d, hq, hkv, bs, dt = shape
    w = workloads.make_decode_workload(f"generic-{_ids(shape)}", seed, len(lengths), hq, hkv, d,
                                       lengths, block_size=bs, with_new_kv=True)
    g = torch.Generator().manual_seed(seed + 1)
    cv = (lambda t: None if t is None else _draw(g, t.shape, F32)) if dt == F32 else \
        (lambda t: None if t is None else t.float().to(dt))
    return workloads.DecodeWorkload(w.name, cv(w.q), cv(w.k_pool), cv(w.v_pool), w.block_tables,
                                    w.context_lens, cv(w.k_new), cv(w.v_new), w.unique_tokens,
                                    dict(w.meta))


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int32 if t.dtype == F32 else torch.int16).numpy().copy()


def _oracle_decode(w: workloads.DecodeWorkload):
    """float64 decode after the page write; the pools after the write as raw bits."""
    dt = w.q.dtype
    kp, vp = _bits(w.k_pool), _bits(w.v_pool)
    R.write_kv_decode(kp, vp, w.block_tables.numpy(), w.context_lens.numpy(), _bits(w.k_new),
                      _bits(w.v_new), w.block_size)
    kf = _np64(torch.from_numpy(kp).view(dt))
    vf = _np64(torch.from_numpy(vp).view(dt))
    out = R.decode_reference(_np64(w.q), kf, vf, w.block_tables.numpy(), w.context_lens.numpy(),
                             w.block_size)
    return out, kp, vp


LENGTHS = [0, 1, 3, 4, 5, 17, 63, 64, 65, 200, 257, 1000, 0, 2100]


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_generic_decode_matches_oracle_with_page_write(shape):
    w = _decode_workload(shape, 700 + shape[0] + shape[1], LENGTHS)
    print(f"generic decode {w.name}", flush=True)
    d = w.to(DEV)
    out = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                           k_new=d.k_new, v_new=d.v_new)
    torch.cuda.synchronize()
    exp, kp, vp = _oracle_decode(w)
    _close(out, exp, shape[4], w.name)
    for b in (w.context_lens == 0).nonzero().flatten().tolist():
        assert torch.count_nonzero(out[b]) == 0, f"inactive row {b}"
    assert (_bits(d.k_pool.cpu()) == kp).all(), "page write (K)"
    assert (_bits(d.v_pool.cpu()) == vp).all(), "page write (V)"


@pytest.mark.parametrize("shape", [SHAPES[0], SHAPES[5], SHAPES[8], SHAPES[13], SHAPES[-1]],
                         ids=_ids)
def test_generic_decode_without_page_write_is_repeatable(shape):
    """Without new rows the pools are untouched, and repeated calls are bit-identical
    (no atomics, a fixed reduction order)."""
    w = _decode_workload(shape, 760 + shape[0], [1, 90, 4096, 7, 333])
    w = workloads.DecodeWorkload(w.name, w.q, w.k_pool, w.v_pool, w.block_tables,
                                 w.context_lens, None, None, w.unique_tokens, w.meta)
    d = w.to(DEV)
    first = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens)
    again = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    dt = shape[4]
    exp = R.decode_reference(_np64(w.q), _np64(w.k_pool), _np64(w.v_pool), w.block_tables.numpy(),
                             w.context_lens.numpy(), w.block_size)
    _close(first, exp, dt, w.name)
    assert (_bits(d.k_pool.cpu()) == _bits(w.k_pool)).all()


def test_generic_and_matrix_core_decodes_share_one_workspace():
    """The per-device workspace starts with the split-K tickets the matrix-core decode
    needs at zero: generic decodes (whose key-split partials live past them) and
    matrix-core decodes alternating on one workspace both stay exact."""
    lens = [1, 90, 4096, 700, 33, 2000]
    wg = _decode_workload((96, 12, 2, 16, FP16), 790, lens)
    wm = _decode_workload((128, 12, 2, 16, FP16), 791, lens)
    need = max(ops.decode_workspace_bytes(len(lens), 12, d, 4096) for d in (96, 128))
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    exp_g = R.decode_reference(_np64(wg.q), _np64(wg.k_pool), _np64(wg.v_pool),
                               wg.block_tables.numpy(), wg.context_lens.numpy(), 16)
    exp_m = R.decode_reference(_np64(wm.q), _np64(wm.k_pool), _np64(wm.v_pool),
                               wm.block_tables.numpy(), wm.context_lens.numpy(), 16)
    dg, dm = wg.to(DEV), wm.to(DEV)
    for rep in range(3):
        og = ops.paged_decode(dg.q, dg.k_pool, dg.v_pool, dg.block_tables, dg.context_lens,
                              workspace=ws)
        om = ops.paged_decode(dm.q, dm.k_pool, dm.v_pool, dm.block_tables, dm.context_lens,
                              workspace=ws)
        torch.cuda.synchronize()
        _close(og, exp_g, FP16, f"generic, round {rep}")
        _close(om, exp_m, FP16, f"matrix-core, round {rep}")
    assert torch.count_nonzero(ws[:65536 * 4]) == 0, "split-K tickets left nonzero"


def test_generic_decode_replays_from_a_graph():
    """The generic decode (its split launch and merge launch, partials in the caller's
    workspace) captured in a HIP graph: three replays, with eager decodes of another
    shape on the same workspace between them, each bit-identical to the eager call."""
    lens = [1, 90, 4096, 700, 33, 2000]
    w = _decode_workload((96, 12, 2, 16, BF16), 795, lens)
    w = workloads.DecodeWorkload(w.name, w.q, w.k_pool, w.v_pool, w.block_tables,
                                 w.context_lens, None, None, w.unique_tokens, w.meta)
    other = _decode_workload((80, 8, 2, 16, BF16), 796, [17, 300, 1200])
    d, o = w.to(DEV), other.to(DEV)
    need = max(ops.decode_workspace_bytes(len(lens), 12, 96, 4096),
               ops.decode_workspace_bytes(3, 8, 80, o.block_tables.shape[1] * 16))
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(d.q)
    eager = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens,
                             workspace=ws).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens, out=out,
                         workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens, out=out,
                         workspace=ws)
    for rep in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        ops.paged_decode(o.q, o.k_pool, o.v_pool, o.block_tables, o.context_lens, workspace=ws)
        torch.cuda.synchronize()
    exp = R.decode_reference(_np64(w.q), _np64(w.k_pool), _np64(w.v_pool), w.block_tables.numpy(),
                             w.context_lens.numpy(), 16)
    _close(out, exp, BF16, "graph replay")


def test_generic_decode_strided_q_and_scale():
    """q rows with a batch stride wider than Hq * D (a fused qkv buffer's q slice) and an
    explicit scale."""
    d, hq, hkv, bs = 96, 6, 2, 16
    w = _decode_workload((d, hq, hkv, bs, FP16), 771, [5, 129, 40])
    qkv = torch.zeros(3, (hq + 2 * hkv) * d, dtype=FP16)
    qkv[:, :hq * d] = w.q.reshape(3, -1)
    q = qkv.to(DEV)[:, :hq * d].view(3, hq, d)
    dd = w.to(DEV)
    out = ops.paged_decode(q, dd.k_pool, dd.v_pool, dd.block_tables, dd.context_lens, scale=0.07)
    torch.cuda.synchronize()
    exp = R.decode_reference(_np64(w.q), _np64(w.k_pool), _np64(w.v_pool), w.block_tables.numpy(),
                             w.context_lens.numpy(), bs, scale=0.07)
    _close(out, exp, FP16, "strided q")


def _prefill_case(shape, seed, n_new, cached):
    d, hq, hkv, bs, dt = shape
    g = torch.Generator().manual_seed(seed)
    ctx = [c + n for c, n in zip(cached, n_new)]
    pages = [max(math.ceil(x / bs), 1) for x in ctx]
    nb = sum(pages) + 3
    k_pool = _draw(g, (nb, bs, hkv, d), dt)
    v_pool = _draw(g, (nb, bs, hkv, d), dt)
    perm = torch.randperm(nb, generator=g)
    width = max(pages)
    tables = torch.zeros(len(ctx), width, dtype=torch.int32)
    at = 0
    for i, p in enumerate(pages):
        tables[i, :p] = perm[at:at + p]
        tables[i, p:] = perm[at + p - 1]
        at += p
    offs = np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32)
    q = _draw(g, (int(offs[-1]), hq, d), dt)
    return q, torch.tensor(offs), torch.tensor(ctx, dtype=torch.int32), tables, k_pool, v_pool


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_generic_prefill_matches_oracle(shape):
    """Ragged chunks over cached context: a chunk from position 0, one after 999 cached
    keys, an empty chunk and a one-token chunk."""
    n_new, cached = [70, 5, 0, 1, 33], [0, 999, 12, 40, 7]
    q, offs, ctx, tables, kp, vp = _prefill_case(shape, 800 + shape[0] + shape[1], n_new, cached)
    out = ops.prefill_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), tables.to(DEV), offs.to(DEV),
                            ctx.to(DEV), max(n_new))
    torch.cuda.synchronize()
    exp = R.prefill_reference(_np64(q), offs.numpy(), ctx.numpy(), _np64(kp), _np64(vp),
                              tables.numpy(), shape[3])
    _close(out, exp, shape[4], f"prefill {_ids(shape)}")


@pytest.mark.parametrize("shape", [(256, 32, 4, 16, FP16), (160, 32, 4, 16, BF16),
                                   (96, 32, 4, 16, FP16)], ids=_ids)
def test_prefill_with_more_than_65536_rows_at_one_row_tile(shape):
    """2100 new tokens x 32 query heads = 67200 (token, head) rows, past the size at
    which the tile kernel's plan takes two row tiles per wave: at head_dim 256 (and
    dims padded to it) the kernel has one, and its grid is sized for that; at 96
    (padded to 128, 96 dims computed) the two-tile form runs."""
    n_new, cached = [2100, 3], [0, 50]
    q, offs, ctx, tables, kp, vp = _prefill_case(shape, 900 + shape[0], n_new, cached)
    out = ops.prefill_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), tables.to(DEV), offs.to(DEV),
                            ctx.to(DEV), max(n_new))
    torch.cuda.synchronize()
    exp = R.prefill_reference(_np64(q), offs.numpy(), ctx.numpy(), _np64(kp), _np64(vp),
                              tables.numpy(), shape[3])
    _close(out, exp, shape[4], f"prefill {_ids(shape)} 67200 rows")


@pytest.mark.parametrize("d,hq,hkv", [(96, 12, 2), (256, 8, 1), (128, 32, 1)])
def test_generic_shared_prefix_equals_plain_decode(d, hq, hkv):
    """fe_paged_decode_shared_prefix at shapes the shared-prefix kernels do not take
    (head_dim 96: the generic kernel; 256 and a group of 32: the piece kernel) attends
    every row over its own table (whose first pages are the shared ones): the same
    result as fe_paged_decode."""
    bs = 16
    g = torch.Generator().manual_seed(781 + d + hq)
    prefix, suffixes = 160, [1, 30, 77, 200]
    pre_pages = prefix // bs
    pages = [pre_pages + math.ceil(s / bs) for s in suffixes]
    nb = pre_pages + sum(p - pre_pages for p in pages) + 2
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    width = max(pages)
    tables = torch.zeros(len(suffixes), width, dtype=torch.int32)
    at = pre_pages
    for i, p in enumerate(pages):
        tables[i, :pre_pages] = perm[:pre_pages]
        tables[i, pre_pages:p] = perm[at:at + p - pre_pages]
        tables[i, p:] = tables[i, p - 1]
        at += p - pre_pages
    ctx = torch.tensor([prefix + s for s in suffixes], dtype=torch.int32)
    q = _draw(g, (len(suffixes), hq, d), FP16)
    kp = _draw(g, (nb, bs, hkv, d), FP16)
    vp = _draw(g, (nb, bs, hkv, d), FP16)
    offs = torch.tensor([0, len(suffixes)], dtype=torch.int32, device=DEV)
    plens = torch.tensor([prefix], dtype=torch.int32, device=DEV)
    qd, kd, vd, td, cd = (t.to(DEV) for t in (q, kp, vp, tables, ctx))
    shared = ops.paged_decode_shared_prefix(qd, kd, vd, td, cd, offs, plens)
    plain = ops.paged_decode(qd, kd, vd, td, cd)
    torch.cuda.synchronize()
    assert torch.equal(shared, plain)
    exp = R.decode_reference(_np64(q), _np64(kp), _np64(vp), tables.numpy(), ctx.numpy(), bs)
    _close(shared, exp, FP16, "shared prefix, generic shape")


def _dense_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos0: int) -> np.ndarray:
    """Dense causal attention in float64 with torch's SDPA (an independent routine): q
    [n, Hq, D] at positions pos0 .. pos0 + n - 1 over k, v [L, Hkv, D]."""
    hq, hkv = q.shape[1], k.shape[1]
    qq = q.double().transpose(0, 1)
    kk = k.double().repeat_interleave(hq // hkv, 1).transpose(0, 1).contiguous()
    vv = v.double().repeat_interleave(hq // hkv, 1).transpose(0, 1).contiguous()
    mask = torch.arange(k.shape[0])[None, :] <= (pos0 + torch.arange(q.shape[0]))[:, None]
    o = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask)
    return o.transpose(0, 1).numpy()


def test_reference_synthetic_cache_full_incremental_and_multi():
    """The reference synthetic test's attention, at its shapes: CacheLayout(2, 40, 4, 2,
    8) in float32, request "a" of 9 tokens and "b" of 4; full prefill of both, then
    "a" again in chunks of 3, 5 and 1 tokens (test_synthetic_qwen.py:88-104), through
    the attention backend interface, against dense causal attention."""
    gen = torch.Generator().manual_seed(19)
    cache = PagedKVCache(CacheLayout(2, 40, 4, 2, 8), device=DEV, dtype=F32)
    lens = {"a": 9, "b": 4}
    rows = {r: (_draw(gen, (n, 2, 8), F32), _draw(gen, (n, 2, 8), F32), _draw(gen, (n, 4, 8), F32))
            for r, n in lens.items()}
    for r, n in lens.items():
        cache.reserve(r, n)
    for layer in range(2):
        for r, n in lens.items():
            k, v, q = rows[r]
            cache.write(layer, r, 0, (k + layer).to(DEV), (v - layer).to(DEV))
    for layer in range(2):
        for r, n in lens.items():
            k, v, q = rows[r]
            got = attention.attention_for_request(q.to(DEV), cache, layer, r, n,
                                                  torch.arange(n, device=DEV))
            torch.cuda.synchronize()
            exp = _dense_causal(q, k + layer, v - layer, 0)
            _close(got, exp, F32, f"full {r} layer {layer}")
    # "a" again: free it, re-reserve, and feed the chunks as they are written
    cache.free_request("a")
    cache.reserve("a", lens["a"])
    k, v, q = rows["a"]
    for lo, hi in ((0, 3), (3, 8), (8, 9)):
        cache.write(0, "a", lo, k[lo:hi].to(DEV), v[lo:hi].to(DEV))
        got = attention.attention_for_request(q[lo:hi].to(DEV), cache, 0, "a", hi,
                                              torch.arange(lo, hi, device=DEV))
        torch.cuda.synchronize()
        exp = _dense_causal(q[lo:hi], k[:hi], v[:hi], lo)
        _close(got, exp, F32, f"chunk {lo}:{hi}")
    cache.assert_invariants()


def test_generic_shapes_outside_the_envelope_are_refused():
    q = torch.zeros(1, 2, 1024, dtype=FP16, device=DEV)  # head_dim 1024 > 512
    pool = torch.zeros(2, 16, 1, 1024, dtype=FP16, device=DEV)
    t = torch.zeros(1, 1, dtype=torch.int32, device=DEV)
    c = torch.ones(1, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported"):
        ops.paged_decode(q, pool, pool, t, c)
    q = torch.zeros(1, 67, 128, dtype=FP16, device=DEV)  # group 67 (prime) x 128 > 8192
    pool = torch.zeros(2, 16, 1, 128, dtype=FP16, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported"):
        ops.paged_decode(q, pool, pool, t, c)
    # the prefill kernels take any group size; head_dim 1024 is refused there too
    q = torch.zeros(1, 2, 1024, dtype=FP16, device=DEV)
    pool = torch.zeros(2, 16, 1, 1024, dtype=FP16, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported"):
        ops.prefill_paged(q, pool, pool, t, torch.tensor([0, 1], dtype=torch.int32, device=DEV),
                          c, 1)
    assert _lib.FE_ERR_UNSUPPORTED == -2
