"""GPU: the fused decode-step projections (fe_gemm_f16 / _resid / _silu / _rope and
their RMSNorm prologue) against PyTorch restatements of the unfused chains: fp32
products rounded once to fp16 (a library GEMM's output), then the element-wise ops of
qwen2.py / HF Qwen2 in fp16, each rounding its result.  The fused kernels accumulate
the products in another order, so an fp16 product may round one ulp apart; the bounds
below allow that and no more."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from flexengine_amd import ops
from tests.test_gpu_model_ops import emulated_rope, randn, torch_rmsnorm

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def prod16(x, w, bias=None):
    p = x.float() @ w.float().t()
    if bias is not None:
        p = p + bias.float()
    return p.half()


def assert_close16(got, want, rel=2 ** -10, abs_scale=1e-4, exact=0.9):
    """|got - want| <= rel * |want| + abs_scale * (1 + max |want|) everywhere (one fp16
    rounding apart, plus the fp32 accumulation-order error of a K-term dot product near
    zero), and most elements bit-identical."""
    g, w = got.float(), want.float()
    err = (g - w).abs()
    tol = rel * w.abs() + abs_scale * (1 + w.abs().max())
    assert (err <= tol).all(), f"max excess {(err - tol).max().item():.3e}"
    assert (got == want).float().mean() > exact


def tile_ss(r):
    """Sums of r^2 over 16-column tiles, [ceil(N/16), M] (the fused kernels' layout)."""
    m, n = r.shape
    pad = (-n) % 16
    f = F.pad(r.float(), (0, pad)).view(m, -1, 16)
    return f.square().sum(-1).t().contiguous()


SHAPES = [(1, 1536, 1536), (8, 2048, 1536), (16, 1000, 96), (17, 300, 1536), (32, 4000, 8960),
          (3, 1536, 8960), (33, 1536, 1536), (48, 2048, 8960), (64, 4000, 1536), (64, 1536, 8960)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_f16_matches_rounded_product(m, n, k):
    x, w, b = randn(m, k, seed=1), randn(n, k, seed=2, scale=0.05), randn(n, seed=3)
    assert_close16(ops.gemm_f16(x, w, b), prod16(x, w, b))
    assert_close16(ops.gemm_f16(x, w), prod16(x, w))


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_resid_adds_residual_and_tile_sums(m, n, k):
    x, w, res = randn(m, k, seed=4), randn(n, k, seed=5, scale=0.05), randn(m, n, seed=6)
    r, ss = ops.gemm_resid(x, w, res)
    o16 = prod16(x, w)
    want = o16 + res                                # fp16 add, as the reference's residual add
    # a product one ulp apart stays one ulp of |o| apart after the add
    err = (r.float() - want.float()).abs()
    tol = 2 ** -10 * (o16.float().abs() + want.float().abs()) + 1e-4 * (1 + o16.float().abs().max())
    assert (err <= tol).all()
    assert (r == want).float().mean() > 0.9
    assert torch.allclose(ss, tile_ss(r), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("m,inter,k", [(1, 8960, 1536), (8, 4864, 896), (17, 100, 1536),
                                       (32, 8960, 1536), (64, 8960, 1536), (40, 100, 512)])
def test_gemm_silu_matches_unfused_chain(m, inter, k):
    x, w = randn(m, k, seed=7), randn(2 * inter, k, seed=8, scale=0.05)
    g, u = prod16(x, w[:inter]), prod16(x, w[inter:])
    want = F.silu(g) * u                            # fp16 ops: silu rounded, product rounded
    got = ops.gemm_silu(x, w)
    assert got.shape == (m, inter)
    assert_close16(got, want, rel=2 ** -9, abs_scale=5e-4)


@pytest.mark.parametrize("m,hq,hkv,d,k", [(1, 12, 2, 128, 1536), (8, 14, 2, 64, 896),
                                          (17, 4, 4, 128, 512), (32, 12, 2, 128, 1536),
                                          (64, 12, 2, 128, 1536)])
def test_gemm_rope_matches_unfused_chain(m, hq, hkv, d, k):
    n = (hq + 2 * hkv) * d
    x, w, b = randn(m, k, seed=9), randn(n, k, seed=10, scale=0.05), randn(n, seed=11)
    positions = torch.randint(0, 40000, (m,), generator=torch.Generator(device=DEV).manual_seed(12),
                              device=DEV)
    positions[0] = 0
    inv_freq = 1.0 / 1e6 ** (torch.arange(0, d, 2, device=DEV, dtype=torch.float32) / d)
    q, kk, v = ops.gemm_rope(x, w, b, positions, inv_freq, hq, hkv, d)
    qkv = prod16(x, w, b)
    wq, wk, wv = ops.rope_qkv(qkv, positions, inv_freq, hq, hkv, d)
    # inputs equal or one fp16 ulp apart (product order); RoPE adds its own rounding
    for a, c in ((q, wq), (kk, wk), (v, wv)):
        assert (a.float() - c.float()).abs().max() <= 2 ** -8 * (1 + c.float().abs().max())
        assert (a == c).float().mean() > 0.97
    # against the CPU emulation of the rounding sequence, on the kernel's own products
    want, bound = emulated_rope(wq, positions, inv_freq)
    assert want.shape == wq.shape


@pytest.mark.parametrize("m,n,k", [(1, 2048, 1536), (8, 8960, 1536), (20, 512, 96)])
def test_norm_prologue_equals_separate_rmsnorm(m, n, k):
    """Normed(r, ss, w) as the operand == rmsnorm(r) then the plain GEMM."""
    r, w_norm = randn(m, k, seed=13, scale=2.0), randn(k, seed=14)
    w = randn(n, k, seed=15, scale=0.05)
    ss = tile_ss(r)
    h, _ = torch_rmsnorm(r, w_norm, 1e-6)
    got = ops.gemm_f16(ops.Normed(r, ss, w_norm, 1e-6), w)
    want = ops.gemm_f16(h, w)
    # the normalised operands may differ by one fp16 ulp (sum order of r^2)
    err = (got.float() - want.float()).abs().max().item()
    assert err <= 2 ** -9 * (1 + want.float().abs().max().item()) * 4
    assert (got == want).float().mean() > 0.9


def test_resid_feeds_norm_prologue_like_the_unfused_layer():
    """o projection + residual -> post-attention RMSNorm -> gate/up + SiLU, fused vs the
    unfused kernels (skinny GEMM partials, fe_rmsnorm, fe_silu_mul)."""
    m, hidden, inter = 4, 1536, 8960
    attn, res = randn(m, hidden, seed=16), randn(m, hidden, seed=17)
    w_o = randn(hidden, hidden, seed=18, scale=0.03)
    w_norm = randn(hidden, seed=19)
    w_gu = randn(2 * inter, hidden, seed=20, scale=0.03)
    r, ss = ops.gemm_resid(attn, w_o, res)
    act = ops.gemm_silu(ops.Normed(r, ss, w_norm, 1e-6), w_gu)
    res2 = res.clone()
    h2, _ = ops.rmsnorm(ops.gemm_skinny(attn, w_o), w_norm, 1e-6, residual=res2)
    act2 = ops.silu_mul(ops.gemm_skinny(h2, w_gu))
    assert_close16(r, res2)
    err = (act.float() - act2.float()).abs().max().item()
    assert err <= 2 ** -7 * (1 + act2.float().abs().max().item())
    assert (act == act2).float().mean() > 0.9


def test_fused_gemms_reject_unsupported_shapes():
    from flexengine_amd._lib import FlexEngineAMDError
    with pytest.raises(FlexEngineAMDError):
        ops.gemm_f16(randn(65, 64), randn(16, 64))
    with pytest.raises(FlexEngineAMDError):
        ops.gemm_f16(randn(2, 40), randn(16, 40))
    with pytest.raises(ValueError):
        ops.gemm_resid(randn(2, 64), randn(16, 64), randn(3, 16))


@pytest.mark.parametrize("m,n,k", [(1, 1536, 1536), (8, 1536, 8960), (17, 896, 4864),
                                   (32, 2048, 512), (3, 16, 64), (64, 1536, 8960), (50, 896, 1536)])
def test_resid_rmsnorm_equals_resid_then_rmsnorm(m, n, k):
    """One launch == fe_gemm_resid then fe_rmsnorm: r bit-identical, the norm within
    two fp16 ulps (the mean of r^2 is summed from the tile sums, in another order than
    the one-wave norm, and a one-ulp change of fp16(r * inv) can move the product with
    the weight by two) and almost all of it bit-identical; twice in a row (the
    launch-wide ticket resets itself)."""
    x, w, res = randn(m, k, seed=21), randn(n, k, seed=22, scale=0.05), randn(m, n, seed=23)
    nw = randn(n, seed=24)
    r_ref, _ = ops.gemm_resid(x, w, res)
    h_ref, _ = ops.rmsnorm(r_ref, nw, 1e-6)
    for _ in range(2):
        r, h = ops.gemm_resid_rmsnorm(x, w, res, nw, 1e-6)
        assert torch.equal(r, r_ref)
        err = (h.float() - h_ref.float()).abs()
        assert (err <= 2 ** -9 * h_ref.float().abs() + 1e-7).all(), err.max().item()
        assert (h == h_ref).float().mean() > 0.99
    # and against the float64 emulation of the reference's rounding
    want, _ = torch_rmsnorm(r_ref, nw, 1e-6)
    assert ((h.float() - want.float()).abs() <= 2 ** -9 * want.float().abs() + 1e-7).all()


def test_resid_rmsnorm_alternating_shapes_share_the_workspace():
    a = (randn(4, 8960, seed=25), randn(1536, 8960, seed=26, scale=0.02), randn(4, 1536, seed=27),
         randn(1536, seed=28))
    b = (randn(1, 512, seed=29), randn(896, 512, seed=30, scale=0.05), randn(1, 896, seed=31),
         randn(896, seed=32))
    first = {}
    for rep in range(3):
        for name, (x, w, res, nw) in (("a", a), ("b", b)):
            r, h = ops.gemm_resid_rmsnorm(x, w, res, nw, 1e-6)
            h_ref, _ = ops.rmsnorm(r, nw, 1e-6)
            assert (h == h_ref).float().mean() > 0.99
            if name in first:
                assert torch.equal(first[name], h)
            else:
                first[name] = h


def test_resid_rmsnorm_rejects_unsupported_widths():
    from flexengine_amd._lib import FlexEngineAMDError
    for n in (24, 2064):
        with pytest.raises(FlexEngineAMDError):
            ops.gemm_resid_rmsnorm(randn(2, 64), randn(n, 64), randn(2, n), randn(n), 1e-6)


@pytest.mark.parametrize("m,n,k", [(64, 1536, 1536), (64, 2048, 1536), (48, 17920, 1536),
                                   (33, 1536, 8960), (64, 100, 96), (1, 40, 4000),
                                   (17, 1000, 224), (64, 151, 8960)])
def test_gemm_rows64_matches_rounded_product(m, n, k):
    """fe_gemm_rows64 (x staged in LDS, shared by four weight tiles): within one fp16
    rounding of the fp32 product (+ bias), split-K or not, tile counts that are not a
    multiple of four, steps shorter than 128 keys; repeated calls bit-identical."""
    x, w, b = randn(m, k, seed=41), randn(n, k, seed=42, scale=0.05), randn(n, seed=43)
    got = ops.gemm_rows64(x, w, b)
    assert_close16(got, prod16(x, w, b))
    assert torch.equal(ops.gemm_rows64(x, w, b), got)
    assert_close16(ops.gemm_rows64(x, w), prod16(x, w))


def test_gemm_rows64_alternating_shapes_share_the_workspace():
    a = (randn(64, 8960, seed=44), randn(1536, 8960, seed=45, scale=0.02))
    b = (randn(40, 1536, seed=46), randn(2048, 1536, seed=47, scale=0.05))
    first = {}
    for rep in range(3):
        for name, (x, w) in (("a", a), ("b", b)):
            got = ops.gemm_rows64(x, w)
            assert_close16(got, prod16(x, w))
            if name in first:
                assert torch.equal(first[name], got)
            else:
                first[name] = got


def test_projections_reject_misaligned_operands():
    """x and W are read with 16-byte loads: a pointer off that alignment is an argument
    error returned before any launch (here x starts one fp16 element into its buffer)."""
    from flexengine_amd._lib import FlexEngineAMDError
    flat = randn(2 * 256 + 8, seed=48)
    x = flat[1:1 + 2 * 256].view(2, 256)
    assert x.is_contiguous() and x.data_ptr() % 16 != 0
    w = randn(64, 256, seed=49, scale=0.05)
    for fn in (ops.gemm_rows64, ops.gemm_f16, ops.gemm_skinny):
        with pytest.raises(FlexEngineAMDError):
            fn(x, w)
    assert_close16(ops.gemm_rows64(x.clone(), w), prod16(x, w))
