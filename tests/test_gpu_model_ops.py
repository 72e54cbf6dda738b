"""GPU: the decoder-layer kernels (include/flexengine_amd_model.h) against
plain PyTorch restatements of the ops they fuse (fp16 element-wise semantics)
and an fp32 matrix product for the skinny GEMM, including ragged sizes."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from flexengine_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def randn(*shape, seed=0, scale=1.0):
    return (torch.randn(shape, generator=gen(seed), device=DEV) * scale).half()


def torch_rmsnorm(x, w, eps, residual=None):
    r = x if residual is None else x + residual  # fp16 add
    f = r.float()
    return w * (f * torch.rsqrt(f.square().mean(-1, keepdim=True) + eps)).half(), r


def ulps(a, b):
    """max difference in fp16 units in the last place of b."""
    d = (a.float() - b.float()).abs()
    ulp = torch.where(b.float().abs() < 6.1e-5, torch.full_like(d, 6e-8),
                      2.0 ** (torch.floor(torch.log2(b.float().abs().clamp_min(6.1e-5))) - 10))
    return (d / ulp).max().item()


@pytest.mark.parametrize("rows,hidden", [(1, 1536), (5, 1536), (64, 896), (3, 8192)])
def test_rmsnorm_matches_torch(rows, hidden):
    """The sum of squares adds in another order than PyTorch's, so fp16(r * rsqrt(..))
    can round one ulp apart for a rare element, which the weight multiply scales by |w|
    (here N(0, 1)): at most 2 ulps, nearly all elements bit-identical."""
    x, res, w = randn(rows, hidden, seed=1), randn(rows, hidden, seed=2), randn(hidden, seed=3)
    out, _ = ops.rmsnorm(x, w, 1e-6)
    want, _ = torch_rmsnorm(x, w, 1e-6)
    assert ulps(out, want) <= 2 and (out == want).float().mean() > 0.999
    r = res.clone()
    out, r2 = ops.rmsnorm(x, w, 1e-6, residual=r)
    want, want_r = torch_rmsnorm(x, w, 1e-6, residual=res)
    assert r2 is r and torch.equal(r, want_r)          # residual add is bit-exact
    assert ulps(out, want) <= 2 and (out == want).float().mean() > 0.999


def test_rmsnorm_reads_skinny_partials():
    x, w_lin, w = randn(7, 256, seed=4), randn(1536, 256, seed=5, scale=0.1), randn(1536, seed=6)
    res = randn(7, 1536, seed=7)
    part = ops.gemm_skinny(x, w_lin)
    o16 = part.sum(0).half()
    r = res.clone()
    out, _ = ops.rmsnorm(part, w, 1e-6, residual=r)
    want, want_r = torch_rmsnorm(o16, w, 1e-6, residual=res)
    assert ulps(r, want_r) <= 1 and ulps(out, want) <= 2


def emulated_rope(x16, positions, inv_freq):
    """RoPE of fp16 rows x16 [rows, H, D] with the kernel's rounding sequence, on the
    CPU: angle = fp32(pos * inv_freq); c, s = fp16 of the correctly rounded cos/sin
    (float64); each product and sum rounded to fp16."""
    x = x16.cpu().float()
    half = x.shape[-1] // 2
    ang = positions.cpu().float()[:, None] * inv_freq.cpu()[None, :]        # fp32 product
    c = ang.double().cos().half().float()[:, None, :]
    s = ang.double().sin().half().float()[:, None, :]
    a, b = x[..., :half], x[..., half:]
    r16 = lambda t: t.half().float()
    o1 = r16(r16(a * c) + r16(-b * s))
    o2 = r16(r16(b * c) + r16(a * s))
    bound = 2.0 ** (torch.floor(torch.log2((a.abs() + b.abs()).clamp_min(2 ** -14))) - 9)
    return torch.cat([o1, o2], -1), torch.cat([bound, bound], -1)


@pytest.mark.parametrize("rows,hq,hkv,d", [(1, 12, 2, 128), (9, 14, 2, 64), (33, 4, 4, 128)])
def test_rope_qkv_matches_emulated_rounding(rows, hq, hkv, d):
    qkv = randn(rows, (hq + 2 * hkv) * d, seed=8)
    positions = torch.randint(0, 40000, (rows,), generator=gen(9), device=DEV)
    positions[0] = 0
    inv_freq = 1.0 / 1e6 ** (torch.arange(0, d, 2, device=DEV, dtype=torch.float32) / d)
    q, k, v = ops.rope_qkv(qkv, positions, inv_freq, hq, hkv, d)
    for got, src in ((q, qkv[:, :hq * d].view(rows, hq, d)),
                     (k, qkv[:, hq * d:(hq + hkv) * d].view(rows, hkv, d))):
        want, bound = emulated_rope(src, positions, inv_freq)
        err = (got.cpu().float() - want).abs()
        # exact but for a cos/sin whose fp16 rounding flips: 2 ulps of |x1| + |x2|
        assert (err <= bound).all()
        assert (err == 0).float().mean() > 0.99
    assert torch.equal(v, qkv[:, (hq + hkv) * d:].reshape(rows, hkv, d))
    # position 0 is the identity
    assert torch.equal(q[0], qkv[0, :hq * d].view(hq, d))


def test_rope_qkv_from_partials_adds_bias():
    rows, hq, hkv, d, hidden = 4, 12, 2, 128, 512
    h, w = randn(rows, hidden, seed=10), randn((hq + 2 * hkv) * d, hidden, seed=11, scale=0.05)
    bias = randn((hq + 2 * hkv) * d, seed=12)
    positions = torch.tensor([0, 1, 511, 4095], device=DEV)
    inv_freq = 1.0 / 1e6 ** (torch.arange(0, d, 2, device=DEV, dtype=torch.float32) / d)
    q, k, v = ops.rope_qkv(ops.gemm_skinny(h, w), positions, inv_freq, hq, hkv, d, bias=bias)
    qkv = (h.float() @ w.float().t() + bias.float()).half()   # one rounding, like a library GEMM
    q2, k2, v2 = ops.rope_qkv(qkv, positions, inv_freq, hq, hkv, d)
    # the fp32 sums differ only in order: inputs equal or one fp16 ulp apart
    for a, b in ((q, q2), (k, k2), (v, v2)):
        assert (a.float() - b.float()).abs().max() <= 2 ** -8 * (1 + b.float().abs().max())


@pytest.mark.parametrize("rows,inter", [(1, 8960), (16, 4864), (40, 128)])
def test_silu_mul_matches_torch(rows, inter):
    gu = randn(rows, 2 * inter, seed=13, scale=3.0)
    out = ops.silu_mul(gu)
    want = F.silu(gu[:, :inter]) * gu[:, inter:]
    assert ulps(out, want) <= 1


@pytest.mark.parametrize("m,n,k", [(1, 2048, 1536), (3, 1536, 8960), (8, 17920, 1536),
                                   (16, 1000, 96), (17, 300, 1536), (32, 151936, 1536)])
def test_gemm_skinny_matches_fp32_product(m, n, k):
    x, w = randn(m, k, seed=14), randn(n, k, seed=15, scale=0.05)
    part = ops.gemm_skinny(x, w)
    assert part.shape[1:] == (m, n)
    want = x.float() @ w.float().t()
    got = part.sum(0)
    err = (got - want).abs().max().item()
    assert err <= 1e-4 * (1 + want.abs().max().item()), err


def test_gemm_skinny_rejects_unsupported_shapes():
    from flexengine_amd._lib import FlexEngineAMDError
    with pytest.raises(FlexEngineAMDError):
        ops.gemm_skinny(randn(33, 64), randn(16, 64))
    with pytest.raises(FlexEngineAMDError):
        ops.gemm_skinny(randn(2, 40), randn(16, 40))
