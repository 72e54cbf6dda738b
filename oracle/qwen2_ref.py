"""Independent dense forward of flexengine_amd.model.Qwen2Model's network.

TEST INFRASTRUCTURE ONLY: imported by tests/ (never by the package).  A
float64 CPU restatement of one sequence's causal forward -- embedding,
RMSNorm, q/k/v projections with bias, RoPE (rotate_half with
inv_freq = theta^(-2i/D), src/flexengine/inference/models/qwen2.py:15-17,46,
73-77), GQA by repeat_interleave (q head h uses kv head h // G), softmax
attention with the causal mask t <= i, o_proj, SiLU-gated MLP, final norm and
the (tied) LM head -- with no paging and no HIP kernel, in the style of the
reference's independent_reference (tests/unit/test_synthetic_qwen.py:58-87).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def rotate_half(t: torch.Tensor) -> torch.Tensor:
    """qwen2.py:15-17: (x1, x2) -> (-x2, x1) over the two halves of the last dim."""
    half = t.shape[-1] // 2
    return torch.cat((-t[..., half:], t[..., :half]), -1)


def reference_logits(model, ids: list[int]) -> torch.Tensor:
    """Last-token logits [vocab] (float64, CPU) of the token sequence `ids`
    at positions 0..len(ids)-1."""
    cfg = model.cfg
    nq, nkv, dim = model.nq, model.nkv, model.dim
    f64 = torch.float64

    def w(t):
        return t.detach().to("cpu", f64)

    n = len(ids)
    x = w(model.embed)[torch.tensor(ids)]
    pos = torch.arange(n, dtype=f64)
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, dim, 2, dtype=f64) / dim))
    ang = torch.outer(pos, inv)
    cos, sin = torch.cat((ang, ang), -1).cos()[:, None], torch.cat((ang, ang), -1).sin()[:, None]

    def rope(t):
        return t * cos + rotate_half(t) * sin

    def norm(t, weight):
        return w(weight) * (t * torch.rsqrt(t.square().mean(-1, keepdim=True) + cfg.rms_norm_eps))

    mask = torch.ones((n, n), dtype=torch.bool).tril()
    inter = cfg.intermediate_size
    for lw in model.layer_weights:
        h = norm(x, lw.input_norm)
        qkv = h @ w(lw.w_qkv).t() + w(lw.b_qkv)
        q = rope(qkv[:, :nq * dim].reshape(n, nq, dim))
        k = rope(qkv[:, nq * dim:(nq + nkv) * dim].reshape(n, nkv, dim))
        v = qkv[:, (nq + nkv) * dim:].reshape(n, nkv, dim)
        k = k.repeat_interleave(nq // nkv, 1)
        v = v.repeat_interleave(nq // nkv, 1)
        s = torch.einsum("qhd,khd->hqk", q, k) / math.sqrt(dim)
        p = torch.softmax(s.masked_fill(~mask, float("-inf")), -1)
        o = torch.einsum("hqk,khd->qhd", p, v).reshape(n, nq * dim)
        x = x + o @ w(lw.w_o).t()
        gu = norm(x, lw.post_norm) @ w(lw.w_gate_up).t()
        x = x + (F.silu(gu[:, :inter]) * gu[:, inter:]) @ w(lw.w_down).t()
    return (norm(x[-1:], model.final_norm) @ w(model.lm_head).t())[0]
