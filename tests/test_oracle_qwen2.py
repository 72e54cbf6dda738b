"""CPU: pins oracle/qwen2_ref.py (the dense forward the GPU model tests compare
against) to an independent implementation, transformers' Qwen2ForCausalLM,
with the same random weights; a planted mistake in the oracle's RoPE must be
caught by the same comparison."""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from oracle import qwen2_ref

transformers = pytest.importorskip("transformers")


def hf_and_mirror(seed=3, hq=4, hkv=2, d=8, hidden=32, layers=2, vocab=64, inter=48, norms_random=True):
    torch.manual_seed(seed)
    cfg = transformers.Qwen2Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                                   num_hidden_layers=layers, num_attention_heads=hq,
                                   num_key_value_heads=hkv, head_dim=d, rope_theta=1e6,
                                   rms_norm_eps=1e-6, tie_word_embeddings=True,
                                   max_position_embeddings=256)
    hf = transformers.Qwen2ForCausalLM(cfg).double().eval()
    with torch.no_grad():
        for p in hf.parameters():
            p.normal_(0.0, 0.2)
        if not norms_random:
            for name, p in hf.named_parameters():
                if "norm" in name:
                    p.fill_(1.0)
    layers_w = []
    for layer in hf.model.layers:
        a = layer.self_attn
        layers_w.append(SimpleNamespace(
            input_norm=layer.input_layernorm.weight, post_norm=layer.post_attention_layernorm.weight,
            w_qkv=torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]),
            b_qkv=torch.cat([a.q_proj.bias, a.k_proj.bias, a.v_proj.bias]),
            w_o=a.o_proj.weight,
            w_gate_up=torch.cat([layer.mlp.gate_proj.weight, layer.mlp.up_proj.weight]),
            w_down=layer.mlp.down_proj.weight))
    mirror = SimpleNamespace(
        cfg=SimpleNamespace(rope_theta=1e6, rms_norm_eps=1e-6, intermediate_size=inter),
        nq=hq, nkv=hkv, dim=d, embed=hf.model.embed_tokens.weight, layer_weights=layers_w,
        final_norm=hf.model.norm.weight, lm_head=hf.lm_head.weight)
    return hf, mirror


@pytest.mark.parametrize("hq,hkv", [(4, 2), (4, 1), (6, 6)])
def test_dense_reference_matches_transformers_qwen2(hq, hkv):
    hf, mirror = hf_and_mirror(hq=hq, hkv=hkv, hidden=8 * hq)
    ids = [3, 17, 5, 42, 8, 8, 61, 0, 29, 11]
    with torch.no_grad():
        want = hf(torch.tensor([ids])).logits[0, -1]
    got = qwen2_ref.reference_logits(mirror, ids)
    # transformers builds its RoPE tables in float32: agreement to ~1e-7 relative
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-6)


def test_planted_rope_mistake_is_caught(monkeypatch):
    """A rotate_half without the sign flip (a plausible slip) must fail the comparison.
    (A uniform position offset would not: RoPE scores depend on i - j only.)"""
    hf, mirror = hf_and_mirror()
    ids = [3, 17, 5, 42, 8, 8, 61]
    with torch.no_grad():
        want = hf(torch.tensor([ids])).logits[0, -1]

    def no_sign(t):
        half = t.shape[-1] // 2
        return torch.cat((t[..., half:], t[..., :half]), -1)

    monkeypatch.setattr(qwen2_ref, "rotate_half", no_sign)
    got = qwen2_ref.reference_logits(mirror, ids)
    assert (got - want).abs().max() > 1e-3
