"""A Qwen2 decoder that runs its attention on the HIP paged-attention kernels.

The caller side of the hot path: the two forwards of FlexEngine's
Qwen2Adapter (src/flexengine/inference/models/qwen2.py) with the same
semantics, on this package's kernels and random-initialised weights (there is
no network for checkpoints).

* forward(chunks, cache) -- the ragged mixed batch of qwen2.py:79-136: every
  chunk (request_id, input_ids, start) is a run of tokens at absolute
  positions start..start+n-1; per layer the new K/V rows are written to the
  paged pool *before* attention, and attention is causal per request.  All
  chunks' K/V go through one fe_write_kv_ragged launch and all chunks'
  attention through one fe_prefill_paged_planned launch (the reference loops
  over requests), whose work split one fe_prefill_plan launch per forward
  computes for every layer.
  Returns the last-token logits of each chunk.
* decode_static(input_ids, positions, block_tables, active_mask, cache) -- the
  graph-compatible one-token step of qwen2.py:138-186 over fixed padded batch
  tensors; one fe_paged_decode_plan launch per step (the split-K partition and
  block rows, the same for every layer), then per layer the page write of the
  new token and the attention in one fe_paged_decode_planned launch.  Inactive
  rows leave the pool untouched and give zero logits.

RoPE follows qwen2.py:15-17,46,73-77: inv_freq = theta^(-2i/D), the half-split
rotate_half, cos/sin cast to the activation dtype.  RMSNorm computes in fp32
and casts back before the weight, like transformers' Qwen2RMSNorm.  Both, the
residual adds and the SiLU product run as fused HIP kernels
(include/flexengine_amd_model.h); the projections run on the skinny HIP GEMM
for decode-sized batches and on the library GEMM (hipBLASLt via torch) above.
Default configuration: Qwen2.5-1.5B (28 layers, hidden 1536, 12/2 heads,
head_dim 128, intermediate 8960, vocab 151936, tied embeddings, q/k/v bias,
RMS eps 1e-6, theta 1e6).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from flexengine_amd import attention, ops



@dataclass
class Qwen2Config:
    vocab_size: int = 151936
    hidden_size: int = 1536
    intermediate_size: int = 8960
    num_hidden_layers: int = 28
    num_attention_heads: int = 12
    num_key_value_heads: int = 2
    head_dim: int = 128
    rope_theta: float = 1000000.0
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = True

    @property
    def parameters(self) -> int:
        h, i, d = self.hidden_size, self.intermediate_size, self.head_dim
        qkv = h * (self.num_attention_heads + 2 * self.num_key_value_heads) * d
        qkv += (self.num_attention_heads + 2 * self.num_key_value_heads) * d
        per_layer = qkv + self.num_attention_heads * d * h + 3 * h * i + 2 * h
        head = 0 if self.tie_word_embeddings else self.vocab_size * h
        return self.vocab_size * h + self.num_hidden_layers * per_layer + h + head


@dataclass
class Chunk:
    """A run of new tokens of one request (engine/scheduler/policies.py:15-18)."""
    request_id: str
    input_ids: list[int]
    start: int


class _Layer:
    def __init__(self, cfg: Qwen2Config, dev, dtype, gen, std):
        h, i, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        nqkv = (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * d

        def randn(*shape):
            return (torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dtype)

        self.input_norm = torch.ones(h, device=dev, dtype=dtype)
        self.post_norm = torch.ones(h, device=dev, dtype=dtype)
        # q, k and v projections stacked into one GEMM: rows [q | k | v]
        self.w_qkv = randn(nqkv, h)
        self.b_qkv = randn(nqkv)
        self.w_o = randn(h, cfg.num_attention_heads * d)
        # gate and up stacked into one GEMM: rows [gate | up]
        self.w_gate_up = randn(2 * i, h)
        self.w_down = randn(h, i)


class Qwen2Model:
    def __init__(self, cfg: Qwen2Config | None = None, device: str | torch.device = "cuda:0",
                 dtype=torch.float16, seed: int = 5, std: float = 0.02):
        self.cfg = cfg = cfg or Qwen2Config()
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("Qwen2Model runs its attention on the HIP kernels: ROCm GPU only")
        if cfg.num_attention_heads % cfg.num_key_value_heads:
            raise ValueError("Invalid GQA head ratio")
        self.dtype = dtype
        self.nq, self.nkv, self.dim = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.layers = cfg.num_hidden_layers
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        self.embed = (torch.randn((cfg.vocab_size, cfg.hidden_size), generator=gen, device=self.device,
                                  dtype=torch.float32) * std).to(dtype)
        self.layer_weights = [_Layer(cfg, self.device, dtype, gen, std) for _ in range(self.layers)]
        self.final_norm = torch.ones(cfg.hidden_size, device=self.device, dtype=dtype)
        self.lm_head = self.embed if cfg.tie_word_embeddings else (
            torch.randn((cfg.vocab_size, cfg.hidden_size), generator=gen, device=self.device,
                        dtype=torch.float32) * std).to(dtype)
        self.inv_freq = 1.0 / cfg.rope_theta ** (
            torch.arange(0, self.dim, 2, device=self.device, dtype=torch.float32) / self.dim)
        self.scale = 1.0 / math.sqrt(self.dim)

    # ---- building blocks ----------------------------------------------------------
    # Per layer: fused add + RMSNorm, the q/k/v GEMM, RoPE + split, attention, the o
    # GEMM, add + RMSNorm, the gate/up GEMM, SiLU product, the down GEMM.  GEMMs of
    # up to ops.SKINNY_MAX_ROWS rows run on the skinny HIP GEMM, whose fp32 partials
    # the next kernel sums; larger ones on the library GEMM.

    def _qkv(self, h: torch.Tensor, lw: _Layer, positions: torch.Tensor):
        qkv = ops.linear(h, lw.w_qkv, lw.b_qkv)
        return ops.rope_qkv(qkv, positions, self.inv_freq, self.nq, self.nkv, self.dim,
                            bias=lw.b_qkv)

    def _after_attention(self, x: torch.Tensor, attn: torch.Tensor, lw: _Layer,
                         next_norm: torch.Tensor) -> torch.Tensor:
        """Residual stream update of one layer after its attention; x is updated in
        place and the normalised input of the next layer (or of the LM head) returned."""
        o = ops.linear(attn.reshape(x.shape[0], self.nq * self.dim), lw.w_o)
        h2, _ = ops.rmsnorm(o, lw.post_norm, self.cfg.rms_norm_eps, residual=x)
        act = ops.silu_mul(ops.linear(h2, lw.w_gate_up))
        h, _ = ops.rmsnorm(ops.linear(act, lw.w_down), next_norm, self.cfg.rms_norm_eps, residual=x)
        return h

    def _next_norm(self, layer: int) -> torch.Tensor:
        return (self.layer_weights[layer + 1].input_norm if layer + 1 < self.layers
                else self.final_norm)

    def _logits(self, h: torch.Tensor) -> torch.Tensor:
        out = ops.linear(h, self.lm_head)
        if out.dtype == torch.float32:  # skinny-GEMM partials
            out = (out.sum(0) if out.shape[0] > 1 else out[0]).to(self.dtype)
        return out

    # ---- the two forwards ---------------------------------------------------------

    @torch.inference_mode()
    def forward(self, chunks: list[Chunk], cache) -> list[torch.Tensor]:
        """Ragged mixed batch (qwen2.py:79-136); returns the last-token logits per chunk."""
        lengths = [len(c.input_ids) for c in chunks]
        if not chunks or any(n < 1 for n in lengths):
            raise ValueError("empty forward chunks")
        dev = self.device
        ids = torch.tensor([t for c in chunks for t in c.input_ids], dtype=torch.long).to(dev)
        pos_list = [p for c in chunks for p in range(c.start, c.start + len(c.input_ids))]
        positions = torch.tensor(pos_list, dtype=torch.long).to(dev)
        # the write's checks of allocator.py:107-125 on the host bookkeeping (slots
        # reserved, no shared block written); the slot map itself is computed on
        # the device from the block tables (fe_write_kv_ragged), which are
        # gathered from the cache's device mirror (fe_gather_tables)
        bs = cache.layout.block_size
        for c in chunks:
            end = c.start + len(c.input_ids)
            if c.start < 0 or end > cache.available_slots(c.request_id):
                raise IndexError("KV slots not reserved")
            table = cache.tables[c.request_id]
            if any(cache.refs[table[p]] > 1 for p in range(c.start // bs, (end - 1) // bs + 1)):
                raise RuntimeError("cannot write a shared immutable KV block")
        width = max(len(cache.tables[c.request_id]) for c in chunks)
        tables = cache.device_tables([c.request_id for c in chunks], width)
        q_offsets = torch.tensor([0] + [sum(lengths[:j + 1]) for j in range(len(lengths))],
                                 dtype=torch.int32).to(dev)
        ctx = torch.tensor([c.start + n for c, n in zip(chunks, lengths)], dtype=torch.int32).to(dev)
        max_q = max(lengths)
        # the prefill's work split of this step, shared by every layer (None when
        # the sizes take the tile kernel)
        plan = ops.prefill_paged_plan(q_offsets, ctx, len(pos_list),
                                      self.cfg.num_attention_heads, self.cfg.num_key_value_heads,
                                      width, bs)
        x = self.embed.index_select(0, ids)
        h, _ = ops.rmsnorm(x, self.layer_weights[0].input_norm, self.cfg.rms_norm_eps)
        for layer, lw in enumerate(self.layer_weights):
            q, k, v = self._qkv(h, lw, positions)
            ops.write_kv_ragged(k, v, cache.k[layer], cache.v[layer], tables, q_offsets, ctx)
            attn = ops.prefill_paged(q, cache.k[layer], cache.v[layer], tables, q_offsets, ctx,
                                     max_q, scale=self.scale, plan=plan)
            h = self._after_attention(x, attn, lw, self._next_norm(layer))
        ends = torch.tensor([sum(lengths[:j + 1]) - 1 for j in range(len(lengths))],
                            dtype=torch.long).to(dev)
        logits = self._logits(h.index_select(0, ends))
        return [logits[j] for j in range(len(lengths))]

    @torch.inference_mode()
    def decode_static(self, input_ids: torch.Tensor, positions: torch.Tensor,
                      block_tables: torch.Tensor, active_mask: torch.Tensor, cache) -> torch.Tensor:
        """Graph-compatible one-token decode over fixed padded batch tensors
        (qwen2.py:138-186): logits [B, vocab], zero for inactive rows."""
        batch = input_ids.shape[0]
        if input_ids.ndim != 1 or positions.shape != (batch,) or active_mask.reshape(-1).shape != (batch,):
            raise ValueError("invalid static decode inputs")
        active = active_mask.reshape(-1)
        # the batched backend contract's conversions, once per step for all layers
        # (paged_attention.py:115,131,138): length = position + 1, 0 for inactive rows
        ctx = attention.context_lens_from_positions(positions, active)
        tables = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
        tables = tables.contiguous()
        # the decode plan (split-K partition and block rows) of this step, shared by
        # every layer: the tables and lengths are the same for all of them
        nb, bs, hkv = cache.k[0].shape[0], cache.k[0].shape[1], cache.k[0].shape[2]
        plan = ops.paged_decode_plan(tables, ctx, nb, hkv, bs) if bs % 16 == 0 else None
        x = self.embed.index_select(0, input_ids)
        h, _ = ops.rmsnorm(x, self.layer_weights[0].input_norm, self.cfg.rms_norm_eps)
        if batch <= ops.SKINNY_MAX_ROWS and self.cfg.hidden_size % 32 == 0:
            logits = self._decode_layers_fused(x, h, positions, tables, ctx, cache, plan)
        else:
            for layer, lw in enumerate(self.layer_weights):
                q, k, v = self._qkv(h, lw, positions)
                attn = ops.paged_decode(q, cache.k[layer], cache.v[layer], tables, ctx,
                                        scale=self.scale, k_new=k, v_new=v, plan=plan)
                h = self._after_attention(x, attn, lw, self._next_norm(layer))
            logits = self._logits(h)
        return logits * active.to(logits.dtype)[:, None]

    def _decode_layers_fused(self, x, h, positions, tables, ctx, cache, plan=None) -> torch.Tensor:
        """The decode layers at decode batch sizes on the fused projections: five
        launches per layer -- q/k/v + bias + RoPE, the paged decode with the page
        write, o + residual + RMSNorm, gate/up + SiLU, down + residual + the next
        RMSNorm -- where the unfused chain needs nine.  The residual stream alternates
        between fresh tensors (r1 after attention, r2 after the MLP).  Each norm runs
        in the residual projection that produces its input (the workgroup finishing
        the last tile normalises the rows); normalising the operand inside the next
        projection instead measured slower, every lane transforming its 16 MFMA
        columns.  Hidden sizes the fused norm does not take use a separate
        fe_rmsnorm launch."""
        eps = self.cfg.rms_norm_eps
        res = x
        rows = x.shape[0]
        fused_norm = ops.resid_rmsnorm_supported(self.cfg.hidden_size)
        for layer, lw in enumerate(self.layer_weights):
            q, k, v = ops.gemm_rope(h, lw.w_qkv, lw.b_qkv, positions, self.inv_freq,
                                    self.nq, self.nkv, self.dim)
            attn = ops.paged_decode(q, cache.k[layer], cache.v[layer], tables, ctx, scale=self.scale,
                                    k_new=k, v_new=v, plan=plan)
            o_in = attn.reshape(rows, self.nq * self.dim)
            if fused_norm:
                r1, h2 = ops.gemm_resid_rmsnorm(o_in, lw.w_o, res, lw.post_norm, eps)
                act = ops.gemm_silu(h2, lw.w_gate_up)
                r2, h = ops.gemm_resid_rmsnorm(act, lw.w_down, r1, self._next_norm(layer), eps)
            else:
                r1, _ = ops.gemm_resid(o_in, lw.w_o, res)
                h2, _ = ops.rmsnorm(r1, lw.post_norm, eps)
                act = ops.gemm_silu(h2, lw.w_gate_up)
                r2, _ = ops.gemm_resid(act, lw.w_down, r1)
                h, _ = ops.rmsnorm(r2, self._next_norm(layer), eps)
            res = r2
        return ops.gemm_f16(h, self.lm_head)
