"""GPU: the package's Qwen2 decoder on the HIP kernels against an independent
dense float64 forward (oracle/qwen2_ref.py), incremental prefill, the
graph-compatible decode step, and hipGraph bucket replay against eager.

Follows the reference's tests/unit/test_synthetic_qwen.py (full vs incremental
prefill, multi-request isolation), tests/gpu/test_cuda_graph.py and
tests/gpu/test_engine_cuda_graph.py:45-57 (graph tokens == eager tokens for
active counts 1, 2, 3, 4, 5, 8; 9 falls back), with a small random-init
configuration instead of HF weights.
"""
from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu

from flexengine_amd.decode_step import GraphDecodeStep  # noqa: E402
from flexengine_amd.kv_cache import CacheLayout, PagedKVCache  # noqa: E402
from flexengine_amd.model import Chunk, Qwen2Config, Qwen2Model  # noqa: E402
from oracle.qwen2_ref import reference_logits  # noqa: E402

DEV = "cuda:0"
# logits of the fp16 model vs the float64 dense forward: fp16 activations through every
# layer, so the error scales with the logits' magnitude (one fp16 ulp is ~1e-3 relative);
# bounds relative to max|logit|: max error 0.5%, mean error 0.1%.  A wrong RoPE sign, GQA
# map, mask or KV slot moves logits by tens of percent.
MAX_REL, MEAN_REL = 5e-3, 1e-3


def tiny(d=64, hq=4, hkv=2, layers=2, std=0.1, seed=7):
    cfg = Qwen2Config(vocab_size=320, hidden_size=hq * d, intermediate_size=192,
                      num_hidden_layers=layers, num_attention_heads=hq, num_key_value_heads=hkv,
                      head_dim=d)
    return Qwen2Model(cfg, DEV, seed=seed, std=std)


def cache_for(model, num_blocks=96, block_size=4):
    return PagedKVCache(CacheLayout(model.layers, num_blocks, block_size, model.nkv, model.dim),
                        device=DEV, fill=float("nan"))


def close(got, want):
    scale = want.abs().max().item()
    err = (got.double().cpu() - want).abs()
    assert err.max().item() <= MAX_REL * scale, (err.max().item(), scale)
    assert err.mean().item() <= MEAN_REL * scale, (err.mean().item(), scale)


@pytest.mark.parametrize("d,hq,hkv", [(64, 4, 2), (128, 6, 1)])
def test_forward_full_incremental_and_multi_request(d, hq, hkv):
    model = tiny(d, hq, hkv)
    cache = cache_for(model)
    a = [2, 5, 3, 8, 9, 4, 7, 12, 10, 31, 44, 17, 9]
    b = [16, 8, 9, 2]
    cache.reserve("a", len(a))
    cache.reserve("b", len(b))
    got = model.forward([Chunk("a", a, 0), Chunk("b", b, 0)], cache)
    close(got[0], reference_logits(model, a))
    close(got[1], reference_logits(model, b))
    # incremental prefill of the same request (chunks of 3, 5 and the rest)
    cache.free_request("a")
    cache.reserve("a", len(a))
    model.forward([Chunk("a", a[:3], 0)], cache)
    model.forward([Chunk("a", a[3:8], 3)], cache)
    last = model.forward([Chunk("a", a[8:], 8)], cache)[0]
    close(last, reference_logits(model, a))
    cache.assert_invariants()


def test_mixed_prefill_and_decode_chunks_in_one_forward():
    model = tiny()
    cache = cache_for(model)
    seqs = {"p": [3, 1, 4, 1, 5, 9, 2, 6], "d": [2, 7, 1, 8, 2, 8]}
    for rid, ids in seqs.items():
        cache.reserve(rid, len(ids))
    model.forward([Chunk("d", seqs["d"][:-1], 0)], cache)
    got = model.forward([Chunk("p", seqs["p"], 0), Chunk("d", seqs["d"][-1:], len(seqs["d"]) - 1)],
                        cache)
    close(got[0], reference_logits(model, seqs["p"]))
    close(got[1], reference_logits(model, seqs["d"]))


def test_decode_static_matches_dense_and_masks_inactive_rows():
    model = tiny()
    cache = cache_for(model)
    seqs = [[5, 6, 7, 8, 9], [1, 2], [11, 12, 13, 14, 15, 16, 17, 18, 19]]
    for i, ids in enumerate(seqs):
        cache.reserve(str(i), len(ids))
        model.forward([Chunk(str(i), ids[:-1], 0)], cache)
    # rows 0..2 decode their last token; row 3 is padding
    width = max(len(cache.tables[str(i)]) for i in range(3))
    tables = cache.block_table([str(i) for i in range(3)], width)
    tables = torch.cat([tables, tables[:1]]).long()
    ids = torch.tensor([s[-1] for s in seqs] + [0], device=DEV)
    pos = torch.tensor([len(s) - 1 for s in seqs] + [0], device=DEV)
    active = torch.tensor([1, 1, 1, 0], device=DEV)
    logits = model.decode_static(ids, pos, tables, active, cache)
    for i, s in enumerate(seqs):
        close(logits[i], reference_logits(model, s))
    assert torch.count_nonzero(logits[3]) == 0


def greedy(model, cache, step, prompts, new_tokens, graph: bool):
    """Prefill every prompt eagerly, then decode new_tokens tokens per request,
    through the graph step (graph=True) or eager decode_static."""
    ids = {rid: list(p) for rid, p in prompts.items()}
    for rid, p in prompts.items():
        cache.reserve(rid, len(p) + new_tokens)
        logits = model.forward([Chunk(rid, p, 0)], cache)[0]
        ids[rid].append(int(logits.argmax()))
    for _ in range(new_tokens - 1):
        chunks = [Chunk(rid, [toks[-1]], len(toks) - 1) for rid, toks in ids.items()]
        out = step(chunks) if graph else None
        if out is None:
            inputs = step.graph_inputs(chunks, len(chunks))
            out = model.decode_static(**inputs, active_mask=torch.ones(len(chunks), device=DEV),
                                      cache=cache)
        for chunk, row in zip(chunks, out):
            ids[chunk.request_id].append(int(row.argmax()))
    return ids


@pytest.mark.parametrize("active", [1, 2, 3, 4, 5, 8, 9])
def test_graph_replay_tokens_equal_eager(active):
    model = tiny(layers=2, std=0.3)
    prompts = {f"r{i}": [(7 * i + j) % 300 + 1 for j in range(3 + 2 * i)] for i in range(active)}
    runs = {}
    for graph in (False, True):
        cache = cache_for(model, num_blocks=160)
        step = GraphDecodeStep(model, cache, max_model_len=64)
        runs[graph] = greedy(model, cache, step, prompts, 4, graph)
        stats = step.manager.stats()
    assert runs[True] == runs[False]
    if active <= 8:
        assert stats["replays"] >= 1 and stats["captures"] >= 1
        assert stats["padded_slots"] >= (1 if active in (3, 5) else 0)
        assert stats["fallbacks"] == 0
    else:
        assert stats["fallbacks"] >= 1 and stats["replays"] == 0


def test_graph_staging_addresses_are_stable_across_replays():
    model = tiny()
    cache = cache_for(model)
    step = GraphDecodeStep(model, cache, max_model_len=32)
    for rid in ("x", "y", "z"):
        cache.reserve(rid, 8)
        model.forward([Chunk(rid, [1, 2, 3], 0)], cache)
    chunks = [Chunk("x", [4], 3), Chunk("y", [5], 3), Chunk("z", [6], 3)]
    first = step(chunks)
    addrs = step.manager.staging_addresses(4)
    second = step([Chunk("x", [7], 4), Chunk("y", [8], 4), Chunk("z", [9], 4)])
    assert first is not None and second is not None
    assert step.manager.staging_addresses(4) == addrs
    assert step.manager.stats()["padded_slots"] == 2 and step.manager.stats()["captures"] == 1


def test_full_size_qwen25_15b_shapes_decode_and_prefill():
    """The 1.5B configuration itself (28 layers, 12/2 heads, D 128): one prefill
    and two graph-replayed decode steps give finite logits of the right shape."""
    model = Qwen2Model(Qwen2Config(), DEV)
    assert abs(model.cfg.parameters - 1.5437e9) / 1.5437e9 < 0.01
    cache = PagedKVCache(CacheLayout(28, 64, 16, 2, 128), device=DEV)
    cache.reserve("a", 40)
    cache.reserve("b", 40)
    logits = model.forward([Chunk("a", list(range(1, 20)), 0), Chunk("b", [5, 6, 7], 0)], cache)
    assert logits[0].shape == (151936,) and torch.isfinite(logits[0]).all()
    step = GraphDecodeStep(model, cache, max_model_len=64)
    out = step([Chunk("a", [int(logits[0].argmax())], 19), Chunk("b", [int(logits[1].argmax())], 3)])
    assert out is not None and torch.isfinite(out[0]).all()
    out = step([Chunk("a", [int(out[0].argmax())], 20), Chunk("b", [int(out[1].argmax())], 4)])
    assert out is not None and step.manager.stats()["replays"] == 2


# --------------------------------------------------------------------------------------
# C5 at its stated configuration: Qwen2.5-1.5B shapes, contexts U{512..4096}
# --------------------------------------------------------------------------------------

C5_ROWS = 64
C5_STEPS = 12


@pytest.fixture(scope="module")
def c5():
    """Random-init Qwen2.5-1.5B (seed 5) and a paged cache holding 64 requests with
    L ~ U{512..4096} tokens of N(0, 1) K/V in every layer (bench_model's set-up)."""
    model = Qwen2Model(Qwen2Config(), DEV, seed=5)
    gen = torch.Generator().manual_seed(505)
    lengths = torch.randint(512, 4097, (C5_ROWS,), generator=gen).tolist()
    tokens = torch.randint(0, model.cfg.vocab_size, (C5_ROWS,), generator=gen).tolist()
    bs = 16
    # spare blocks: the scratch requests of a bucket-8 and a bucket-64 graph step
    blocks = sum((n + C5_STEPS + bs) // bs + 1 for n in lengths) + 64 + 64
    cache = PagedKVCache(CacheLayout(model.layers, blocks, bs, model.nkv, model.dim), device=DEV)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    for layer in range(model.layers):
        cache.k[layer].normal_(generator=g)
        cache.v[layer].normal_(generator=g)
    for b, n in enumerate(lengths):
        cache.reserve(f"r{b}", n + C5_STEPS + 1)
    step = GraphDecodeStep(model, cache, max_model_len=4096 + C5_STEPS + 32)
    state = {"pos": list(lengths), "tok": tokens}
    yield model, cache, step, state
    del step, cache, model
    torch.cuda.empty_cache()


def _eager(model, cache, step, chunks):
    inputs = step.graph_inputs(chunks, len(chunks))
    return model.decode_static(**inputs, active_mask=torch.ones(len(chunks), device=DEV),
                               cache=cache)


def _agree(graph_rows, eager_rows, what):
    """Logits within the model tolerance; greedy tokens equal wherever the eager
    top-2 margin exceeds the tolerance (a near-tie may flip either way)."""
    g = torch.stack(list(graph_rows)).double().cpu()
    e = eager_rows.double().cpu()
    scale = e.abs().max().item()
    err = (g - e).abs()
    print(f"{what}: max err {err.max().item():.3e} mean {err.mean().item():.3e} "
          f"(max |logit| {scale:.3f})", flush=True)
    assert err.max().item() <= MAX_REL * scale, what
    assert err.mean().item() <= MEAN_REL * scale, what
    top2 = e.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * MAX_REL * scale
    assert torch.equal(g.argmax(-1)[clear], e.argmax(-1)[clear]), what


def test_c5_buckets_captured_together_replay_interleaved_like_eager(c5):
    """tests/gpu/test_engine_cuda_graph.py:45-57 at the C5 configuration: buckets 1, 2,
    4 and 8 captured lazily in one GraphDecodeStep (the engine's order), replayed in
    interleaved order for active counts 1, 2, 3, 4, 5, 8, each step matching eager
    decode_static on the same cache state; 9 rows fall back.  Later replays of a
    bucket captured before a larger one exercise the graph-owned workspaces."""
    model, cache, step, st = c5
    for n in (8, 1, 4, 2, 3, 5, 1, 8, 2, 4):
        chunks = [Chunk(f"r{b}", [st["tok"][b]], st["pos"][b]) for b in range(n)]
        eager = _eager(model, cache, step, chunks)
        out = step(chunks)
        assert out is not None, f"{n} rows fell back"
        _agree(out, eager, f"C5 {n} active rows (bucket {step.manager.bucket_for(n)})")
        for b in range(n):
            st["tok"][b] = int(out[b].argmax())
            st["pos"][b] += 1
    stats = step.manager.stats()
    assert stats["captures"] == 4 and stats["fallbacks"] == 0 and stats["replays"] == 10
    assert stats["padded_slots"] == 1 + 3         # 3 rows in bucket 4, 5 rows in bucket 8
    assert step([Chunk(f"r{b}", [st["tok"][b]], st["pos"][b]) for b in range(9)]) is None
    assert step.manager.stats()["fallbacks"] == 1


# Full-depth tolerance against the float32 reference: the 2-layer bounds above,
# scaled by sqrt(28 / 2) for the independent fp16 roundings of 14x as many layers
# (each layer rounds at about ten points), i.e. max 2e-2 and mean 4e-3 of
# max |logit|.  A wrong row, position, head map or KV slot moves logits by tens
# of percent.
DEEP_MAX_REL, DEEP_MEAN_REL = 2e-2, 4e-3


@torch.inference_mode()
def _fp32_decode_reference(model, cache, chunks):
    """Plain PyTorch float32 decode step of the same model on the same cache: fp32
    weights, RMSNorm, RoPE (qwen2.py:73-77), attention over the cached K/V of
    positions < p (read back from the pool) plus the step's own K/V at p, and the
    tied LM head.  Logits [B, vocab] float32."""
    cfg = model.cfg
    eps, d, hq, hkv = cfg.rms_norm_eps, model.dim, model.nq, model.nkv
    grp = hq // hkv
    dev = model.device
    bs = cache.layout.block_size
    pos = torch.tensor([c.start for c in chunks], device=dev)
    x = model.embed.index_select(0, torch.tensor([c.input_ids[0] for c in chunks],
                                                 device=dev)).float()
    ang = pos[:, None].float() * model.inv_freq[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[:, None, :]

    def rms(t, w):
        return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + eps) * w.float()

    def rope(t):
        rot = torch.cat([-t[..., d // 2:], t[..., :d // 2]], -1)
        return t * cos + rot * sin

    tables = [torch.tensor(cache.tables[c.request_id], device=dev) for c in chunks]
    for layer, lw in enumerate(model.layer_weights):
        h = rms(x, lw.input_norm)
        qkv = h @ lw.w_qkv.float().t() + lw.b_qkv.float()
        q = rope(qkv[:, :hq * d].reshape(-1, hq, d))
        k = rope(qkv[:, hq * d:(hq + hkv) * d].reshape(-1, hkv, d))
        v = qkv[:, (hq + hkv) * d:].reshape(-1, hkv, d)
        attn = torch.empty_like(q)
        for b, c in enumerate(chunks):
            p = c.start
            kc = cache.k[layer][tables[b]].reshape(-1, hkv, d)[:p].float()
            vc = cache.v[layer][tables[b]].reshape(-1, hkv, d)[:p].float()
            kc = torch.cat([kc, k[b:b + 1]], 0).repeat_interleave(grp, dim=1)   # [p+1, Hq, D]
            vc = torch.cat([vc, v[b:b + 1]], 0).repeat_interleave(grp, dim=1)
            w = torch.softmax((kc * q[b][None]).sum(-1) / math.sqrt(d), dim=0)  # [p+1, Hq]
            attn[b] = (w[..., None] * vc).sum(0)
        x = x + attn.reshape(-1, hq * d) @ lw.w_o.float().t()
        gu = rms(x, lw.post_norm) @ lw.w_gate_up.float().t()
        g, u = gu.chunk(2, dim=-1)
        x = x + (torch.nn.functional.silu(g) * u) @ lw.w_down.float().t()
    return rms(x, model.final_norm) @ model.lm_head.float().t()


def _near(got_rows, ref, what):
    g = torch.stack(list(got_rows)).double().cpu() if not torch.is_tensor(got_rows) \
        else got_rows.double().cpu()
    e = ref.double().cpu()
    scale = e.abs().max().item()
    err = (g - e).abs()
    print(f"{what}: max err {err.max().item():.3e} mean {err.mean().item():.3e} "
          f"(max |logit| {scale:.3f})", flush=True)
    assert err.max().item() <= DEEP_MAX_REL * scale, what
    assert err.mean().item() <= DEEP_MEAN_REL * scale, what
    top2 = e.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * DEEP_MAX_REL * scale
    assert torch.equal(g.argmax(-1)[clear], e.argmax(-1)[clear]), what


def test_c5_eager_b64_and_bucket8_replays_against_fp32(c5):
    """Batch invariance at 64 rows: one eager decode_static step over all 64 rows
    (fe_gemm_rows64 for every projection but the LM head, unfused layer kernels)
    and eight bucket-8 graph replays of the same rows (fused projections), on the
    same cache state, each against a plain PyTorch float32 decode step of the same
    model."""
    model, cache, step, st = c5
    chunks = [Chunk(f"r{b}", [st["tok"][b]], st["pos"][b]) for b in range(C5_ROWS)]
    eager = _eager(model, cache, step, chunks)
    rows = []
    for i in range(0, C5_ROWS, 8):
        out = step(chunks[i:i + 8])
        assert out is not None
        rows.extend(out)
    ref = _fp32_decode_reference(model, cache, chunks)
    _near(eager, ref, "C5 eager B=64 vs fp32")
    _near(rows, ref, "C5 8 x bucket 8 vs fp32")
    _near(rows, eager.float(), "C5 8 x bucket 8 vs eager B=64")


def test_c5_b64_graph_replays_against_fp32_and_eager(c5):
    """The 64-row step as bench.py's c5.b64_graph runs it: decode_static captured in
    a 64-row bucket, where ops.linear routes differently than eagerly (inside a
    capture only the deep down projection takes fe_gemm_rows64; q/k/v, o, gate/up
    and the LM head take the library GEMM).  Two replays on the same cache state,
    each against the float32 decode and the eager 64-row step."""
    from flexengine_amd.graphs import DecodeGraphManager
    model, cache, step8, st = c5
    step = GraphDecodeStep(model, cache, max_model_len=4096 + C5_STEPS + 32,
                           manager=DecodeGraphManager(DEV, buckets=(C5_ROWS,)))
    chunks = [Chunk(f"r{b}", [st["tok"][b]], st["pos"][b]) for b in range(C5_ROWS)]
    ref = _fp32_decode_reference(model, cache, chunks)
    eager = _eager(model, cache, step, chunks)
    for rep in range(2):
        out = step(chunks)
        assert out is not None, "the 64-row bucket fell back"
        _near(out, ref, f"C5 64-row graph replay {rep} vs fp32")
        _near(out, eager.float(), f"C5 64-row graph replay {rep} vs eager B=64")
    stats = step.manager.stats()
    assert stats["captures"] == 1 and stats["replays"] == 2 and stats["fallbacks"] == 0
