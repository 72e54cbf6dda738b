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
