"""Decode throughput of the package's Qwen2.5-1.5B on one GPU (config C5).

    python -m flexengine_amd.bench_model [--batches 1,2,3,4,8] [--eager-batch 64]
                                         [--steps 32] [--warmup 4]

Random-initialised Qwen2.5-1.5B (weights N(0, 0.02) fp16, norms 1, seed 5);
every sequence starts with a KV cache of L ~ U{512..4096} tokens pre-filled
with N(0, 1) values, then decodes greedily (argmax) one token per step.
Batches of 1..8 run as hipGraph replays of the bucket that holds them (3 -> 4,
5..7 -> 8, padded rows inactive), as FlexEngine's graph decode path does; the
large batch runs eagerly and also as a captured graph of its own size.
One JSON line per configuration: tokens/s, ms per step, and the HBM bytes a
step must read (weights + the KV of every active sequence) as GB/s.
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import torch

from flexengine_amd.decode_step import GraphDecodeStep
from flexengine_amd.graphs import DecodeGraphManager
from flexengine_amd.kv_cache import CacheLayout, PagedKVCache
from flexengine_amd.model import Chunk, Qwen2Config, Qwen2Model


def make_cache(model: Qwen2Model, lengths: list[int], steps: int, seed: int) -> PagedKVCache:
    bs = 16
    blocks = sum((n + steps + bs) // bs + 1 for n in lengths) + 16
    cache = PagedKVCache(CacheLayout(model.layers, blocks, bs, model.nkv, model.dim), device=model.device)
    gen = torch.Generator(device=model.device)
    gen.manual_seed(seed)
    for layer in range(model.layers):  # N(0, 1) K/V everywhere, one layer at a time
        cache.k[layer].normal_(generator=gen)
        cache.v[layer].normal_(generator=gen)
    for b, n in enumerate(lengths):
        cache.reserve(f"r{b}", n + steps + 1)
    return cache


def run(model, batch: int, steps: int, warmup: int, mode: str, seed: int = 5) -> dict:
    rng = torch.Generator().manual_seed(seed * 1000 + batch)
    lengths = torch.randint(512, 4097, (batch,), generator=rng).tolist()
    tokens = torch.randint(0, model.cfg.vocab_size, (batch,), generator=rng).tolist()
    cache = make_cache(model, lengths, warmup + steps, seed)
    dev = model.device
    if mode == "bucket":
        step = GraphDecodeStep(model, cache, max_model_len=4096 + warmup + steps + 16)
    else:
        step = GraphDecodeStep(model, cache, max_model_len=4096 + warmup + steps + 16,
                               manager=DecodeGraphManager(dev, buckets=(batch,)))
    pos = list(lengths)

    def one():
        chunks = [Chunk(f"r{b}", [tokens[b]], pos[b]) for b in range(batch)]
        if mode == "eager":
            inputs = step.graph_inputs(chunks, batch)
            logits = model.decode_static(**inputs, active_mask=torch.ones(batch, device=dev),
                                         cache=cache)
        else:
            out = step(chunks)
            if out is None:
                raise RuntimeError("graph step fell back to eager")
            logits = torch.stack(out)
        nxt = logits.argmax(-1).tolist()
        for b in range(batch):
            tokens[b] = nxt[b]
            pos[b] += 1

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / steps
    weights = model.cfg.parameters * 2
    # K/V bytes read per step at the timed steps' mean context
    kv_mean = (sum(lengths) + batch * (warmup + steps / 2)) * model.layers * 2 * model.nkv * model.dim * 2
    bucket = step.manager.bucket_for(batch) if mode == "bucket" else batch
    return {"metric": "decode tok/s Qwen2.5-1.5B", "batch": batch, "mode": mode,
            "graph_batch": None if mode == "eager" else bucket, "tok_s": round(batch / sec, 1),
            "ms_per_step": round(sec * 1e3, 3), "mean_context": round(sum(lengths) / batch + warmup + steps / 2),
            "hbm_bytes_per_step": int(weights + kv_mean),
            "hbm_GB_s": round((weights + kv_mean) / sec / 1e9, 1), "steps": steps, "warmup": warmup,
            "data": "synthetic: random-init weights N(0,0.02), KV N(0,1), L~U{512..4096}, seed 5"}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--batches", default="1,2,3,4,8")
    p.add_argument("--eager-batch", type=int, default=64)
    p.add_argument("--steps", type=int, default=32)
    p.add_argument("--warmup", type=int, default=4)
    args = p.parse_args(argv)
    if not torch.cuda.is_available():
        print("bench_model needs a ROCm GPU", file=sys.stderr)
        return 2
    model = Qwen2Model(Qwen2Config(), "cuda:0", seed=5)
    for b in [int(x) for x in args.batches.split(",") if x]:
        print(json.dumps(run(model, b, args.steps, args.warmup, "bucket")), flush=True)
    if args.eager_batch:
        for mode in ("eager", "graph"):
            print(json.dumps(run(model, args.eager_batch, args.steps, args.warmup, mode)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
