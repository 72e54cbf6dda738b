"""CPU: host-side logic -- KV-cache bookkeeping, graph buckets, workload generators.

The bookkeeping cases restate the reference's allocator tests
(tests/unit/test_allocator.py, test_attention.py:25-31) and graph-manager
tests (tests/gpu/test_cuda_graph.py:7-26), which run on the CPU there too.
"""
from __future__ import annotations

import math

import pytest
import torch

from flexengine_amd import attention, workloads
from flexengine_amd.graphs import DecodeGraphManager
from flexengine_amd.kv_cache import CacheExhausted, CacheLayout, PagedKVCache


def make_cache(n=10, block=4):
    return PagedKVCache(CacheLayout(2, n, block, 2, 8), device="cpu")


def test_reserve_across_boundaries():
    c = make_cache(10, 4)
    c.reserve("a", 3)
    c.reserve("a", 5)
    c.reserve("b", 7)
    assert c.tables["a"] == [0, 1] and c.tables["b"] == [2, 3]
    c.assert_invariants()
    c.free_request("a")
    c.free_request("b")
    c.assert_invariants()
    assert c.free_blocks == 10


def test_reserve_is_atomic_and_oom_handled():
    c = make_cache(3, 2)
    c.reserve("a", 4)
    with pytest.raises(CacheExhausted):
        c.reserve("b", 4)
    assert "b" not in c.tables
    c.free_request("a")
    c.reserve("b", 4)
    c.assert_invariants()


def test_block_reuse_no_leak():
    c = make_cache(7, 4)
    for _ in range(500):
        c.reserve("x", 17)
        c.free_request("x")
    assert c.free_blocks == 7
    c.assert_invariants()


def test_invalid_slot_raises_before_any_device_work():
    c = make_cache()
    c.reserve("a", 4)
    with pytest.raises(IndexError):
        c.write(0, "a", 4, torch.zeros(1, 2, 8, dtype=torch.float16),
                torch.zeros(1, 2, 8, dtype=torch.float16))


def test_write_on_cpu_pool_fails_loudly():
    c = make_cache()
    c.reserve("a", 4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        c.write(0, "a", 0, torch.zeros(2, 2, 8, dtype=torch.float16),
                torch.zeros(2, 2, 8, dtype=torch.float16))


def test_retain_and_release_block():
    c = make_cache()
    c.reserve("a", 4)
    block = c.tables["a"][0]
    c.retain_block(block)
    c.free_request("a")
    assert c.refs[block] == 1 and block not in c.free
    c.release_block(block)
    assert c.refs[block] == 0 and block in c.free
    c.assert_invariants()


def test_noncontiguous_table_order():
    """test_attention.py:25-31: interleaved reservations give table [0, 3, 4]."""
    c = PagedKVCache(CacheLayout(1, 8, 2, 1, 8), device="cpu")
    c.reserve("a", 2)
    c.reserve("other", 4)
    c.reserve("a", 5)
    assert c.tables["a"] == [0, 3, 4]


def test_attach_prefix_and_block_table_padding():
    c = make_cache(12, 4)
    c.reserve("p", 8)
    c.attach_prefix("q", c.tables["p"])
    c.reserve("q", 10)
    assert c.refs[0] == 2 and len(c.tables["q"]) == 3
    t = c.block_table(["p", "q"], width=4)
    assert t.dtype == torch.int32 and t.tolist() == [[0, 1, 1, 1], [0, 1, 2, 2]]
    with pytest.raises(ValueError):
        c.attach_prefix("q", [5])
    c.assert_invariants()


def test_graph_bucket_selection_and_stats_on_cpu():
    m = DecodeGraphManager(device="cpu")
    assert [m.bucket_for(n) for n in (1, 2, 3, 4, 5, 8)] == [1, 2, 4, 4, 8, 8]
    assert m.bucket_for(9) is None and m.eligible(1) is False
    before = m.stats()
    m.record_fallback()
    assert m.stats_delta(before) == {"captures": 0, "replays": 0, "fallbacks": 1,
                                     "padded_slots": 0, "graph_pool_bytes": 0}
    out = m.run(lambda input_ids: input_ids + 1, {"input_ids": torch.arange(9).reshape(9, 1)})
    assert torch.equal(out, torch.arange(1, 10).reshape(9, 1))
    assert m.stats()["fallbacks"] == 2
    with pytest.raises(ValueError):
        DecodeGraphManager(device="cpu", buckets=(0, 2))


def test_context_lens_from_positions():
    pos = torch.tensor([4, 0, 9])
    act = torch.tensor([1.0, 1.0, 0.0])
    assert attention.context_lens_from_positions(pos, act).tolist() == [5, 1, 0]


def test_attention_interface_validation():
    c = make_cache()
    c.reserve("r", 4)
    q = torch.zeros(1, 4, 8, dtype=torch.float16)
    with pytest.raises(ValueError, match="invalid query shape"):
        attention.attention_for_request(q, c, 0, "r", 4, torch.zeros(2, dtype=torch.long))
    with pytest.raises(ValueError, match="multiple of KV heads"):
        attention.attention_for_request(torch.zeros(1, 3, 8), c, 0, "r", 4, torch.zeros(1))
    with pytest.raises(ValueError, match="Unknown attention backend"):
        attention.attention_for_request(q, c, 0, "r", 4, torch.zeros(1), backend="triton")


def test_workload_generators_are_deterministic_and_sized():
    a, b = workloads.c1_workload(), workloads.c1_workload()
    assert torch.equal(a.q, b.q) and torch.equal(a.block_tables, b.block_tables)
    assert a.k_pool.shape == (256, 16, 2, 64) and a.q.shape == (8, 14, 64)
    assert all(16 <= n <= 512 for n in a.context_lens.tolist())
    lens = workloads.c2_lengths()
    assert len(lens) == 64 and min(lens) >= 128 and max(lens) <= 4096
    w = workloads.c2_workload()
    pages = sum(math.ceil(n / 16) for n in lens)
    assert w.k_pool.shape[0] == math.ceil(1.25 * pages)
    # every sequence's pages are distinct physical blocks (no sharing in C2)
    used = [int(x) for b, n in enumerate(lens) for x in w.block_tables[b, :math.ceil(n / 16)]]
    assert len(used) == len(set(used))
    # algorithmic bytes: 1 KiB of K+V per token dominate
    assert abs(w.algorithmic_bytes() - sum(lens) * 1024) < 0.01 * sum(lens) * 1024


def test_c3_prefix_sharing_structure():
    w = workloads.c3_workload(groups=2, per_group=4)
    t = w.block_tables
    assert torch.equal(t[0, :128], t[3, :128]) and not torch.equal(t[0, :128], t[4, :128])
    assert w.unique_tokens < int(w.context_lens.sum())


def test_qwen25_15b_parameter_count():
    from flexengine_amd.model import Qwen2Config
    # 1.5437 B parameters with tied embeddings (public model card)
    assert abs(Qwen2Config().parameters - 1.5437e9) / 1.5437e9 < 0.005


def test_model_requires_gpu():
    from flexengine_amd.model import Qwen2Config, Qwen2Model
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Qwen2Model(Qwen2Config(num_hidden_layers=1, vocab_size=16), device="cpu")


def test_device_tables_need_a_gpu_cache():
    """The step path builds its block tables on the device (fe_gather_tables); a
    cache that does not live on a GPU refuses instead of filling them on the host."""
    cache = PagedKVCache(CacheLayout(1, 40, 4, 2, 8), device="cpu")
    cache.reserve("a", 6)
    with pytest.raises(RuntimeError, match="GPU"):
        cache.device_tables(["a"], 4)
