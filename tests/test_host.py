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


# --------------------------------------------------------------------------------------
# cache internals of this package's own design
# --------------------------------------------------------------------------------------

def test_free_ring_reuses_blocks_in_release_order():
    c = make_cache(6, 4)
    c.reserve("a", 8)          # blocks 0, 1
    c.reserve("b", 8)          # blocks 2, 3
    c.free_request("b")        # ring: 4, 5, 2, 3
    c.free_request("a")        # ring: 4, 5, 2, 3, 0, 1
    assert list(c.free) == [4, 5, 2, 3, 0, 1]
    c.reserve("c", 12)
    assert c.tables["c"] == [4, 5, 2]
    assert 3 in c.free and 4 not in c.free and 99 not in c.free
    c.assert_invariants()


def test_refs_are_read_only_and_count_pins():
    c = make_cache()
    c.reserve("a", 8)
    b = c.tables["a"][1]
    c.retain_block(b)
    c.retain_block(b)
    assert c.refs[b] == 3
    with pytest.raises(ValueError):
        c.refs[b] = 0
    with pytest.raises(ValueError):
        c.release_block(c.tables["a"][0])          # no pin on that block
    with pytest.raises(ValueError):
        c.retain_block(9)                          # free block
    with pytest.raises(ValueError):
        c.retain_block(-1)
    c.free_request("a")
    assert c.refs[b] == 2 and b not in c.free and c.free_blocks == 9
    c.release_block(b)
    c.release_block(b)
    assert b in c.free and c.free_blocks == 10
    c.assert_invariants()


def test_table_reorder_only_accepts_a_permutation_of_the_own_blocks():
    c = make_cache(12, 4)
    c.reserve("a", 12)
    c.reserve("b", 4)
    c.tables["a"] = list(reversed(c.tables["a"]))
    assert c.tables["a"] == [2, 1, 0]
    with pytest.raises(ValueError):
        c.tables["a"] = [2, 1, 3]          # 3 belongs to b
    with pytest.raises(ValueError):
        c.tables["a"] = [2, 1]
    assert c.tables["a"] == [2, 1, 0]
    c.assert_invariants()


def test_shared_block_write_is_refused_before_any_device_work():
    """tests/unit/test_prefix_cache.py:85: a request never writes a block it shares."""
    c = make_cache(12, 4)
    c.reserve("src", 8)
    c.attach_prefix("child", c.tables["src"])
    c.reserve("child", 9)
    with pytest.raises(RuntimeError, match="shared immutable"):
        c.write(0, "child", 0, torch.zeros(1, 2, 8, dtype=torch.float16),
                torch.zeros(1, 2, 8, dtype=torch.float16))
    with pytest.raises(ValueError):
        c.attach_prefix("x", [0, 0])
    with pytest.raises(ValueError):
        c.attach_prefix("y", [11])                  # never allocated
    with pytest.raises(ValueError):
        c.attach_prefix("child", [0])               # already has a table
    c.assert_invariants()


def test_page_table_matrix_grows_and_rows_are_reused():
    c = make_cache(400, 1)
    for i in range(40):                              # more rows than the first matrix
        c.reserve(f"r{i}", 3)
    c.reserve("r0", 100)                             # wider than the first matrix
    assert len(c.tables["r0"]) == 100 and c.tables["r1"] == [3, 4, 5]
    c.free_request("r5")
    c.reserve("new", 2)
    assert len(c.tables) == 40 and "r5" not in c.tables and "new" in c.tables
    assert c.available_slots("r5") == 0 and c.missing_blocks("new", 5) == 3
    t = c.block_table(["new", "r1"], width=4, pad_block=7)
    assert t.tolist() == [c.tables["new"] + [7, 7], [3, 4, 5, 7]]
    c.assert_invariants()


# --------------------------------------------------------------------------------------
# graph records own the workspaces their kernels recorded
# --------------------------------------------------------------------------------------

class _EagerRecorder(DecodeGraphManager):
    """Stands in for hipGraph capture on the CPU: the 'graph' re-runs decode on the
    staging tensors into the captured output, as a replayed graph would."""

    def eligible(self, active_count):
        return self.bucket_for(active_count) is not None

    def _record(self, decode, staging, mask):
        decode(**staging, active_mask=mask)                # warm-up
        out = decode(**staging, active_mask=mask)

        class _Rerun:
            def replay(self):
                out.copy_(decode(**staging, active_mask=mask))
        return _Rerun(), out, 0


def test_graph_records_keep_their_workspaces_when_the_library_replaces_them():
    from flexengine_amd import ops
    cpu = torch.device("cpu")
    recorded = {}

    def decode(input_ids, active_mask):
        rows = input_ids.shape[0]
        ws = ops.decode_workspace(cpu, rows << 20, kind="test-graph")
        ws[0] = rows
        recorded.setdefault(rows, ws.data_ptr())
        return (input_ids.float() + ws[0].float()) * active_mask

    m = _EagerRecorder(device="cpu")
    m.capture(1, decode, {"input_ids": torch.ones(1, 1)})
    # an eager batch of 16 rows replaces the per-device workspace with a larger one
    decode(torch.ones(16, 1), torch.ones(16, 1))
    m.capture(8, decode, {"input_ids": torch.ones(8, 1)})
    held1 = [t.data_ptr() for t in m.workspaces(1)]
    held8 = [t.data_ptr() for t in m.workspaces(8)]
    assert recorded[1] in held1                  # bucket 1's buffer is still owned
    assert recorded[1] != recorded[16] and recorded[16] in held8
    import gc
    gc.collect()
    assert [t.data_ptr() for t in m.workspaces(1)] == held1
    out = m.replay(1, {"input_ids": torch.tensor([[5.0]])})
    assert out.tolist() == [[6.0]]
    out = m.replay(5, {"input_ids": torch.arange(1.0, 6.0).reshape(5, 1)})
    assert out.tolist() == [[9.0], [10.0], [11.0], [12.0], [13.0]]   # + bucket rows (8)
    st = m.stats()
    assert st["captures"] == 2 and st["replays"] == 2 and st["padded_slots"] == 3


def test_replay_pads_with_zeros_and_a_zero_mask():
    m = _EagerRecorder(device="cpu")

    def decode(input_ids, positions, active_mask):
        return (input_ids.float() + positions.float()) * active_mask

    m.capture(4, decode, {"input_ids": torch.ones(4, 1, dtype=torch.long),
                          "positions": torch.ones(4, 1, dtype=torch.long)})
    addrs = m.staging_addresses(4)
    got = m.replay(3, {"input_ids": torch.tensor([[3], [7], [11]]),
                       "positions": torch.tensor([[2], [4], [6]])})
    assert got.tolist() == [[5.0], [11.0], [17.0]]
    assert m.staging_addresses(4) == addrs
    assert m._graphs[4].staging["input_ids"][3].item() == 0
    assert m._graphs[4].mask.reshape(-1).tolist() == [1.0, 1.0, 1.0, 0.0]
    with pytest.raises(ValueError):
        m.replay(3, {"input_ids": torch.zeros(3, 1, dtype=torch.long)})
    with pytest.raises(ValueError):
        m.replay(2, {"input_ids": torch.zeros(3, 1, dtype=torch.long),
                     "positions": torch.zeros(3, 1, dtype=torch.long)})
    with pytest.raises(ValueError):
        m.replay(1, {"input_ids": torch.zeros(1, 1, dtype=torch.long),
                     "positions": torch.zeros(1, 1, dtype=torch.long)})   # bucket 1 not captured
    with pytest.raises(ValueError):
        m.capture(3, decode, {"input_ids": torch.ones(3, 1)})             # not a bucket


def test_nested_workspace_scopes_close_by_identity():
    # the outer scope holds [A, B], the inner one [B, A]: closing the inner scope
    # must neither compare A with B elementwise nor remove the outer scope
    from flexengine_amd import ops
    cpu = torch.device("cpu")
    with ops.hold_workspaces() as outer:
        a = ops.decode_workspace(cpu, 4 << 20, kind="test-nest-a")
        b = ops.decode_workspace(cpu, 8 << 20, kind="test-nest-b")
        with ops.hold_workspaces() as inner:
            ops.decode_workspace(cpu, 8 << 20, kind="test-nest-b")
            ops.decode_workspace(cpu, 4 << 20, kind="test-nest-a")
            assert [t is x for t, x in zip(inner, (b, a))] == [True, True]
        assert ops._HOLDERS[-1] is outer
        assert not any(h is inner for h in ops._HOLDERS)
        # a scope equal to the outer one element by element closes itself only
        with ops.hold_workspaces() as same:
            ops.decode_workspace(cpu, 4 << 20, kind="test-nest-a")
            ops.decode_workspace(cpu, 8 << 20, kind="test-nest-b")
        assert ops._HOLDERS[-1] is outer and same == outer
    assert not any(h is outer for h in ops._HOLDERS)
