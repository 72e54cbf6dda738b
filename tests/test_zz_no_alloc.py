"""GPU: fe_paged_decode_noalloc -- the decode entry point that allocates nothing
(its split-K scratch is a static per-GPU device array) -- against
fe_paged_decode with a caller-owned workspace, through the C ABI.

The two share their kernels, so outputs and the fused page write must be
byte-identical; both are also held to the hot-path tolerance against the
float64 oracle.  Two calls in a row, the second on a smaller batch (the
scratch keeps the first call's partials), then a call that needs more scratch
than the array holds, which must be refused before anything is launched.
The captured form is checked first, so that in a process that runs this file
alone the first call on the device (which looks up the array and records its
ticket-clear kernel) happens inside the graph capture.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from flexengine_amd import _lib, ops, workloads
from oracle import paged_ref as R
from tests.parity import assert_attention_close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _args(d, out, k_new=True):
    nb, bs, hkv, hd = d.k_pool.shape
    return ((d.q.data_ptr(), d.q.stride(0), out.data_ptr(),
             d.k_new.data_ptr() if k_new else None, d.v_new.data_ptr() if k_new else None,
             d.k_new.stride(0) if k_new else 0, d.k_pool.data_ptr(), d.v_pool.data_ptr(), nb,
             d.block_tables.data_ptr(), d.block_tables.shape[1], d.context_lens.data_ptr()),
            (d.q.shape[0], d.q.shape[1], hkv, hd, bs, 1.0 / hd ** 0.5, 0,
             torch.cuda.current_stream().cuda_stream))


def _run_workspace_form(w):
    """(out, k_pool, v_pool) of fe_paged_decode with a fresh caller-owned workspace."""
    d = w.to(DEV)
    out = torch.full_like(d.q, float("nan"))
    head, tail = _args(d, out)
    need = ops.decode_workspace_bytes(w.batch, w.q.shape[1], w.q.shape[2],
                                      w.block_tables.shape[1] * w.block_size)
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    rc = _lib.load().fe_paged_decode(*head, ws.data_ptr(), need, *tail)
    assert rc == 0, _lib.error_string(rc)
    torch.cuda.synchronize()
    return out.cpu(), d.k_pool.cpu(), d.v_pool.cpu()


def _same_bits(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_aa_noalloc_decode_captured_in_a_graph_replays_like_the_workspace_form():
    """fe_paged_decode_noalloc recorded into a HIP graph (torch.cuda.graph) at C2 and
    replayed twice: each replay's output and fused page write byte-identical to the
    workspace form's.  Then eager calls after the first allocate nothing: the
    device's free memory is unchanged across them."""
    w = workloads.c2_workload()
    o_ws, k_ws, v_ws = _run_workspace_form(w)
    d = w.to(DEV)
    out = torch.full_like(d.q, float("nan"))
    lib = _lib.load()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        head, tail = _args(d, out)    # the capture stream is current here
        rc = lib.fe_paged_decode_noalloc(*head, *tail)
    assert rc == 0, _lib.error_string(rc)
    for rep in range(2):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert _same_bits(out.cpu(), o_ws), f"replay {rep}"
        assert _same_bits(d.k_pool.cpu(), k_ws) and _same_bits(d.v_pool.cpu(), v_ws), f"replay {rep}"
    del g
    head, tail = _args(d, out)
    assert lib.fe_paged_decode_noalloc(*head, *tail) == 0
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        assert lib.fe_paged_decode_noalloc(*head, *tail) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert _same_bits(out.cpu(), o_ws)


def _run_both(w):
    """(out, k_pool, v_pool) of fe_paged_decode and of fe_paged_decode_noalloc on
    separate device copies of the same workload."""
    lib = _lib.load()
    results = []
    for noalloc in (False, True):
        d = w.to(DEV)
        out = torch.full_like(d.q, float("nan"))
        head, tail = _args(d, out)
        if noalloc:
            rc = lib.fe_paged_decode_noalloc(*head, *tail)
        else:
            need = ops.decode_workspace_bytes(w.batch, w.q.shape[1], w.q.shape[2],
                                              w.block_tables.shape[1] * w.block_size)
            ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
            rc = lib.fe_paged_decode(*head, ws.data_ptr(), need, *tail)
        assert rc == 0, _lib.error_string(rc)
        torch.cuda.synchronize()
        results.append((out.cpu(), d.k_pool.cpu(), d.v_pool.cpu()))
    return results


def _check(w, what):
    (o_ws, k_ws, v_ws), (o_na, k_na, v_na) = _run_both(w)
    assert torch.equal(o_ws.view(torch.int16), o_na.view(torch.int16)), what
    assert torch.equal(k_ws.view(torch.int16), k_na.view(torch.int16)), what
    assert torch.equal(v_ws.view(torch.int16), v_na.view(torch.int16)), what
    kp, vp = w.k_pool.numpy().copy(), w.v_pool.numpy().copy()
    R.write_kv_decode(kp, vp, w.block_tables.numpy(), w.context_lens.numpy(), w.k_new.numpy(),
                      w.v_new.numpy(), w.block_size)
    exp = R.decode_reference(w.q.numpy(), kp, vp, w.block_tables.numpy(),
                             w.context_lens.numpy(), w.block_size)
    assert_attention_close(o_na.numpy(), exp, what=what)
    assert np.array_equal(k_na.numpy().view(np.int16), kp.view(np.int16)), what


def test_noalloc_decode_matches_the_workspace_entry_point_twice():
    """C2 (64 rows, contexts up to 4096, fused page write), then a smaller call
    (16 rows of another seed, G = 7 at D = 64) on the same scratch."""
    _check(workloads.c2_workload(), "noalloc C2")
    small = workloads.make_decode_workload("small", 21, 16, 14, 2, 64,
                                           [1, 17, 40, 129, 513, 700, 16, 3, 900, 64, 65, 2,
                                            1000, 333, 31, 5], with_new_kv=True)
    _check(small, "noalloc 16 rows")


def test_noalloc_decode_at_other_head_dims_and_groups_then_c2():
    """Head_dim 96 (the generic kernel: its key-split partials in the scratch past the
    split-K tickets) and a group of 32 split into virtual KV heads, each byte-identical
    to the workspace form; then C2 again on the same scratch, whose tickets the
    generic kernel has left at zero."""
    lens = [1, 90, 700, 4000, 33, 2048]
    _check(workloads.make_decode_workload("d96", 23, len(lens), 12, 2, 96, lens,
                                          with_new_kv=True), "noalloc D 96")
    _check(workloads.make_decode_workload("g32", 24, len(lens), 32, 1, 128, lens,
                                          with_new_kv=True), "noalloc group 32")
    _check(workloads.c2_workload(), "noalloc C2 after")


def test_noalloc_refuses_calls_beyond_its_scratch():
    """A call whose partials exceed the 16 MiB array returns FE_ERR_SCRATCH_LIMIT and
    launches nothing (the output keeps its contents)."""
    w = workloads.make_decode_workload("big", 22, 4, 12, 2, 128, [100, 200, 300, 400])
    d = w.to(DEV)
    out = torch.full_like(d.q, 7.0)
    head, tail = _args(d, out, k_new=False)
    lib = _lib.load()
    # 8192 pieces per KV head: (8192 + 4) * 12 * 128 * 4 bytes of partials > 16 MiB
    tail = tail[:6] + (8192,) + tail[7:]
    need = ops.decode_workspace_bytes(4, 12, 128, d.block_tables.shape[1] * 16, 8192)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.fe_paged_decode_noalloc(*head, *tail)
    assert rc == _lib.FE_ERR_SCRATCH_LIMIT, rc
    assert "16 MiB" in _lib.error_string(rc)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
