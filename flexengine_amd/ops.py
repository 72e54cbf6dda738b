"""Tensor-level wrappers around the C ABI (device memory and streams from PyTorch).

Every function validates shapes, dtypes and devices on the host, then makes one
asynchronous call into libfe_paged.so on the current HIP stream.  None of them
synchronises the host or allocates inside the library, so all of them may be
captured into a HIP graph (torch.cuda.graph) as long as the caller provides
the workspace / output buffers or lets them come from the graph pool.
"""
from __future__ import annotations

import contextlib
from dataclasses import dataclass
import functools
import math

import torch

from flexengine_amd import _lib

FP16 = torch.float16
BF16 = torch.bfloat16
FP32 = torch.float32
# K/V element types of the page movers, the decode and the prefill (the fe_*_bf16
# forms take bf16, the fe_*_f32 forms float32)
KV_DTYPES = (FP16, BF16, FP32)
# 16-bit types only: plans, the shared-prefix decode and the LSE merge's output
DTYPES_16 = (FP16, BF16)
_SFX = {FP16: "", BF16: "_bf16", FP32: "_f32"}
# the page movers copy bytes: one form for both 16-bit types, one for fp32
_MOVER_SFX = {FP16: "", BF16: "", FP32: "_f32"}


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            "flexengine_amd kernels run on a ROCm GPU only; got tensors on " + str(dev)
        )
    for t in tensors[1:]:
        if t is not None and t.device != dev:
            raise ValueError(f"all tensors must be on {dev}; got {t.device}")
    return dev


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


@functools.lru_cache(maxsize=4096)
def _pure_size(name: str, *args: int) -> int:
    """A workspace size that depends on its integer arguments only (memoised: a
    ctypes round trip per launch is host time the eager step pays)."""
    return int(getattr(_lib.load(), name)(*args))


def _stream(dev: torch.device) -> int:
    """The current HIP stream of `dev` (the raw handle: torch.cuda.current_stream
    builds a Stream object per call, ~4 us of host time on every launch)."""
    if _RAW_STREAM is not None and dev.index is not None:
        return _RAW_STREAM(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check_pool(k_pool: torch.Tensor, v_pool: torch.Tensor,
                dtypes: tuple = (FP16,)) -> tuple[int, int, int, int]:
    if k_pool.shape != v_pool.shape or k_pool.ndim != 4:
        raise ValueError("K/V pools must both be [num_blocks, block_size, kv_heads, head_dim]")
    if k_pool.dtype not in dtypes or v_pool.dtype != k_pool.dtype:
        names = " or ".join(str(t).replace("torch.", "") for t in dtypes)
        raise ValueError(f"K/V pools must be {names} (both the same)")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("K/V pools must be contiguous")
    nb, bs, hkv, d = k_pool.shape
    return nb, bs, hkv, d


def _int32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32 (convert once with .to(torch.int32))")
    return t.contiguous()


# ---------------------------------------------------------------------------------------
# KV page write / gather
# ---------------------------------------------------------------------------------------

def write_kv(k_new: torch.Tensor, v_new: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
             slot_block: torch.Tensor, slot_offset: torch.Tensor) -> None:
    """k_pool[slot_block[t], slot_offset[t]] = k_new[t] (and v); negative blocks are skipped."""
    dev = _require_gpu(k_new, v_new, k_pool, v_pool, slot_block, slot_offset)
    nb, bs, hkv, d = _check_pool(k_pool, v_pool, KV_DTYPES)
    if k_new.shape != v_new.shape or k_new.ndim != 3 or tuple(k_new.shape[1:]) != (hkv, d):
        raise ValueError("K/V shapes must be [tokens, kv_heads, head_dim]")
    if k_new.dtype != k_pool.dtype or v_new.dtype != k_pool.dtype:
        raise ValueError("wrong KV dtype")
    if k_new.stride() != v_new.stride() or k_new.stride(2) != 1 or k_new.stride(1) != d:
        raise ValueError("new K/V rows must have contiguous heads and equal strides")
    t = k_new.shape[0]
    slot_block, slot_offset = _int32(slot_block, "slot_block"), _int32(slot_offset, "slot_offset")
    if slot_block.shape != (t,) or slot_offset.shape != (t,):
        raise ValueError("slot arrays must be [tokens]")
    _lib.call("fe_write_kv" + _MOVER_SFX[k_pool.dtype], k_new.data_ptr(), v_new.data_ptr(),
              k_new.stride(0),
              k_pool.data_ptr(), v_pool.data_ptr(), nb, slot_block.data_ptr(),
              slot_offset.data_ptr(), t, hkv, d, bs, _stream(dev))


def write_kv_ragged(k_new: torch.Tensor, v_new: torch.Tensor, k_pool: torch.Tensor,
                    v_pool: torch.Tensor, block_tables: torch.Tensor, q_offsets: torch.Tensor,
                    context_lens: torch.Tensor) -> None:
    """Writes the new rows of ragged chunks with the slot map computed on the device:
    rows q_offsets[s]..q_offsets[s+1]-1 are the last positions of sequence s's
    context_lens[s] tokens (the arrays prefill_paged takes; fe_write_kv_ragged)."""
    dev = _require_gpu(k_new, v_new, k_pool, v_pool, block_tables, q_offsets, context_lens)
    nb, bs, hkv, d = _check_pool(k_pool, v_pool, KV_DTYPES)
    if k_new.shape != v_new.shape or k_new.ndim != 3 or tuple(k_new.shape[1:]) != (hkv, d):
        raise ValueError("K/V shapes must be [tokens, kv_heads, head_dim]")
    if k_new.dtype != k_pool.dtype or v_new.dtype != k_pool.dtype:
        raise ValueError("wrong KV dtype")
    if k_new.stride() != v_new.stride() or k_new.stride(2) != 1 or k_new.stride(1) != d:
        raise ValueError("new K/V rows must have contiguous heads and equal strides")
    block_tables = _int32(block_tables, "block_tables")
    q_offsets, context_lens = _int32(q_offsets, "q_offsets"), _int32(context_lens, "context_lens")
    s = context_lens.shape[0]
    if block_tables.ndim != 2 or block_tables.shape[0] != s or q_offsets.shape != (s + 1,):
        raise ValueError("block_tables must be [S, W], q_offsets [S+1], context_lens [S]")
    _lib.call("fe_write_kv_ragged" + _MOVER_SFX[k_pool.dtype], k_new.data_ptr(), v_new.data_ptr(),
              k_new.stride(0),
              k_pool.data_ptr(), v_pool.data_ptr(), nb, block_tables.data_ptr(),
              block_tables.shape[1], q_offsets.data_ptr(), context_lens.data_ptr(), s,
              k_new.shape[0], hkv, d, bs, _stream(dev))


def gather_tables(mirror: torch.Tensor, row_len: torch.Tensor, rows: torch.Tensor, width: int,
                  pad_block: int = -1) -> torch.Tensor:
    """int32 [len(rows), width] block tables from the device mirror rows (fe_gather_tables);
    entries past a row's length are pad_block, or its last block when pad_block < 0."""
    dev = _require_gpu(mirror, row_len, rows)
    mirror, row_len, rows = _int32(mirror, "mirror"), _int32(row_len, "row_len"), _int32(rows, "rows")
    if mirror.ndim != 2 or row_len.shape != (mirror.shape[0],) or rows.ndim != 1:
        raise ValueError("mirror must be [R, M], row_len [R], rows [B]")
    width = max(int(width), 1)
    out = torch.empty((rows.shape[0], width), dtype=torch.int32, device=dev)
    _lib.call("fe_gather_tables", mirror.data_ptr(), mirror.shape[1], row_len.data_ptr(),
              mirror.shape[0], rows.data_ptr(), rows.shape[0], width, int(pad_block),
              out.data_ptr(), width, _stream(dev))
    return out


def write_kv_decode(k_new: torch.Tensor, v_new: torch.Tensor, k_pool: torch.Tensor,
                    v_pool: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor) -> None:
    """Writes row b at position context_lens[b]-1 of sequence b; rows with length 0 are skipped."""
    dev = _require_gpu(k_new, v_new, k_pool, v_pool, block_tables, context_lens)
    nb, bs, hkv, d = _check_pool(k_pool, v_pool, KV_DTYPES)
    batch = k_new.shape[0]
    if k_new.shape != v_new.shape or tuple(k_new.shape[1:]) != (hkv, d):
        raise ValueError("K/V shapes must be [batch, kv_heads, head_dim]")
    if k_new.dtype != k_pool.dtype or v_new.dtype != k_pool.dtype:
        raise ValueError("wrong KV dtype")
    if k_new.stride() != v_new.stride() or k_new.stride(2) != 1 or k_new.stride(1) != d:
        raise ValueError("new K/V rows must have contiguous heads and equal strides")
    block_tables = _int32(block_tables, "block_tables")
    context_lens = _int32(context_lens, "context_lens")
    if block_tables.ndim != 2 or block_tables.shape[0] != batch or context_lens.shape != (batch,):
        raise ValueError("block_tables must be [batch, W] and context_lens [batch]")
    _lib.call("fe_write_kv_decode" + _MOVER_SFX[k_pool.dtype], k_new.data_ptr(), v_new.data_ptr(),
              k_new.stride(0),
              k_pool.data_ptr(), v_pool.data_ptr(), nb, block_tables.data_ptr(),
              block_tables.shape[1], context_lens.data_ptr(), batch, hkv, d, bs, _stream(dev))


def gather_kv(k_pool: torch.Tensor, v_pool: torch.Tensor, block_tables: torch.Tensor,
              context_lens: torch.Tensor, out_offsets: torch.Tensor,
              total_tokens: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Materialises every sequence's K/V rows: returns [total_tokens, kv_heads, head_dim] pair."""
    dev = _require_gpu(k_pool, v_pool, block_tables, context_lens, out_offsets)
    nb, bs, hkv, d = _check_pool(k_pool, v_pool, KV_DTYPES)
    block_tables = _int32(block_tables, "block_tables")
    context_lens = _int32(context_lens, "context_lens")
    out_offsets = _int32(out_offsets, "out_offsets")
    batch = context_lens.shape[0]
    if block_tables.ndim != 2 or block_tables.shape[0] != batch or out_offsets.shape != (batch + 1,):
        raise ValueError("block_tables [batch, W], context_lens [batch], out_offsets [batch+1]")
    k_out = torch.empty((total_tokens, hkv, d), dtype=k_pool.dtype, device=dev)
    v_out = torch.empty_like(k_out)
    _lib.call("fe_gather_kv" + _MOVER_SFX[k_pool.dtype], k_pool.data_ptr(), v_pool.data_ptr(), nb,
              block_tables.data_ptr(),
              block_tables.shape[1], context_lens.data_ptr(), out_offsets.data_ptr(),
              k_out.data_ptr(), v_out.data_ptr(), batch, total_tokens, hkv, d, bs, _stream(dev))
    return k_out, v_out


# ---------------------------------------------------------------------------------------
# decode
# ---------------------------------------------------------------------------------------

_WORKSPACES: dict[tuple, torch.Tensor] = {}
# open hold_workspaces() scopes, innermost last
_HOLDERS: list[list[torch.Tensor]] = []


@contextlib.contextmanager
def hold_workspaces():
    """Collects every workspace decode_workspace() hands out inside the block.

    A per-device workspace is replaced by a larger one when a call needs more
    bytes, and the old buffer returns to the caching allocator once nothing
    references it.  Work recorded into a HIP graph keeps the old address, so a
    caller that captures kernels keeps the collected list for as long as the
    graph may be replayed."""
    held: list[torch.Tensor] = []
    _HOLDERS.append(held)
    try:
        yield held
    finally:
        # by identity: list equality would compare the held tensors elementwise
        for i in range(len(_HOLDERS) - 1, -1, -1):
            if _HOLDERS[i] is held:
                del _HOLDERS[i]
                break


def decode_workspace_bytes(batch: int, num_q_heads: int, head_dim: int, max_context: int,
                           target_splits: int = 0) -> int:
    """Workspace bytes for fe_paged_decode; max_context = table width * block size."""
    return int(_lib.load().fe_paged_decode_workspace_size(batch, num_q_heads, head_dim,
                                                          max_context, target_splits))


def decode_workspace(device: torch.device, nbytes: int, kind: str = "decode") -> torch.Tensor:
    """A per-device workspace reused by every decode (or, kind="prefill", prefill)
    call on that device.

    Calls on one stream are ordered, so sharing is safe there; callers running
    these kernels on several streams at once must pass their own zero-filled
    workspace.  A larger request replaces the buffer; see hold_workspaces() for
    callers that record the kernels into a graph.
    """
    key = (device.type, device.index, kind)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        # zero-filled once: the split-K tickets at its start must begin at zero
        # (every call leaves them at zero again)
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    for held in _HOLDERS:
        if not any(t is ws for t in held):
            held.append(ws)
    return ws


def _decode_args(q, k_pool, v_pool, block_tables, context_lens, scale, k_new, v_new, out):
    """Checks of the decode entry points; returns the normalised arguments."""
    dev = _require_gpu(q, k_pool, v_pool, block_tables, context_lens, k_new, v_new, out)
    nb, bs, hkv, d = _check_pool(k_pool, v_pool, KV_DTYPES)
    dt = k_pool.dtype
    if q.ndim != 3 or q.shape[2] != d or q.dtype != dt:
        raise ValueError("q must be [batch, num_q_heads, head_dim] of the pools' dtype")
    batch, hq, _ = q.shape
    if q.stride(2) != 1 or q.stride(1) != d:
        raise ValueError("q heads must be contiguous")
    if hq % hkv:
        raise ValueError("Q heads must be a multiple of KV heads")
    block_tables = _int32(block_tables, "block_tables")
    context_lens = _int32(context_lens, "context_lens")
    if block_tables.ndim != 2 or block_tables.shape[0] != batch or context_lens.shape != (batch,):
        raise ValueError("block_tables must be [batch, W] and context_lens [batch]")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new must be given together")
    new_stride = 0
    if k_new is not None:
        if k_new.shape != (batch, hkv, d) or v_new.shape != k_new.shape:
            raise ValueError("k_new/v_new must be [batch, kv_heads, head_dim]")
        if k_new.dtype != dt or v_new.dtype != dt:
            raise ValueError("k_new/v_new must have the pools' dtype")
        if k_new.stride() != v_new.stride() or k_new.stride(2) != 1 or k_new.stride(1) != d:
            raise ValueError("k_new/v_new heads must be contiguous with equal strides")
        new_stride = k_new.stride(0)
    if out is None:
        out = torch.empty((batch, hq, d), dtype=dt, device=dev)
    elif out.shape != (batch, hq, d) or out.dtype != dt or not out.is_contiguous():
        raise ValueError("out must be a contiguous [batch, num_q_heads, head_dim] of q's dtype")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    return dev, nb, bs, hkv, d, batch, hq, block_tables, context_lens, new_stride, out, scale


@dataclass(frozen=True)
class DecodePlan:
    """A decode step's split-K partition and block rows (fe_paged_decode_plan),
    for the block_tables / context_lens tensors it was computed from."""
    buffer: torch.Tensor
    tables_ptr: int
    lens_ptr: int
    shape: tuple  # (batch, kv_heads, table width, block size, num_blocks, target_splits)


def paged_decode_plan(block_tables: torch.Tensor, context_lens: torch.Tensor, num_blocks: int,
                      kv_heads: int, block_size: int, *, target_splits: int = 0,
                      out: DecodePlan | None = None) -> DecodePlan:
    """Computes the plan every layer's paged_decode(..., plan=) of one decode step
    reuses (the tables and lengths must not change between those calls).
    `out` reuses an earlier plan's buffer for the same sizes (graph capture)."""
    dev = _require_gpu(block_tables, context_lens)
    block_tables = _int32(block_tables, "block_tables")
    context_lens = _int32(context_lens, "context_lens")
    batch, width = block_tables.shape
    shape = (batch, int(kv_heads), width, int(block_size), int(num_blocks), int(target_splits))
    need = int(_lib.load().fe_paged_decode_plan_size(batch, int(kv_heads), width * block_size,
                                                      int(target_splits)))
    if out is not None:
        if out.shape != shape:
            raise ValueError(f"plan buffer is for sizes {out.shape}, not {shape}")
        buffer = out.buffer
    else:
        buffer = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    _lib.call("fe_paged_decode_plan", block_tables.data_ptr(), width, context_lens.data_ptr(),
              int(num_blocks), batch, int(kv_heads), int(block_size), int(target_splits),
              buffer.data_ptr(), buffer.numel(), _stream(dev))
    return DecodePlan(buffer, block_tables.data_ptr(), context_lens.data_ptr(), shape)


def paged_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                 block_tables: torch.Tensor, context_lens: torch.Tensor, *,
                 scale: float | None = None, k_new: torch.Tensor | None = None,
                 v_new: torch.Tensor | None = None, out: torch.Tensor | None = None,
                 workspace: torch.Tensor | None = None, target_splits: int = 0,
                 plan: DecodePlan | None = None) -> torch.Tensor:
    """Single-token paged decode attention over one layer's pools.

    q [B, Hq, D] fp16, bf16 or float32, the pools' dtype (rows may be strided,
    heads contiguous); pools [NB, BS, Hkv, D]; block_tables int32 [B, W];
    context_lens int32 [B] (0 = inactive row -> zeros).  With k_new/v_new
    ([B, Hkv, D]) the new token's K/V are written to the pool at position
    context_lens-1 in the same launch.  With `plan` (paged_decode_plan on these
    block_tables / context_lens; 16-bit pools) the launch reads the partition and
    first block rows from it (fe_paged_decode_planned); same results.
    """
    (dev, nb, bs, hkv, d, batch, hq, block_tables, context_lens, new_stride, out,
     scale) = _decode_args(q, k_pool, v_pool, block_tables, context_lens, scale, k_new, v_new, out)
    need = decode_workspace_bytes(batch, hq, d, block_tables.shape[1] * bs, target_splits)
    if workspace is None:
        workspace = decode_workspace(dev, need)
    args = (q.data_ptr(), q.stride(0), out.data_ptr(), _ptr(k_new), _ptr(v_new), new_stride,
            k_pool.data_ptr(), v_pool.data_ptr(), nb, block_tables.data_ptr(),
            block_tables.shape[1], context_lens.data_ptr(), workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), batch, hq, hkv, d, bs, float(scale),
            int(target_splits))
    sfx = _SFX[q.dtype]
    if plan is None:
        _lib.call("fe_paged_decode" + sfx, *args, _stream(dev))
        return out
    if q.dtype not in DTYPES_16:
        raise ValueError("decode plans are for fp16 / bf16 pools (the fp32 decode has none)")
    shape = (batch, hkv, block_tables.shape[1], bs, nb, int(target_splits))
    if plan.shape != shape or plan.tables_ptr != block_tables.data_ptr() or \
            plan.lens_ptr != context_lens.data_ptr():
        raise ValueError("the plan was computed for other block_tables / context_lens or sizes")
    _lib.call("fe_paged_decode_planned" + sfx, *args, plan.buffer.data_ptr(),
              plan.buffer.numel(), _stream(dev))
    return out


def paged_decode_shared_prefix(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                               block_tables: torch.Tensor, context_lens: torch.Tensor,
                               group_offsets: torch.Tensor, group_prefix_lens: torch.Tensor, *,
                               scale: float | None = None, k_new: torch.Tensor | None = None,
                               v_new: torch.Tensor | None = None,
                               out: torch.Tensor | None = None,
                               workspace: torch.Tensor | None = None,
                               target_splits: int = 0) -> torch.Tensor:
    """paged_decode for a batch whose sequences form groups sharing prefix blocks.

    Group s is the batch rows group_offsets[s] .. group_offsets[s+1]-1 (int32
    [S+1], ascending; rows outside every group decode normally); its first
    group_prefix_lens[s] keys (int32 [S], rounded down to whole blocks) are the
    blocks at the start of row group_offsets[s]'s table, shared by every member.
    Same result as paged_decode: the shared keys are attended once per group,
    the private suffixes per row, merged by log-sum-exp (fe_paged_decode_shared_prefix,
    or its _bf16 / _f32 form for bfloat16 / float32 q and pools).
    """
    (dev, nb, bs, hkv, d, batch, hq, block_tables, context_lens, new_stride, out,
     scale) = _decode_args(q, k_pool, v_pool, block_tables, context_lens, scale, k_new, v_new, out)
    group_offsets = _int32(group_offsets, "group_offsets")
    group_prefix_lens = _int32(group_prefix_lens, "group_prefix_lens")
    if group_offsets.ndim != 1 or group_prefix_lens.ndim != 1 or \
            group_offsets.shape[0] != group_prefix_lens.shape[0] + 1:
        raise ValueError("group_offsets must be [S+1] and group_prefix_lens [S]")
    if group_offsets.device != dev or group_prefix_lens.device != dev:
        raise ValueError("group arrays must be on the GPU")
    ngroups = group_prefix_lens.shape[0]
    need = int(_lib.load().fe_paged_decode_shared_prefix_workspace_size(
        batch, hq, hkv, d, block_tables.shape[1] * bs, ngroups, int(target_splits)))
    if workspace is None:
        workspace = decode_workspace(dev, need)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace too small: need {need} bytes")
    _lib.call("fe_paged_decode_shared_prefix" + _SFX[q.dtype], q.data_ptr(), q.stride(0),
              out.data_ptr(),
              _ptr(k_new), _ptr(v_new), new_stride, k_pool.data_ptr(), v_pool.data_ptr(), nb,
              block_tables.data_ptr(), block_tables.shape[1], context_lens.data_ptr(),
              group_offsets.data_ptr(), group_prefix_lens.data_ptr(), ngroups,
              workspace.data_ptr(), workspace.numel() * workspace.element_size(), batch, hq, hkv,
              d, bs, float(scale), int(target_splits), _stream(dev))
    return out


def lse_merge(part_out: torch.Tensor, part_lse: torch.Tensor, with_lse: bool = False,
              dtype: torch.dtype = FP16) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Merges S split results: part_out fp32 [S, R, D], part_lse fp32 [S, R] (natural log);
    the output [R, D] in `dtype` (float16: fe_lse_merge, bfloat16: fe_lse_merge_bf16)."""
    if dtype not in DTYPES_16:
        raise ValueError("the merged output is float16 or bfloat16")
    dev = _require_gpu(part_out, part_lse)
    if part_out.ndim != 3 or part_lse.shape != part_out.shape[:2]:
        raise ValueError("part_out must be [S, R, D] and part_lse [S, R]")
    if part_out.dtype != torch.float32 or part_lse.dtype != torch.float32:
        raise ValueError("partials must be float32")
    part_out, part_lse = part_out.contiguous(), part_lse.contiguous()
    s, r, d = part_out.shape
    out = torch.empty((r, d), dtype=dtype, device=dev)
    out_lse = torch.empty((r,), dtype=torch.float32, device=dev) if with_lse else None
    sfx = "_bf16" if dtype == BF16 else ""
    _lib.call("fe_lse_merge" + sfx, part_out.data_ptr(), part_lse.data_ptr(), s, r, d, out.data_ptr(),
              _ptr(out_lse), _stream(dev))
    return (out, out_lse) if with_lse else out


# ---------------------------------------------------------------------------------------
# prefill
# ---------------------------------------------------------------------------------------

@dataclass(frozen=True)
class PrefillPlan:
    """A step's stream-K prefill work split (fe_prefill_plan), for the tensors
    and sizes it was computed from."""
    buffer: torch.Tensor
    q_offsets_ptr: int
    lens_ptr: int
    shape: tuple  # (num_seqs, total_q, num_q_heads, kv_heads, table_stride, block_size)


def prefill_paged_plan(q_offsets: torch.Tensor, context_lens: torch.Tensor, total_q: int,
                       num_q_heads: int, kv_heads: int, table_stride: int, block_size: int, *,
                       out: PrefillPlan | None = None) -> PrefillPlan | None:
    """The work split every layer's prefill_paged(..., plan=) of one step reuses (the
    offsets and lengths must not change between those calls); None when the sizes
    take the tile kernel, which has no plan.  `out` reuses an earlier plan's buffer."""
    dev = _require_gpu(q_offsets, context_lens)
    q_offsets = _int32(q_offsets, "q_offsets")
    context_lens = _int32(context_lens, "context_lens")
    num_seqs = context_lens.shape[0]
    shape = (num_seqs, int(total_q), int(num_q_heads), int(kv_heads), int(table_stride),
             int(block_size))
    need = int(_lib.load().fe_prefill_plan_size(num_seqs, int(total_q), int(num_q_heads),
                                                int(kv_heads)))
    if out is not None:
        if out.shape != shape:
            raise ValueError(f"plan buffer is for sizes {out.shape}, not {shape}")
        buffer = out.buffer
    else:
        buffer = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    rc = _lib.load().fe_prefill_plan(q_offsets.data_ptr(), context_lens.data_ptr(), num_seqs,
                                     int(total_q), int(num_q_heads), int(kv_heads),
                                     int(table_stride), int(block_size), buffer.data_ptr(),
                                     buffer.numel(), _stream(dev))
    if rc == _lib.FE_ERR_UNSUPPORTED:
        return None
    _lib.check("fe_prefill_plan", rc)
    return PrefillPlan(buffer, q_offsets.data_ptr(), context_lens.data_ptr(), shape)


# a planned launch's verdict on its plan (include/flexengine_amd.h FE_PLAN_ERR_*)
PLAN_ERR_SIZES = 1   # other sizes or other block_tables / q_offsets / context_lens tensors
PLAN_ERR_STALE = 2   # the lengths changed after the plan was computed
_PLAN_ERROR_OFFSET = {"DecodePlan": 60, "PrefillPlan": 124}


def plan_error(plan: DecodePlan | PrefillPlan) -> int:
    """The plan's error word as the planned launches since the plan call left it:
    0, PLAN_ERR_SIZES or PLAN_ERR_STALE (those launches wrote NaN instead of using
    the plan).  Reads the word back from the device, after the stream's work."""
    off = _PLAN_ERROR_OFFSET[type(plan).__name__]
    return int(plan.buffer[off:off + 4].view(torch.int32).item())


def prefill_paged(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                  block_tables: torch.Tensor, q_offsets: torch.Tensor,
                  context_lens: torch.Tensor, max_q_len: int, *, scale: float | None = None,
                  out: torch.Tensor | None = None,
                  plan: PrefillPlan | None = None) -> torch.Tensor:
    """Ragged causal prefill: q [total_q, Hq, D]; sequence s owns rows
    q_offsets[s]:q_offsets[s+1] at positions context_lens[s]-n_s .. context_lens[s]-1.
    fp16, bf16 or float32 (q, out and the pools alike).  With `plan`
    (prefill_paged_plan on these q_offsets / context_lens and sizes; 16-bit pools)
    the launch reads its work split from it (fe_prefill_paged_planned); same results."""
    dev = _require_gpu(q, k_pool, v_pool, block_tables, q_offsets, context_lens, out)
    nb, bs, hkv, d = _check_pool(k_pool, v_pool, KV_DTYPES)
    if q.ndim != 3 or q.shape[2] != d or q.dtype != k_pool.dtype or not q.is_contiguous():
        raise ValueError("q must be a contiguous [total_q, num_q_heads, head_dim] of the pools' dtype")
    total_q, hq, _ = q.shape
    if hq % hkv:
        raise ValueError("Q heads must be a multiple of KV heads")
    block_tables = _int32(block_tables, "block_tables")
    q_offsets = _int32(q_offsets, "q_offsets")
    context_lens = _int32(context_lens, "context_lens")
    num_seqs = context_lens.shape[0]
    if q_offsets.shape != (num_seqs + 1,) or block_tables.ndim != 2 or block_tables.shape[0] != num_seqs:
        raise ValueError("q_offsets [S+1], block_tables [S, W], context_lens [S]")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of q's shape and dtype")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    need = int(_lib.load().fe_prefill_workspace_size(num_seqs, total_q, hq, hkv, d))
    ws = decode_workspace(dev, need, kind="prefill")
    args = (q.data_ptr(), out.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), nb,
            block_tables.data_ptr(), block_tables.shape[1], q_offsets.data_ptr(),
            context_lens.data_ptr(), num_seqs, total_q, int(max_q_len), hq, hkv, d, bs,
            float(scale), ws.data_ptr(), ws.numel())
    sfx = _SFX[q.dtype]
    if plan is None:
        _lib.call("fe_prefill_paged" + sfx, *args, _stream(dev))
        return out
    if q.dtype not in DTYPES_16:
        raise ValueError("prefill plans are for fp16 / bf16 pools (the fp32 prefill has none)")
    shape = (num_seqs, total_q, hq, hkv, block_tables.shape[1], bs)
    if plan.shape != shape or plan.q_offsets_ptr != q_offsets.data_ptr() or \
            plan.lens_ptr != context_lens.data_ptr():
        raise ValueError("the plan was computed for other q_offsets / context_lens or sizes")
    _lib.call("fe_prefill_paged_planned" + sfx, *args, plan.buffer.data_ptr(),
              plan.buffer.numel(), _stream(dev))
    return out


# ---------------------------------------------------------------------------------------
# decoder-layer kernels (include/flexengine_amd_model.h)
# ---------------------------------------------------------------------------------------

SKINNY_MAX_ROWS = 32


def _source(t: torch.Tensor) -> tuple[int, int, int, int, int]:
    """(ptr, row stride, splits, rows, cols) of a sourced input: fp16 rows [rows, cols]
    (unit column stride) or fp32 skinny-GEMM partials [splits, rows, cols]."""
    if t.dtype == torch.float32:
        if t.ndim != 3 or not t.is_contiguous():
            raise ValueError("partials must be contiguous float32 [splits, rows, cols]")
        s, rows, cols = t.shape
        return t.data_ptr(), cols, s, rows, cols
    if t.dtype != FP16 or t.ndim != 2 or t.stride(1) != 1:
        raise ValueError("input must be float16 [rows, cols] with unit column stride")
    return t.data_ptr(), t.stride(0), 0, t.shape[0], t.shape[1]


def gemm_skinny(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fp32 partial products [splits, M, N] of x [M, K] @ weight[N, K]^T (M <= 32);
    consumers (rmsnorm, rope_qkv, silu_mul) sum the splits."""
    dev = _require_gpu(x, weight)
    if x.ndim != 2 or weight.ndim != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("x [M, K] and weight [N, K] required")
    if x.dtype != FP16 or weight.dtype != FP16 or not x.is_contiguous() or not weight.is_contiguous():
        raise ValueError("x and weight must be contiguous float16")
    m, k = x.shape
    n = weight.shape[0]
    splits = int(_lib.load().fe_gemm_skinny_splits(n, k))
    part = torch.empty((splits, m, n), dtype=torch.float32, device=dev)
    _lib.call("fe_gemm_skinny", x.data_ptr(), m, k, weight.data_ptr(), n, part.data_ptr(), splits,
              _stream(dev))
    return part


ROWS64_MAX_ROWS = 64
# fe_gemm_rows64 is taken only for deep projections (K >= ROWS64_MIN_DEPTH * N): there
# few output tiles leave the library GEMM's grid a fraction of the chip, while the
# rows kernel splits K over it (Qwen2.5-1.5B down projection at 64 rows: 21.4 us vs
# 25.6 us).  For wide outputs (q/k/v, o, gate/up, LM head) the library GEMM measured
# 10-45% faster at 64 rows.
ROWS64_MIN_DEPTH = 4
# Outside graph capture a 64-row step is bound by the host's launch rate: a library
# GEMM call costs ~20 us of host time against ~4 us for the HIP kernel, which then
# wins on every projection although its kernel is up to ~30% slower on wide outputs;
# inside a captured graph the launches are paid once and the kernel time decides.
# Outputs wider than this (the LM head: the step's last launch, whose kernel time the
# host waits out) stay on the library GEMM.
ROWS64_EAGER_MAX_N = 32768


def gemm_rows64(x: torch.Tensor, weight: torch.Tensor,
                bias: torch.Tensor | None = None) -> torch.Tensor:
    """fp16(x @ weight^T + bias) [M, N] for M <= 64 rows (fe_gemm_rows64: the
    workgroup's four weight tiles share each x chunk through LDS)."""
    dev = _require_gpu(x, weight, bias)
    if x.ndim != 2 or weight.ndim != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("x [M, K] and weight [N, K] required")
    if x.dtype != FP16 or weight.dtype != FP16 or not weight.is_contiguous():
        raise ValueError("x and weight must be float16, weight contiguous")
    if bias is not None and (bias.shape != (weight.shape[0],) or bias.dtype != FP16):
        raise ValueError("bias must be float16 [N]")
    x = x.contiguous()
    m, k = x.shape
    n = weight.shape[0]
    out = torch.empty((m, n), dtype=FP16, device=dev)
    need = _pure_size("fe_gemm_rows64_workspace_size", m, n, k)
    ws = decode_workspace(dev, need, kind="rows64")
    _lib.call("fe_gemm_rows64", x.data_ptr(), m, k, weight.data_ptr(), n, _ptr(bias),
              out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """x @ weight^T (+ bias): the skinny HIP GEMM's fp32 partials (bias left to the
    consumer) for at most SKINNY_MAX_ROWS rows, fe_gemm_rows64 in fp16 (bias added)
    up to ROWS64_MAX_ROWS rows when K >= ROWS64_MIN_DEPTH * N or, outside graph
    capture, N <= ROWS64_EAGER_MAX_N; the library GEMM in fp16 otherwise."""
    if x.shape[0] <= SKINNY_MAX_ROWS and x.shape[1] % 32 == 0:
        return gemm_skinny(x.contiguous(), weight)
    if x.shape[0] <= ROWS64_MAX_ROWS and x.shape[1] % 32 == 0:
        if x.shape[1] >= ROWS64_MIN_DEPTH * weight.shape[0]:
            return gemm_rows64(x, weight, bias)
        if weight.shape[0] <= ROWS64_EAGER_MAX_N and not torch.cuda.is_current_stream_capturing():
            _warm_library_gemm(x, weight)
            return gemm_rows64(x, weight, bias)
    return torch.nn.functional.linear(x, weight, bias)


_LIBRARY_GEMM_WARM: set = set()


def _warm_library_gemm(x: torch.Tensor, weight: torch.Tensor) -> None:
    """One eager library GEMM per device and dtype before the eager path stops using
    it: a graph captured later takes the library GEMM for these shapes, and its
    first use must not fall inside the capture (the library sets itself up then)."""
    key = (x.device, x.dtype)
    if key not in _LIBRARY_GEMM_WARM:
        torch.nn.functional.linear(x[:1], weight[:16])
        _LIBRARY_GEMM_WARM.add(key)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """(weight * norm(x + residual), x + residual); with residual=None the second
    value is None.  x is fp16 [rows, hidden] or skinny partials; the residual is
    updated in place."""
    ptr, _, splits, rows, hidden = _source(x)
    dev = _require_gpu(x, weight, residual)
    out = torch.empty((rows, hidden), dtype=FP16, device=dev)
    if residual is not None and (residual.shape != (rows, hidden) or not residual.is_contiguous()):
        raise ValueError("residual must be a contiguous [rows, hidden] tensor")
    _lib.call("fe_rmsnorm", ptr, splits, _ptr(residual), _ptr(residual), weight.data_ptr(),
              out.data_ptr(), rows, hidden, float(eps), _stream(dev))
    return out, residual


def rope_qkv(qkv: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor, num_q_heads: int,
             kv_heads: int, head_dim: int, bias: torch.Tensor | None = None):
    """Splits a fused [q | k | v] projection into q [rows, Hq, D], k, v [rows, Hkv, D]
    with RoPE applied to q and k (positions int64 [rows])."""
    ptr, stride, splits, rows, cols = _source(qkv)
    if cols != (num_q_heads + 2 * kv_heads) * head_dim:
        raise ValueError("qkv width does not match the head configuration")
    dev = _require_gpu(qkv, positions, inv_freq, bias)
    if positions.dtype != torch.int64 or positions.shape != (rows,):
        raise ValueError("positions must be int64 [rows]")
    q = torch.empty((rows, num_q_heads, head_dim), dtype=FP16, device=dev)
    k = torch.empty((rows, kv_heads, head_dim), dtype=FP16, device=dev)
    v = torch.empty_like(k)
    _lib.call("fe_rope_qkv", ptr, stride, splits, _ptr(bias) if splits else None,
              positions.data_ptr(), inv_freq.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
              rows, num_q_heads, kv_heads, head_dim, _stream(dev))
    return q, k, v


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up over a fused [gate | up] input -> [rows, I]."""
    ptr, stride, splits, rows, cols = _source(gate_up)
    dev = _require_gpu(gate_up)
    inter = cols // 2
    out = torch.empty((rows, inter), dtype=FP16, device=dev)
    _lib.call("fe_silu_mul", ptr, stride, splits, out.data_ptr(), rows, inter, _stream(dev))
    return out


# ---------------------------------------------------------------------------------------
# fused decode-step projections (fe_gemm_f16 / _resid / _silu / _rope)
# ---------------------------------------------------------------------------------------

class Normed:
    """The operand of a fused projection given as its RMSNorm inputs: the residual
    stream r [M, K] fp16, the per-tile sums of r^2 [tiles, M] fp32 that
    gemm_resid wrote with it, the norm weight [K] and eps."""

    def __init__(self, r: torch.Tensor, ss: torch.Tensor, weight: torch.Tensor, eps: float):
        if ss.dtype != torch.float32 or ss.ndim != 2 or ss.shape[1] != r.shape[0]:
            raise ValueError("ss must be float32 [tiles, rows]")
        self.r, self.ss, self.weight, self.eps = r, ss, weight, float(eps)


def _operand(x, weight: torch.Tensor):
    """(x ptr, ss ptr, ss tiles, norm weight ptr, eps, M, K) of a plain fp16 operand
    or a Normed one, checked against weight [N, K]."""
    if isinstance(x, Normed):
        r, ss_ptr, tiles, nw, eps = x.r, x.ss.data_ptr(), x.ss.shape[0], x.weight.data_ptr(), x.eps
        if x.weight.shape != (r.shape[1],) or x.weight.dtype != FP16:
            raise ValueError("norm weight must be float16 [K]")
    else:
        r, ss_ptr, tiles, nw, eps = x, None, 0, None, 0.0
    if r.ndim != 2 or r.dtype != FP16 or not r.is_contiguous():
        raise ValueError("operand must be contiguous float16 [M, K]")
    if weight.ndim != 2 or weight.dtype != FP16 or not weight.is_contiguous() or weight.shape[1] != r.shape[1]:
        raise ValueError("weight must be contiguous float16 [N, K]")
    return r, ss_ptr, tiles, nw, eps


def _fused_ws(dev: torch.device, m: int, n: int, k: int) -> torch.Tensor:
    """The per-device workspace of the fused projections (split-K tickets + partial
    tiles), grown when a larger shape needs more; zero-filled when created."""
    need = _pure_size("fe_gemm_fused_workspace_size", m, n, k)
    return decode_workspace(dev, need, kind="gemm")


def gemm_f16(x, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """fp16(x @ weight^T + bias) for M <= 64 rows; x is fp16 [M, K] or Normed."""
    r, ss, tiles, nw, eps = _operand(x, weight)
    dev = _require_gpu(r, weight, bias)
    out = torch.empty((r.shape[0], weight.shape[0]), dtype=FP16, device=dev)
    ws = _fused_ws(dev, r.shape[0], weight.shape[0], r.shape[1])
    _lib.call("fe_gemm_f16", r.data_ptr(), ss, tiles, nw, eps, r.shape[0], r.shape[1],
              weight.data_ptr(), weight.shape[0], _ptr(bias), out.data_ptr(), ws.data_ptr(),
              ws.numel(), _stream(dev))
    return out


def gemm_resid(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
               out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(r, ss): r = fp16(fp16(x @ weight^T) + residual) [M, N] and the per-16-column
    sums of r^2 [ceil(N/16), M] that the next fused projection normalises with."""
    r_in, _, _, _, _ = _operand(x, weight)
    dev = _require_gpu(r_in, weight, residual)
    m, n = r_in.shape[0], weight.shape[0]
    if residual.shape != (m, n) or residual.dtype != FP16 or not residual.is_contiguous():
        raise ValueError("residual must be contiguous float16 [M, N]")
    out = torch.empty((m, n), dtype=FP16, device=dev) if out is None else out
    if out.data_ptr() == residual.data_ptr() or out.data_ptr() == r_in.data_ptr():
        raise ValueError("out must not alias the residual or the operand")
    ss = torch.empty(((n + 15) // 16, m), dtype=torch.float32, device=dev)
    ws = _fused_ws(dev, m, n, r_in.shape[1])
    _lib.call("fe_gemm_resid", r_in.data_ptr(), m, r_in.shape[1], weight.data_ptr(), n,
              residual.data_ptr(), out.data_ptr(), ss.data_ptr(), ws.data_ptr(), ws.numel(),
              _stream(dev))
    return out, ss


def gemm_resid_rmsnorm(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                       norm_weight: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(r, h): r = fp16(fp16(x @ weight^T) + residual) [M, N] and h = RMSNorm(r) with
    norm_weight, in one launch (fe_gemm_resid_rmsnorm; N % 16 == 0, N <= 2048)."""
    r_in, _, _, _, _ = _operand(x, weight)
    dev = _require_gpu(r_in, weight, residual, norm_weight)
    m, n = r_in.shape[0], weight.shape[0]
    if residual.shape != (m, n) or residual.dtype != FP16 or not residual.is_contiguous():
        raise ValueError("residual must be contiguous float16 [M, N]")
    if norm_weight.shape != (n,) or norm_weight.dtype != FP16 or not norm_weight.is_contiguous():
        raise ValueError("norm_weight must be contiguous float16 [N]")
    out = torch.empty((m, n), dtype=FP16, device=dev)
    h = torch.empty((m, n), dtype=FP16, device=dev)
    ss = torch.empty(((n + 15) // 16, m), dtype=torch.float32, device=dev)
    ws = _fused_ws(dev, m, n, r_in.shape[1])
    _lib.call("fe_gemm_resid_rmsnorm", r_in.data_ptr(), m, r_in.shape[1], weight.data_ptr(), n,
              residual.data_ptr(), out.data_ptr(), ss.data_ptr(), norm_weight.data_ptr(),
              float(eps), h.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
    return out, h


def resid_rmsnorm_supported(n: int) -> bool:
    """Whether fe_gemm_resid_rmsnorm takes an output width of n."""
    return n % 16 == 0 and n <= 2048


def gemm_silu(x, weight: torch.Tensor) -> torch.Tensor:
    """fp16(silu(g) * u) [M, I] of the products with weight = [gate; up] [2I, K]."""
    r, ss, tiles, nw, eps = _operand(x, weight)
    dev = _require_gpu(r, weight)
    if weight.shape[0] % 2:
        raise ValueError("weight must stack gate and up rows")
    out = torch.empty((r.shape[0], weight.shape[0] // 2), dtype=FP16, device=dev)
    ws = _fused_ws(dev, r.shape[0], weight.shape[0], r.shape[1])
    _lib.call("fe_gemm_silu", r.data_ptr(), ss, tiles, nw, eps, r.shape[0], r.shape[1],
              weight.data_ptr(), weight.shape[0], out.data_ptr(), ws.data_ptr(), ws.numel(),
              _stream(dev))
    return out


def gemm_rope(x, weight: torch.Tensor, bias: torch.Tensor | None, positions: torch.Tensor,
              inv_freq: torch.Tensor, num_q_heads: int, kv_heads: int, head_dim: int):
    """q [M, Hq, D], k, v [M, Hkv, D] of weight = [q; k; v] with bias and RoPE on q, k."""
    r, ss, tiles, nw, eps = _operand(x, weight)
    dev = _require_gpu(r, weight, bias, positions, inv_freq)
    if weight.shape[0] != (num_q_heads + 2 * kv_heads) * head_dim:
        raise ValueError("weight rows do not match the head configuration")
    m = r.shape[0]
    if positions.dtype != torch.int64 or positions.shape != (m,):
        raise ValueError("positions must be int64 [rows]")
    q = torch.empty((m, num_q_heads, head_dim), dtype=FP16, device=dev)
    k = torch.empty((m, kv_heads, head_dim), dtype=FP16, device=dev)
    v = torch.empty_like(k)
    ws = _fused_ws(dev, m, weight.shape[0], r.shape[1])
    _lib.call("fe_gemm_rope", r.data_ptr(), ss, tiles, nw, eps, m, r.shape[1], weight.data_ptr(),
              _ptr(bias), positions.data_ptr(), inv_freq.data_ptr(), num_q_heads, kv_heads,
              head_dim, q.data_ptr(), k.data_ptr(), v.data_ptr(), ws.data_ptr(), ws.numel(),
              _stream(dev))
    return q, k, v
