"""Paged KV pool with logical block tables and reference-counted blocks.

Same interface and bookkeeping semantics as FlexEngine's PagedKVCache
(src/flexengine/engine/kv_cache/allocator.py:16-158): pools are
[layers, num_blocks, block_size, kv_heads, head_dim], blocks are handed out
from a FIFO free list, shared blocks carry reference counts and are never
written.  The data movement differs: `write` and `materialize` run the HIP
page-write and gather kernels (fe_write_kv / fe_gather_kv) with the slot
mapping built on the host from the Python tables, so unlike the reference they
never synchronise with the device.  The pools must live on a ROCm GPU for
those two calls; the bookkeeping methods work anywhere.
"""
from __future__ import annotations

import math
from collections import Counter, deque
from collections.abc import Sequence
from dataclasses import dataclass

import torch

from flexengine_amd import ops


class CacheExhausted(RuntimeError):
    pass


@dataclass(frozen=True)
class CacheLayout:
    layers: int
    num_blocks: int
    block_size: int
    kv_heads: int
    head_dim: int


class PagedKVCache:
    def __init__(self, layout: CacheLayout, device="cuda:0", dtype=torch.float16, fill=None):
        if dtype != torch.float16:
            raise ValueError("the HIP kernels store the KV pool in float16")
        self.layout = layout
        self.device = torch.device(device)
        self.dtype = dtype
        shape = (layout.layers, layout.num_blocks, layout.block_size, layout.kv_heads, layout.head_dim)
        self.k = torch.empty(shape, dtype=dtype, device=self.device)
        self.v = torch.empty(shape, dtype=dtype, device=self.device)
        if fill is not None:
            self.k.fill_(fill)
            self.v.fill_(fill)
        self.free: deque[int] = deque(range(layout.num_blocks))
        self.tables: dict[str, list[int]] = {}
        self.refs = [0] * layout.num_blocks
        self.retained_refs = [0] * layout.num_blocks
        # device mirror of `tables` (GPU caches): one int32 row per request,
        # written when the request's blocks change, so a step's tables are
        # gathered on the device (device_tables) instead of filled on the host
        self._mirror: torch.Tensor | None = None
        self._mirror_len: torch.Tensor | None = None
        self._rows: dict[str, int] = {}
        self._free_rows: list[int] = []

    # ---- bookkeeping (allocator.py:38-106) ------------------------------------------

    @property
    def free_blocks(self) -> int:
        return len(self.free)

    @property
    def used_blocks(self) -> int:
        return self.layout.num_blocks - len(self.free)

    def capacity_tokens(self) -> int:
        return self.layout.num_blocks * self.layout.block_size

    def available_slots(self, request_id: str) -> int:
        return len(self.tables.get(request_id, [])) * self.layout.block_size

    def missing_blocks(self, request_id: str, target_tokens: int) -> int:
        need = math.ceil(target_tokens / self.layout.block_size)
        return max(0, need - len(self.tables.get(request_id, [])))

    def reserve(self, request_id: str, target_tokens: int) -> None:
        """Grows the request's table to cover target_tokens; all-or-nothing."""
        if target_tokens < 0:
            raise ValueError("negative target_tokens")
        needed = self.missing_blocks(request_id, target_tokens)
        if needed > len(self.free):
            raise CacheExhausted(f"Need {needed} blocks; only {len(self.free)} free")
        fresh = request_id not in self.tables
        table = self.tables.setdefault(request_id, [])
        for _ in range(needed):
            block = self.free.popleft()
            assert self.refs[block] == 0
            self.refs[block] = 1
            table.append(block)
        if needed or fresh:
            self.sync_device_table(request_id)

    def retain_block(self, block: int) -> None:
        """Adds a non-request owner (e.g. a prefix-cache index)."""
        if block < 0 or block >= self.layout.num_blocks or self.refs[block] <= 0:
            raise ValueError("cannot retain an unallocated block")
        self.refs[block] += 1
        self.retained_refs[block] += 1

    def release_block(self, block: int) -> None:
        if block < 0 or block >= self.layout.num_blocks or self.retained_refs[block] <= 0:
            raise ValueError("block has no retained owner")
        self.retained_refs[block] -= 1
        self._release_ref(block)

    def attach_prefix(self, request_id: str, blocks: Sequence[int]) -> None:
        """Shares already-populated complete blocks with a new request."""
        if request_id in self.tables:
            raise ValueError("request already has a block table")
        block_ids = list(blocks)
        if len(block_ids) != len(set(block_ids)):
            raise ValueError("prefix contains duplicate blocks")
        if any(b < 0 or b >= self.layout.num_blocks or self.refs[b] <= 0 for b in block_ids):
            raise ValueError("prefix contains an unallocated block")
        for block in block_ids:
            self.refs[block] += 1
        self.tables[request_id] = block_ids
        self.sync_device_table(request_id)

    def _release_ref(self, block: int) -> None:
        if self.refs[block] <= 0:
            raise RuntimeError("corrupt block reference count")
        self.refs[block] -= 1
        if self.refs[block] == 0:
            self.free.append(block)

    def free_request(self, request_id: str) -> None:
        for block in self.tables.pop(request_id, []):
            self._release_ref(block)
        row = self._rows.pop(request_id, None)
        if row is not None:
            self._mirror_len[row:row + 1].fill_(0)
            self._free_rows.append(row)

    # ---- slot mapping and device tables --------------------------------------------

    def _locators(self, request_id: str, start: int, count: int) -> tuple[list[int], list[int]]:
        """(block, offset) of logical slots start..start+count-1 (allocator.py:107-114)."""
        if start < 0 or count < 0 or start + count > self.available_slots(request_id):
            raise IndexError("KV slots not reserved")
        table = self.tables[request_id]
        bs = self.layout.block_size
        slots = range(start, start + count)
        return [table[i // bs] for i in slots], [i % bs for i in slots]

    def block_table(self, request_ids: Sequence[str], width: int | None = None,
                    pad_block: int | None = None) -> torch.Tensor:
        """int32 [len(request_ids), width] device table; short rows repeat their last block
        (or pad_block), so every entry is a valid block id."""
        rows = [self.tables[r] for r in request_ids]
        width = width if width is not None else max((len(r) for r in rows), default=1)
        out = torch.zeros((len(rows), max(width, 1)), dtype=torch.int32)
        for i, row in enumerate(rows):
            if len(row) > width:
                raise ValueError("table wider than the requested width")
            if row:
                out[i, :len(row)] = torch.tensor(row, dtype=torch.int32)
            fill = pad_block if pad_block is not None else (row[-1] if row else 0)
            out[i, len(row):] = fill
        return out.to(self.device, non_blocking=True)

    def sync_device_table(self, request_id: str) -> None:
        """Writes the request's table into its row of the device mirror (called by
        reserve / attach_prefix; call it after editing `tables` directly).  A no-op for
        a cache that does not live on a GPU."""
        if self.device.type != "cuda":
            return
        table = self.tables[request_id]
        row = self._rows.get(request_id)
        if row is None:
            row = self._free_rows.pop() if self._free_rows else len(self._rows)
            self._rows[request_id] = row
        self._grow_mirror(row + 1, len(table))
        if table:
            self._mirror[row, :len(table)] = torch.tensor(table, dtype=torch.int32).to(
                self.device, non_blocking=True)
        self._mirror_len[row:row + 1].fill_(len(table))

    def _grow_mirror(self, rows: int, width: int) -> None:
        cur_rows, cur_width = (0, 0) if self._mirror is None else tuple(self._mirror.shape)
        if rows <= cur_rows and width <= cur_width:
            return
        new_rows = max(rows, 2 * cur_rows, 16)
        new_width = max(width, 2 * cur_width, 64)
        mirror = torch.zeros((new_rows, new_width), dtype=torch.int32, device=self.device)
        lens = torch.zeros((new_rows,), dtype=torch.int32, device=self.device)
        if self._mirror is not None:
            mirror[:cur_rows, :cur_width] = self._mirror
            lens[:cur_rows] = self._mirror_len
        self._mirror, self._mirror_len = mirror, lens

    def device_tables(self, request_ids: Sequence[str | None], width: int | None = None,
                      pad_block: int | None = None) -> torch.Tensor:
        """block_table() built on the device: int32 [len(request_ids), width] gathered
        from the mirror rows (fe_gather_tables), so a step copies one row index per
        request instead of its whole table.  None entries are rows of pad_block."""
        from . import ops
        if self.device.type != "cuda":
            raise RuntimeError("device_tables needs a GPU cache")
        rows = []
        for r in request_ids:
            if r is None:
                rows.append(-1)
                continue
            if len(self.tables[r]) > (width if width is not None else len(self.tables[r])):
                raise ValueError("table wider than the requested width")
            rows.append(self._rows[r])
        if width is None:
            width = max((len(self.tables[r]) for r in request_ids if r is not None), default=1)
        if self._mirror is None:
            self._grow_mirror(1, 1)
        idx = torch.tensor(rows, dtype=torch.int32).to(self.device, non_blocking=True)
        return ops.gather_tables(self._mirror, self._mirror_len, idx, width,
                                 -1 if pad_block is None else pad_block)

    # ---- data movement (HIP kernels) --------------------------------------------------

    def write(self, layer: int, request_id: str, start: int, keys: torch.Tensor,
              values: torch.Tensor) -> None:
        """Page write of rows start..start+n-1 (allocator.py:116-127) via fe_write_kv."""
        if keys.shape != values.shape or keys.ndim != 3:
            raise ValueError("K/V shapes must be [tokens, kv_heads, head_dim]")
        if tuple(keys.shape[1:]) != (self.layout.kv_heads, self.layout.head_dim):
            raise ValueError("wrong KV shape")
        if keys.dtype != self.dtype or values.dtype != self.dtype:
            raise ValueError("wrong KV dtype")
        ids, offsets = self._locators(request_id, start, keys.shape[0])
        if any(self.refs[block] > 1 for block in set(ids)):
            raise RuntimeError("cannot write a shared immutable KV block")
        if not ids:
            return
        slots = torch.tensor([ids, offsets], dtype=torch.int32).to(self.device, non_blocking=True)
        ops.write_kv(keys, values, self.k[layer], self.v[layer], slots[0], slots[1])

    def materialize(self, layer: int, request_id: str, length: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Gathers rows 0..length-1 to contiguous [length, Hkv, D] (allocator.py:129-134)
        via fe_gather_kv.  Comparison / test helper, not on the decode path."""
        if length <= 0:
            raise ValueError("length must be >0")
        self._locators(request_id, 0, length)  # validates the range
        table = self.block_table([request_id])
        ctx = torch.tensor([length], dtype=torch.int32).to(self.device)
        offs = torch.tensor([0, length], dtype=torch.int32).to(self.device)
        return ops.gather_kv(self.k[layer], self.v[layer], table, ctx, offs, length)

    def iter_blocks(self, layer: int, request_id: str, length: int):
        """Views of the physical pages covering rows 0..length-1 (allocator.py:136-145)."""
        if length <= 0 or length > self.available_slots(request_id):
            raise ValueError("requested length is invalid/unreserved")
        for j, bid in enumerate(self.tables[request_id]):
            start = j * self.layout.block_size
            if start >= length:
                break
            n = min(self.layout.block_size, length - start)
            yield start, self.k[layer, bid, :n], self.v[layer, bid, :n]

    def assert_invariants(self) -> None:
        used = [item for table in self.tables.values() for item in table]
        free = list(self.free)
        if len(free) != len(set(free)) or set(free) & set(used):
            raise AssertionError("free/used blocks overlap or duplicate")
        request_refs = Counter(used)
        for block in range(self.layout.num_blocks):
            expected = request_refs[block] + self.retained_refs[block]
            if self.refs[block] != expected:
                raise AssertionError("ref count mismatch")
            if (self.refs[block] == 0) != (block in self.free):
                raise AssertionError("free/allocated state mismatch")
