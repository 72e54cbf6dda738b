"""Paged KV pool: physical blocks, per-request page tables, and the GPU copy of
those tables that the decode step gathers from.

The public surface is that of FlexEngine's PagedKVCache
(src/flexengine/engine/kv_cache/allocator.py:12-158) -- the names, argument
meaning and exception types its callers rely on: `layout`, `device`, `dtype`,
the `k` / `v` pools [layers, num_blocks, block_size, kv_heads, head_dim],
`tables[request_id]`, `refs[block]`, `free`, `free_blocks`, `used_blocks`,
`reserve`, `attach_prefix`, `retain_block`, `release_block`, `free_request`,
`write`, `materialize`, `iter_blocks`, `assert_invariants`; CacheExhausted for
a full pool, and "shared immutable" in the error of a write into a shared
block (the substring tests/unit/test_prefix_cache.py:85 matches).

The organisation underneath is this package's own:

* `_Ledger` counts the owners of every block in numpy arrays (all owners, and
  the pinned ones that are not requests, e.g. a prefix-cache index) and keeps
  the free blocks in a ring buffer in release order: a freed block is reused as
  late as possible, so its contents stay valid for prefix matching the longest,
  and a fresh pool hands out blocks 0, 1, 2, ... (the order the reference's
  tests read, e.g. table [0, 3, 4] in tests/unit/test_attention.py:25-31).
* `_PageTables` holds every live request's table as one int32 row of a
  growable host matrix with a length per row.  The matrix is the only copy of
  the tables on the host; `tables` is a mapping view over it.
* A GPU cache keeps a device copy of that matrix (`_DeviceTables`), written
  per changed range of a row: growing a table copies only its new entries, and
  a full re-copy happens only when the matrix itself grows.  The decode step
  builds its block tables on the device from row indices (fe_gather_tables),
  instead of filling them on the host every step.
* `write` and `materialize` run the HIP page-write and gather kernels with the
  slot map computed by numpy from the table row; unlike the reference they
  never synchronise with the device.  The pools must live on a ROCm GPU for
  those two calls; all bookkeeping works anywhere.
* Pools are float16, bfloat16 or float32 (the reference's own default,
  allocator.py:26), each with its HIP kernels (the _bf16 / _f32 entry points).
  The default here is float16 on "cuda:0", the dtype and place the decode path
  is built around; callers that want the reference's float32 pass it.
"""
from __future__ import annotations

from collections.abc import Iterator, Mapping, Sequence
from dataclasses import dataclass

import numpy as np
import torch

from flexengine_amd import ops


class CacheExhausted(RuntimeError):
    """The pool has fewer free blocks than a reservation needs."""


@dataclass(frozen=True)
class CacheLayout:
    layers: int
    num_blocks: int
    block_size: int
    kv_heads: int
    head_dim: int


# ---------------------------------------------------------------------------------------
# block ledger
# ---------------------------------------------------------------------------------------

class _Ledger:
    """Owner counts of every block and the ring of free blocks (release order)."""

    def __init__(self, num_blocks: int):
        self.n = num_blocks
        self.owners = np.zeros(num_blocks, dtype=np.int32)   # requests + pins
        self.pins = np.zeros(num_blocks, dtype=np.int32)     # non-request owners
        self.ring = np.arange(num_blocks, dtype=np.int32)
        self.head = 0
        self.count = num_blocks

    def free_order(self) -> np.ndarray:
        return self.ring[(self.head + np.arange(self.count)) % max(self.n, 1)]

    def take(self, k: int) -> np.ndarray:
        """k blocks off the front of the ring, each now with one owner."""
        got = self.ring[(self.head + np.arange(k)) % max(self.n, 1)].copy()
        self.head = (self.head + k) % max(self.n, 1)
        self.count -= k
        self.owners[got] = 1
        return got

    def add_owner(self, blocks: np.ndarray) -> None:
        np.add.at(self.owners, blocks, 1)

    def drop_owner(self, blocks: np.ndarray) -> None:
        """One owner fewer for each of blocks (distinct ids: a table never lists a
        block twice); blocks left without owners go to the back of the ring, in
        the order given."""
        if blocks.size == 0:
            return
        if (self.owners[blocks] <= 0).any():
            raise RuntimeError("block owner count would drop below zero (ledger corrupted)")
        self.owners[blocks] -= 1
        freed = blocks[self.owners[blocks] == 0]
        slots = (self.head + self.count + np.arange(freed.size)) % self.n
        self.ring[slots] = freed
        self.count += freed.size


class _FreeView:
    """Read-only view of the free blocks, in the order they will be handed out."""

    def __init__(self, ledger: _Ledger):
        self._ledger = ledger

    def __len__(self) -> int:
        return self._ledger.count

    def __iter__(self) -> Iterator[int]:
        return iter(self._ledger.free_order().tolist())

    def __contains__(self, block) -> bool:
        b = int(block)
        return 0 <= b < self._ledger.n and self._ledger.owners[b] == 0


# ---------------------------------------------------------------------------------------
# page tables
# ---------------------------------------------------------------------------------------

class _PageTables:
    """One int32 row per live request in a growable matrix, a length per row."""

    def __init__(self):
        self.row_of: dict[str, int] = {}
        self.mat = np.zeros((16, 64), dtype=np.int32)
        self.lens = np.zeros(16, dtype=np.int32)
        self.spare_rows: list[int] = []
        self.generation = 0     # bumped whenever `mat` is reallocated

    def blocks(self, request_id: str) -> np.ndarray:
        r = self.row_of[request_id]
        return self.mat[r, :self.lens[r]]

    def width_of(self, request_id: str) -> int:
        r = self.row_of.get(request_id)
        return 0 if r is None else int(self.lens[r])

    def _fit(self, rows: int, width: int) -> None:
        cur_rows, cur_width = self.mat.shape
        if rows <= cur_rows and width <= cur_width:
            return
        # grow by doubling the dimension that ran out, so re-copies stay rare
        new_rows = cur_rows if rows <= cur_rows else max(rows, 2 * cur_rows)
        new_width = cur_width if width <= cur_width else max(width, 2 * cur_width)
        mat = np.zeros((new_rows, new_width), np.int32)
        mat[:cur_rows, :cur_width] = self.mat
        lens = np.zeros(mat.shape[0], np.int32)
        lens[:cur_rows] = self.lens
        self.mat, self.lens = mat, lens
        self.generation += 1

    def open_row(self, request_id: str) -> int:
        r = self.row_of.get(request_id)
        if r is None:
            r = self.spare_rows.pop() if self.spare_rows else len(self.row_of)
            self._fit(r + 1, 1)
            self.row_of[request_id] = r
            self.lens[r] = 0
        return r

    def extend(self, request_id: str, new_blocks: np.ndarray) -> tuple[int, int, int]:
        """Appends blocks; returns (row, first changed column, end column)."""
        r = self.open_row(request_id)
        lo = int(self.lens[r])
        hi = lo + new_blocks.size
        self._fit(r + 1, hi)
        self.mat[r, lo:hi] = new_blocks
        self.lens[r] = hi
        return r, lo, hi

    def replace(self, request_id: str, blocks: np.ndarray) -> int:
        r = self.open_row(request_id)
        self._fit(r + 1, blocks.size)
        self.mat[r, :blocks.size] = blocks
        self.lens[r] = blocks.size
        return r

    def close_row(self, request_id: str) -> tuple[int, np.ndarray] | None:
        r = self.row_of.pop(request_id, None)
        if r is None:
            return None
        blocks = self.mat[r, :self.lens[r]].copy()
        self.lens[r] = 0
        self.spare_rows.append(r)
        return r, blocks


class _TablesView(Mapping):
    """`tables[request_id]` -> list of block ids (a fresh list each time).

    Assigning a list that holds exactly the request's blocks in another order
    (e.g. reversed page order, tests/gpu/test_triton_paged_attention.py:15)
    rewrites the row on the host and on the device; any other assignment would
    bypass the owner counts and is refused."""

    def __init__(self, cache: "PagedKVCache"):
        self._cache = cache

    def __getitem__(self, request_id: str) -> list[int]:
        return self._cache._pt.blocks(request_id).tolist()

    def __iter__(self) -> Iterator[str]:
        return iter(list(self._cache._pt.row_of))

    def __len__(self) -> int:
        return len(self._cache._pt.row_of)

    def __contains__(self, request_id) -> bool:
        return request_id in self._cache._pt.row_of

    def __setitem__(self, request_id: str, blocks: Sequence[int]) -> None:
        self._cache._reorder(request_id, blocks)


class _DeviceTables:
    """GPU copy of the page-table matrix and its row lengths (int32)."""

    def __init__(self, device: torch.device):
        self.device = device
        self.mat: torch.Tensor | None = None
        self.lens: torch.Tensor | None = None
        self.generation = -1

    def _upload(self, host: np.ndarray) -> torch.Tensor:
        # a private host copy: the asynchronous copy never reads memory the
        # bookkeeping may change afterwards
        return torch.from_numpy(np.ascontiguousarray(host).copy()).to(self.device, non_blocking=True)

    def push(self, pt: _PageTables, row: int | None = None, lo: int = 0, hi: int | None = None) -> None:
        if self.mat is None or self.generation != pt.generation:
            self.mat = self._upload(pt.mat)
            self.lens = self._upload(pt.lens)
            self.generation = pt.generation
            return
        if row is None:
            return
        hi = int(pt.lens[row]) if hi is None else hi
        if hi > lo:
            self.mat[row, lo:hi].copy_(self._upload(pt.mat[row, lo:hi]), non_blocking=True)
        self.lens[row:row + 1].copy_(self._upload(pt.lens[row:row + 1]), non_blocking=True)


# ---------------------------------------------------------------------------------------
# the cache
# ---------------------------------------------------------------------------------------

class PagedKVCache:
    def __init__(self, layout: CacheLayout, device="cuda:0", dtype=torch.float16, fill=None):
        if dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError(f"KV pools are float16, bfloat16 or float32 on the HIP kernels; "
                             f"got {dtype}")
        self.layout = layout
        self.device = torch.device(device)
        self.dtype = dtype
        shape = (layout.layers, layout.num_blocks, layout.block_size, layout.kv_heads,
                 layout.head_dim)
        self.k = torch.empty(shape, dtype=dtype, device=self.device)
        self.v = torch.empty(shape, dtype=dtype, device=self.device)
        if fill is not None:
            self.k.fill_(fill)
            self.v.fill_(fill)
        self._ledger = _Ledger(layout.num_blocks)
        self._pt = _PageTables()
        self._dev = _DeviceTables(self.device) if self.device.type == "cuda" else None
        self.tables = _TablesView(self)
        self.free = _FreeView(self._ledger)

    # ---- counters ----------------------------------------------------------------

    @property
    def refs(self) -> np.ndarray:
        """Owners per block (requests + pins), read-only."""
        view = self._ledger.owners.view()
        view.flags.writeable = False
        return view

    @property
    def free_blocks(self) -> int:
        return self._ledger.count

    @property
    def used_blocks(self) -> int:
        return self.layout.num_blocks - self._ledger.count

    def capacity_tokens(self) -> int:
        return self.layout.num_blocks * self.layout.block_size

    def available_slots(self, request_id: str) -> int:
        return self._pt.width_of(request_id) * self.layout.block_size

    def missing_blocks(self, request_id: str, target_tokens: int) -> int:
        bs = self.layout.block_size
        return max(0, -(-target_tokens // bs) - self._pt.width_of(request_id))

    # ---- ownership ---------------------------------------------------------------

    def _sync(self, row: int | None = None, lo: int = 0, hi: int | None = None) -> None:
        if self._dev is not None:
            self._dev.push(self._pt, row, lo, hi)

    def reserve(self, request_id: str, target_tokens: int) -> None:
        """Grows the request's table to cover target_tokens slots; takes every block
        it needs or none (CacheExhausted)."""
        if target_tokens < 0:
            raise ValueError(f"target_tokens must be >= 0, got {target_tokens}")
        need = self.missing_blocks(request_id, target_tokens)
        if need > self._ledger.count:
            raise CacheExhausted(f"reserve({request_id!r}, {target_tokens}): {need} more blocks "
                                 f"needed, {self._ledger.count} free")
        row, lo, hi = self._pt.extend(request_id, self._ledger.take(need))
        self._sync(row, lo, hi)

    def attach_prefix(self, request_id: str, blocks: Sequence[int]) -> None:
        """Starts a new request's table with already-written complete blocks it shares."""
        if request_id in self._pt.row_of:
            raise ValueError(f"request {request_id!r} already owns a page table")
        ids = np.asarray(list(blocks), dtype=np.int64)
        if np.unique(ids).size != ids.size:
            raise ValueError("a shared prefix must not list a block twice")
        if ids.size and ((ids < 0) | (ids >= self.layout.num_blocks)).any():
            raise ValueError("a shared prefix may only hold allocated blocks (id out of range)")
        if ids.size and (self._ledger.owners[ids] <= 0).any():
            raise ValueError("a shared prefix may only hold allocated blocks")
        self._ledger.add_owner(ids)
        row, lo, hi = self._pt.extend(request_id, ids.astype(np.int32))
        self._sync(row, lo, hi)

    def _live_block(self, block: int) -> int:
        b = int(block)
        if not 0 <= b < self.layout.num_blocks:
            raise ValueError(f"block {b} is outside the pool of {self.layout.num_blocks}")
        return b

    def retain_block(self, block: int) -> None:
        """Pins an allocated block for an owner that is not a request (a prefix index)."""
        b = self._live_block(block)
        if self._ledger.owners[b] <= 0:
            raise ValueError(f"block {b} is free; only an allocated block can be pinned")
        self._ledger.owners[b] += 1
        self._ledger.pins[b] += 1

    def release_block(self, block: int) -> None:
        """Drops one pin of a block; it returns to the pool with its last owner."""
        b = self._live_block(block)
        if self._ledger.pins[b] <= 0:
            raise ValueError(f"block {b} holds no pin to release")
        self._ledger.pins[b] -= 1
        self._ledger.drop_owner(np.array([b], dtype=np.int32))

    def free_request(self, request_id: str) -> None:
        closed = self._pt.close_row(request_id)
        if closed is None:
            return
        row, blocks = closed
        self._ledger.drop_owner(blocks)
        self._sync(row, 0, 0)   # row length 0 on the device as well

    def _reorder(self, request_id: str, blocks: Sequence[int]) -> None:
        new = np.asarray(list(blocks), dtype=np.int32)
        cur = self._pt.blocks(request_id)
        if new.size != cur.size or not np.array_equal(np.sort(new), np.sort(cur)):
            raise ValueError("a table may only be replaced by a reordering of its own blocks")
        row = self._pt.replace(request_id, new)
        self._sync(row, 0, new.size)

    # ---- device tables ---------------------------------------------------------------

    def sync_device_table(self, request_id: str) -> None:
        """Re-copies the request's row to the device copy (tables stay in sync by
        themselves; kept for callers that want to force it)."""
        row = self._pt.row_of[request_id]
        self._sync(row, 0, int(self._pt.lens[row]))

    def block_table(self, request_ids: Sequence[str], width: int | None = None,
                    pad_block: int | None = None) -> torch.Tensor:
        """int32 [len(request_ids), width] table built on the host and copied to the
        cache's device; entries past a request's blocks repeat its last block (or
        pad_block), so every entry names a real block."""
        rows = [self._pt.blocks(r) for r in request_ids]
        if width is None:
            width = max((r.size for r in rows), default=1)
        width = max(int(width), 1)
        out = np.zeros((len(rows), width), dtype=np.int32)
        for i, blocks in enumerate(rows):
            if blocks.size > width:
                raise ValueError(f"table of {request_ids[i]!r} has {blocks.size} blocks, "
                                 f"more than width {width}")
            out[i, :blocks.size] = blocks
            out[i, blocks.size:] = pad_block if pad_block is not None else (
                blocks[-1] if blocks.size else 0)
        return torch.from_numpy(out).to(self.device, non_blocking=True)

    def device_tables(self, request_ids: Sequence[str | None], width: int | None = None,
                      pad_block: int | None = None) -> torch.Tensor:
        """block_table() gathered on the device from the device copy of the page
        tables (fe_gather_tables): the host sends one row index per request.  None
        entries give rows of pad_block."""
        if self._dev is None:
            raise RuntimeError("device_tables needs a cache whose pools live on a GPU")
        live = [r for r in request_ids if r is not None]
        widest = max((self._pt.width_of(r) for r in live), default=1)
        if width is None:
            width = widest
        elif widest > width:
            raise ValueError(f"a table has {widest} blocks, more than width {width}")
        rows = np.array([-1 if r is None else self._pt.row_of[r] for r in request_ids], np.int32)
        self._sync()
        idx = torch.from_numpy(rows).to(self.device, non_blocking=True)
        return ops.gather_tables(self._dev.mat, self._dev.lens, idx, width,
                                 -1 if pad_block is None else pad_block)

    # ---- data movement (HIP kernels) ---------------------------------------------------

    def _slots(self, request_id: str, start: int, count: int) -> tuple[np.ndarray, np.ndarray]:
        """(block, offset) of the request's logical slots start .. start+count-1."""
        have = self.available_slots(request_id)
        if start < 0 or count < 0 or start + count > have:
            raise IndexError(f"slots [{start}, {start + count}) of {request_id!r} are not "
                             f"reserved ({have} reserved)")
        pos = np.arange(start, start + count)
        bs = self.layout.block_size
        return self._pt.blocks(request_id)[pos // bs], (pos % bs).astype(np.int32)

    def write(self, layer: int, request_id: str, start: int, keys: torch.Tensor,
              values: torch.Tensor) -> None:
        """Stores keys/values [n, kv_heads, head_dim] at slots start .. start+n-1 of
        the request (fe_write_kv)."""
        if keys.ndim != 3 or keys.shape != values.shape:
            raise ValueError("keys and values must both be [tokens, kv_heads, head_dim]")
        if tuple(keys.shape[1:]) != (self.layout.kv_heads, self.layout.head_dim):
            raise ValueError(f"rows must be [{self.layout.kv_heads}, {self.layout.head_dim}], "
                             f"got {tuple(keys.shape[1:])}")
        if keys.dtype != self.dtype or values.dtype != self.dtype:
            raise ValueError(f"keys/values must be {self.dtype}")
        blocks, offsets = self._slots(request_id, start, keys.shape[0])
        shared = blocks[self._ledger.owners[blocks] > 1]
        if shared.size:
            raise RuntimeError(f"block {int(shared[0])} has several owners: shared immutable "
                               "KV blocks are never written")
        if blocks.size == 0:
            return
        slots = torch.from_numpy(np.stack([blocks, offsets])).to(self.device, non_blocking=True)
        ops.write_kv(keys, values, self.k[layer], self.v[layer], slots[0], slots[1])

    def materialize(self, layer: int, request_id: str, length: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous copies [length, kv_heads, head_dim] of the request's first
        `length` K and V rows (fe_gather_kv); a comparison helper, not on the decode
        path."""
        if length <= 0:
            raise ValueError(f"length must be positive, got {length}")
        self._slots(request_id, 0, length)
        table = self.block_table([request_id])
        ctx = torch.tensor([length], dtype=torch.int32).to(self.device)
        offs = torch.tensor([0, length], dtype=torch.int32).to(self.device)
        return ops.gather_kv(self.k[layer], self.v[layer], table, ctx, offs, length)

    def iter_blocks(self, layer: int, request_id: str, length: int):
        """(first position, K page view, V page view) of every page holding one of the
        request's first `length` rows; views of the pool, nothing copied."""
        if not 0 < length <= self.available_slots(request_id):
            raise ValueError(f"length {length} is not within the reserved slots of {request_id!r}")
        bs = self.layout.block_size
        pages = self._pt.blocks(request_id)[:-(-length // bs)]
        for j, block in enumerate(pages.tolist()):
            rows = min(bs, length - j * bs)
            yield j * bs, self.k[layer, block, :rows], self.v[layer, block, :rows]

    # ---- consistency ---------------------------------------------------------------

    def assert_invariants(self) -> None:
        """Owner counts equal table references + pins; the free ring holds each
        ownerless block exactly once; a GPU cache's device tables equal the host's."""
        led, pt = self._ledger, self._pt
        live = [pt.blocks(r) for r in pt.row_of]
        referenced = np.concatenate(live).astype(np.int64) if live else np.zeros(0, np.int64)
        expect = np.bincount(referenced, minlength=led.n)[:led.n] + led.pins
        if not np.array_equal(expect, led.owners):
            raise AssertionError("owner counts differ from table references + pins")
        ring = led.free_order()
        if np.unique(ring).size != ring.size:
            raise AssertionError("a block sits in the free ring twice")
        if not np.array_equal(np.sort(ring), np.flatnonzero(led.owners == 0)):
            raise AssertionError("the free ring differs from the set of ownerless blocks")
        if self._dev is not None and self._dev.mat is not None:
            mat, lens = self._dev.mat.cpu().numpy(), self._dev.lens.cpu().numpy()
            for r in pt.row_of.values():
                n = int(pt.lens[r])
                if lens[r] != n or not np.array_equal(mat[r, :n], pt.mat[r, :n]):
                    raise AssertionError("device page tables differ from the host's")
