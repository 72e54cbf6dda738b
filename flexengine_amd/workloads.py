"""Seeded synthetic inputs for the benchmark configurations C1-C5.

All inputs are drawn on the CPU with torch.Generator().manual_seed(seed) in
float32 and cast to float16, so they are identical on every host; they are
moved to the GPU afterwards.  q, K and V are N(0, 1) and every pool block is
filled, including blocks no sequence uses.  Block tables are slices of a
random permutation of the pool, so consecutive logical pages are scattered.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

FP16 = torch.float16


@dataclass
class DecodeWorkload:
    """One layer of a batched single-token decode step."""

    name: str
    q: torch.Tensor             # [B, Hq, D] fp16
    k_pool: torch.Tensor        # [NB, BS, Hkv, D] fp16
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # [B, W] int32
    context_lens: torch.Tensor  # [B] int32, includes the decoded token
    k_new: torch.Tensor | None = None  # [B, Hkv, D] fp16: page-written at position L-1
    v_new: torch.Tensor | None = None
    unique_tokens: int = 0      # distinct K/V rows attention must read (shared prefixes once)
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    @property
    def block_size(self) -> int:
        return self.k_pool.shape[1]

    def to(self, device) -> "DecodeWorkload":
        def mv(t):
            return None if t is None else t.to(device)
        return DecodeWorkload(self.name, mv(self.q), mv(self.k_pool), mv(self.v_pool),
                              mv(self.block_tables), mv(self.context_lens), mv(self.k_new),
                              mv(self.v_new), self.unique_tokens, dict(self.meta))

    def kv_row_bytes(self) -> int:
        """Bytes of K plus V for one token of one layer (2 * Hkv * D * element size)."""
        _, _, hkv, d = self.k_pool.shape
        return 2 * hkv * d * self.k_pool.element_size()

    def algorithmic_bytes(self, logical: bool = False) -> int:
        """Compulsory HBM bytes of one decode call.

        K/V rows read once each (unique rows; `logical` counts shared prefix
        rows once per sequence), q read and out written once, tables and
        context lengths read, and the page write's k/v rows written (the new
        rows are read once, as row L-1 of the context, from k_new/v_new).
        """
        ctx = self.context_lens.to(torch.int64)
        tokens = int(ctx.sum()) if (logical or not self.unique_tokens) else self.unique_tokens
        b, hq, d = self.q.shape
        nbytes = tokens * self.kv_row_bytes()
        nbytes += 2 * b * hq * d * self.q.element_size()  # q in, out
        pages = int(((ctx + self.block_size - 1) // self.block_size).sum())
        nbytes += 4 * pages + 4 * b                         # table entries + lengths
        if self.k_new is not None:
            nbytes += b * self.kv_row_bytes()               # new rows written to the pool
        return nbytes


@dataclass
class PrefillWorkload:
    """A mixed continuous-batching step: ragged prefill chunks plus decode rows."""

    name: str
    q: torch.Tensor             # [total_q, Hq, D] prefill queries
    q_offsets: torch.Tensor     # [S+1] int32
    context_lens: torch.Tensor  # [S] int32, cached + new tokens
    block_tables: torch.Tensor  # [S, W] int32
    k_pool: torch.Tensor
    v_pool: torch.Tensor
    decode: DecodeWorkload | None = None
    meta: dict = field(default_factory=dict)

    def to(self, device) -> "PrefillWorkload":
        return PrefillWorkload(self.name, self.q.to(device), self.q_offsets.to(device),
                               self.context_lens.to(device), self.block_tables.to(device),
                               self.k_pool.to(device), self.v_pool.to(device),
                               None if self.decode is None else self.decode.to(device),
                               dict(self.meta))

    def flops(self) -> int:
        """4 * Hq * D * (valid query-key pairs): QK^T and PV, multiply-add = 2 flops."""
        hq, d = self.q.shape[1], self.q.shape[2]
        qo = self.q_offsets.tolist()
        total = 0
        for s, ctx in enumerate(self.context_lens.tolist()):
            n = qo[s + 1] - qo[s]
            c = ctx - n
            total += n * c + n * (n + 1) // 2
        return 4 * hq * d * total


def _randn(gen: torch.Generator, *shape) -> torch.Tensor:
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(FP16)


def _tables_from_perm(perm: torch.Tensor, pages: list[int], width: int) -> torch.Tensor:
    """Consecutive slices of a permutation; unused columns repeat the row's last block."""
    rows = torch.zeros((len(pages), width), dtype=torch.int32)
    at = 0
    for b, n in enumerate(pages):
        row = perm[at:at + n].to(torch.int32)
        at += n
        rows[b, :n] = row
        if n < width:
            rows[b, n:] = row[-1] if n else 0
    return rows


def make_decode_workload(name: str, seed: int, batch: int, hq: int, hkv: int, d: int,
                         lengths: list[int], block_size: int = 16, num_blocks: int | None = None,
                         width: int | None = None, with_new_kv: bool = False,
                         pool_factor: float = 1.25) -> DecodeWorkload:
    """Generic generator: private pages per sequence, tables from one random permutation."""
    gen = torch.Generator().manual_seed(seed)
    pages = [math.ceil(n / block_size) for n in lengths]
    need = sum(pages)
    nb = num_blocks if num_blocks is not None else max(need, math.ceil(pool_factor * need))
    if nb < need:
        raise ValueError("pool too small for the requested lengths")
    width = width if width is not None else max(pages)
    q = _randn(gen, batch, hq, d)
    k_pool = _randn(gen, nb, block_size, hkv, d)
    v_pool = _randn(gen, nb, block_size, hkv, d)
    perm = torch.randperm(nb, generator=gen)
    tables = _tables_from_perm(perm, pages, width)
    k_new = v_new = None
    if with_new_kv:
        k_new = _randn(gen, batch, hkv, d)
        v_new = _randn(gen, batch, hkv, d)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    return DecodeWorkload(name, q, k_pool, v_pool, tables, ctx, k_new, v_new,
                          unique_tokens=int(ctx.sum()), meta={"seed": seed})


def shared_prefix_workload(seed: int, groups: list[tuple[int, int]], singles: int = 0,
                           hq: int = 12, hkv: int = 2, d: int = 128, block_size: int = 16,
                           tail: tuple[int, int] = (1, 300),
                           member_lens: dict[int, int] | None = None,
                           with_new_kv: bool = False) -> DecodeWorkload:
    """Decode rows in groups that share prefix blocks, then rows of their own.

    groups: (members, prefix_tokens) per group; the group's first
    prefix_tokens // block_size blocks are shared by all its members (a prefix
    that is not a whole number of blocks shares only the whole blocks, as
    FlexEngine's prefix cache does), each member continues with a private tail
    of U{tail} tokens.  member_lens overrides the length of batch row b (a
    context that ends inside the prefix, or 0 = inactive).  `singles` rows with
    no shared prefix follow the groups.  meta holds group_offsets and
    prefix_lens (the prefix_tokens as given) for fe_paged_decode_shared_prefix.
    """
    gen = torch.Generator().manual_seed(seed)
    member_lens = member_lens or {}
    lengths, shared_of = [], []
    offsets = [0]
    for g, (m, p) in enumerate(groups):
        shared = p // block_size * block_size
        for _ in range(m):
            b = len(lengths)
            t = int(torch.randint(tail[0], tail[1] + 1, (1,), generator=gen))
            lengths.append(member_lens.get(b, shared + t))
            shared_of.append(g)
        offsets.append(len(lengths))
    for _ in range(singles):
        b = len(lengths)
        t = int(torch.randint(tail[0], tail[1] + 1, (1,), generator=gen))
        lengths.append(member_lens.get(b, t))
        shared_of.append(-1)
    batch = len(lengths)
    shared_pages = [p // block_size for _, p in groups]
    # pages each row owns privately (beyond its group's shared pages)
    own = []
    for b, n in enumerate(lengths):
        sp = shared_pages[shared_of[b]] if shared_of[b] >= 0 else 0
        own.append(max(0, math.ceil(n / block_size) - sp))
    nb = sum(shared_pages) + sum(own) + 1
    width = max(1, max((shared_pages[shared_of[b]] if shared_of[b] >= 0 else 0) + own[b]
                       for b in range(batch)))
    q = _randn(gen, batch, hq, d)
    k_pool = _randn(gen, nb, block_size, hkv, d)
    v_pool = _randn(gen, nb, block_size, hkv, d)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    tables = torch.zeros((batch, width), dtype=torch.int32)
    at = 0
    group_blocks = []
    for sp in shared_pages:
        group_blocks.append(perm[at:at + sp])
        at += sp
    for b in range(batch):
        row = []
        if shared_of[b] >= 0:
            row.extend(group_blocks[shared_of[b]].tolist())
        row.extend(perm[at:at + own[b]].tolist())
        at += own[b]
        if not row:
            row = [int(perm[-1])]
        tables[b, :len(row)] = torch.tensor(row, dtype=torch.int32)
        tables[b, len(row):] = row[-1]
    k_new = v_new = None
    if with_new_kv:
        k_new = _randn(gen, batch, hkv, d)
        v_new = _randn(gen, batch, hkv, d)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    unique = sum(sp * block_size for sp in shared_pages) + sum(
        max(0, n - (shared_pages[shared_of[b]] * block_size if shared_of[b] >= 0 else 0))
        for b, n in enumerate(lengths))
    return DecodeWorkload("shared-prefix", q, k_pool, v_pool, tables, ctx, k_new, v_new,
                          unique_tokens=unique,
                          meta={"seed": seed,
                                "group_offsets": torch.tensor(offsets, dtype=torch.int32),
                                "prefix_lens": torch.tensor([p for _, p in groups],
                                                            dtype=torch.int32)})


def c1_workload() -> DecodeWorkload:
    """C1: Qwen2.5-0.5B heads (14/2/64), B=8, L ~ U{16..512}, 256-block pool."""
    gen = torch.Generator().manual_seed(1)
    lengths = torch.randint(16, 513, (8,), generator=gen).tolist()
    return make_decode_workload("C1", 101, 8, 14, 2, 64, lengths, num_blocks=256, width=32)


def c2_lengths(seed: int = 2, batch: int = 64) -> list[int]:
    gen = torch.Generator().manual_seed(seed)
    u = torch.rand(batch, generator=gen, dtype=torch.float64)
    return torch.round(torch.exp(math.log(128) + u * (math.log(4096) - math.log(128)))).long().tolist()


def c2_workload(batch: int = 64) -> DecodeWorkload:
    """C2 (headline): Qwen2.5-1.5B heads (12/2/128), B=64, L log-uniform [128,4096],
    1.25x pool, plus the page write of each sequence's new token."""
    return make_decode_workload("C2", 202, batch, 12, 2, 128, c2_lengths(2, batch), width=256,
                                with_new_kv=True)


def c3_workload(groups: int = 8, per_group: int = 32, prefix: int = 2048) -> DecodeWorkload:
    """C3: shared-prefix long-context decode, B = groups * per_group; each group shares
    `prefix` tokens (prefix/16 physical blocks, refcount per_group) then private tails
    t ~ U{16..2048}."""
    gen = torch.Generator().manual_seed(3)
    bs, hq, hkv, d = 16, 12, 2, 128
    batch = groups * per_group
    tails = torch.randint(16, 2049, (batch,), generator=gen).tolist()
    shared_pages = prefix // bs
    tail_pages = [math.ceil(t / bs) for t in tails]
    nb = groups * shared_pages + sum(tail_pages)
    q = _randn(gen, batch, hq, d)
    k_pool = _randn(gen, nb, bs, hkv, d)
    v_pool = _randn(gen, nb, bs, hkv, d)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    width = shared_pages + max(tail_pages)
    tables = torch.zeros((batch, width), dtype=torch.int32)
    at = groups * shared_pages
    for b in range(batch):
        grp = b // per_group
        tables[b, :shared_pages] = perm[grp * shared_pages:(grp + 1) * shared_pages]
        n = tail_pages[b]
        tables[b, shared_pages:shared_pages + n] = perm[at:at + n]
        at += n
        tables[b, shared_pages + n:] = tables[b, shared_pages + n - 1]
    lengths = [prefix + t for t in tails]
    ctx = torch.tensor(lengths, dtype=torch.int32)
    return DecodeWorkload("C3", q, k_pool, v_pool, tables, ctx, None, None,
                          unique_tokens=groups * prefix + sum(tails),
                          meta={"seed": 3, "groups": groups, "per_group": per_group,
                                "prefix": prefix,
                                "group_offsets": torch.arange(0, batch + 1, per_group,
                                                              dtype=torch.int32),
                                "prefix_lens": torch.full((groups,), prefix, dtype=torch.int32)})


def c4_workload() -> PrefillWorkload:
    """C4: 4 prefill chunks of U{256..500} new tokens over U{0..3072} cached tokens,
    plus 48 decode rows with L ~ U{256..4096}; one 1.25x pool, random tables."""
    gen = torch.Generator().manual_seed(4)
    bs, hq, hkv, d = 16, 12, 2, 128
    n_new = torch.randint(256, 501, (4,), generator=gen).tolist()
    cached = torch.randint(0, 3073, (4,), generator=gen).tolist()
    dec_len = torch.randint(256, 4097, (48,), generator=gen).tolist()
    pre_ctx = [c + n for c, n in zip(cached, n_new)]
    pages_pre = [math.ceil(x / bs) for x in pre_ctx]
    pages_dec = [math.ceil(x / bs) for x in dec_len]
    need = sum(pages_pre) + sum(pages_dec)
    nb = math.ceil(1.25 * need)
    k_pool = _randn(gen, nb, bs, hkv, d)
    v_pool = _randn(gen, nb, bs, hkv, d)
    perm = torch.randperm(nb, generator=gen)
    width = 256
    t_pre = _tables_from_perm(perm[:sum(pages_pre)], pages_pre, width)
    t_dec = _tables_from_perm(perm[sum(pages_pre):need], pages_dec, width)
    total_q = sum(n_new)
    q = _randn(gen, total_q, hq, d)
    q_dec = _randn(gen, 48, hq, d)
    offs = [0]
    for n in n_new:
        offs.append(offs[-1] + n)
    dec = DecodeWorkload("C4-decode", q_dec, k_pool, v_pool, t_dec,
                         torch.tensor(dec_len, dtype=torch.int32), unique_tokens=sum(dec_len),
                         meta={"seed": 4})
    return PrefillWorkload("C4", q, torch.tensor(offs, dtype=torch.int32),
                           torch.tensor(pre_ctx, dtype=torch.int32), t_pre, k_pool, v_pool, dec,
                           meta={"seed": 4, "n_new": n_new, "cached": cached})
