"""Paged bf16 KV cache shared by the full-attention layers.

The reference stores each full layer's KV as one contiguous fp32 tensor that
grows by ``torch.cat`` per token, slot of token p == p, no eviction
(v2/src/router_ia/qwen36_attention_cache.py:334-373).  Here every layer keeps
16-token pages in one preallocated HBM pool; a per-sequence page table maps
logical token t to physical slot ``page_table[row][t // 16] * 16 + t % 16``.
All full layers of a sequence share one page table (they hold the same token
positions), so pages are allocated once per 16 tokens for all layers.

Page layout per layer (bf16, or fp16 for fp16 activations), one 8 KiB tile
per (page, KV head):
    K  [num_pages, Hkv, 8, 4, 16 tokens, 8]  key (token t, dim d) at
       [.., (d % 64) // 8, d // 64, t, d % 8]: the order in which the decode
       kernel's MFMA operand loads read it, one contiguous 1 KiB per load
    V  [num_pages, Hkv, 256 dims, 16 tokens]   (transposed inside the page)
"""

from __future__ import annotations

import random

import torch

from .kernels import ATTN_HEAD_DIM, K_TILE_SHAPE, PAGE_TOKENS


class PageAllocator:
    """Host-side free list and page tables (authoritative copy of the device table)."""

    def __init__(self, num_pages: int, max_seqs: int, max_pages_per_seq: int, *, shuffle_seed: int | None = None):
        if num_pages <= 0 or max_seqs <= 0 or max_pages_per_seq <= 0:
            raise ValueError("num_pages, max_seqs and max_pages_per_seq must be positive")
        self.num_pages = num_pages
        self.max_seqs = max_seqs
        self.max_pages_per_seq = max_pages_per_seq
        free = list(range(num_pages))
        if shuffle_seed is not None:
            random.Random(shuffle_seed).shuffle(free)
        free.reverse()  # pop() hands out pages in list order
        self._free = free
        self.tables: list[list[int]] = [[] for _ in range(max_seqs)]

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def capacity_tokens(self, row: int) -> int:
        return len(self.tables[row]) * PAGE_TOKENS

    def ensure(self, row: int, n_tokens: int) -> list[tuple[int, int]]:
        """Make row hold n_tokens; return the (logical page, physical page) pairs added."""
        need = (n_tokens + PAGE_TOKENS - 1) // PAGE_TOKENS
        if need > self.max_pages_per_seq:
            raise RuntimeError(
                f"sequence row {row} needs {need} pages, page table holds {self.max_pages_per_seq}"
            )
        table = self.tables[row]
        if need - len(table) > len(self._free):
            # all-or-nothing: a failed request leaves the row and the free list unchanged
            raise RuntimeError(f"KV page pool exhausted: row {row} needs {need - len(table)} more pages, "
                               f"{len(self._free)} free")
        added = []
        while len(table) < need:
            page = self._free.pop()
            added.append((len(table), page))
            table.append(page)
        return added

    def pages_needed(self, n_tokens: list[int]) -> int:
        """Pages rows 0..len-1 must take to hold n_tokens[row] tokens; raises if a row's table is too narrow."""
        total = 0
        for row, n in enumerate(n_tokens):
            need = (n + PAGE_TOKENS - 1) // PAGE_TOKENS
            if need > self.max_pages_per_seq:
                raise RuntimeError(
                    f"sequence row {row} needs {need} pages, page table holds {self.max_pages_per_seq}"
                )
            total += max(0, need - len(self.tables[row]))
        return total

    def release(self, row: int) -> None:
        table = self.tables[row]
        self._free.extend(reversed(table))
        table.clear()

    def slot_of(self, row: int, token: int) -> int:
        """Physical slot (page * 16 + offset) of logical token `token` of `row`."""
        return self.tables[row][token // PAGE_TOKENS] * PAGE_TOKENS + token % PAGE_TOKENS


class PagedKVCache:
    """Per-layer K/V page pools plus the device page table."""

    def __init__(
        self,
        num_layers: int,
        num_pages: int,
        max_seqs: int,
        max_pages_per_seq: int,
        *,
        num_kv_heads: int,
        device: torch.device | str,
        shuffle_seed: int | None = None,
        dtype: torch.dtype = torch.bfloat16,
    ):
        if dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("the KV cache holds bf16 or fp16")
        self.device = torch.device(device)
        self.dtype = dtype
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.alloc = PageAllocator(num_pages, max_seqs, max_pages_per_seq, shuffle_seed=shuffle_seed)
        self.k = torch.zeros((num_layers, num_pages, num_kv_heads, *K_TILE_SHAPE), dtype=dtype, device=self.device)
        self.v = torch.zeros((num_layers, num_pages, num_kv_heads, ATTN_HEAD_DIM, PAGE_TOKENS), dtype=dtype,
                             device=self.device)
        self.page_table = torch.full((max_seqs, max_pages_per_seq), -1, dtype=torch.int32, device=self.device)

    def ensure(self, row: int, n_tokens: int) -> None:
        added = self.alloc.ensure(row, n_tokens)
        if added:
            cols = torch.tensor([c for c, _ in added], dtype=torch.long)
            vals = torch.tensor([p for _, p in added], dtype=torch.int32)
            host_row = self.page_table[row].cpu()
            host_row[cols] = vals
            self.page_table[row].copy_(host_row)

    def ensure_many(self, n_tokens: list[int]) -> None:
        """ensure() for rows 0..len-1 with one table upload, all or nothing.

        Every row's need is checked against the page-table width and the free
        list before any page is taken, so a request that cannot be met raises
        with the host tables, the free list and the device table unchanged.
        """
        need = self.alloc.pages_needed(n_tokens)
        if need > self.alloc.free_pages:
            raise RuntimeError(f"KV page pool exhausted: {need} more pages needed, {self.alloc.free_pages} free")
        changed = False
        try:
            for row, n in enumerate(n_tokens):
                if self.alloc.ensure(row, n):
                    changed = True
        finally:
            if changed:
                self.upload_tables()

    def upload_tables(self) -> None:
        host = torch.full(tuple(self.page_table.shape), -1, dtype=torch.int32)
        for row, table in enumerate(self.alloc.tables):
            if table:
                host[row, : len(table)] = torch.tensor(table, dtype=torch.int32)
        self.page_table.copy_(host)

    def release(self, row: int) -> None:
        self.alloc.release(row)
        self.page_table[row].fill_(-1)

    def write_tokens(self, layer: int, row: int, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Store already-positioned K/V rows [T, Hkv, 256] at logical tokens start..start+T of `row`.

        Bulk loader for resident context (prefilled caches, restored state); the
        per-token decode path appends through ria_kv_append instead.  Pages must
        already be allocated.
        """
        count = int(k.shape[0])
        if count == 0:
            return
        table = self.alloc.tables[row]
        if (start + count + PAGE_TOKENS - 1) // PAGE_TOKENS > len(table):
            raise RuntimeError("write_tokens beyond the row's allocated pages")
        tok = torch.arange(start, start + count)
        pages = torch.tensor(table, dtype=torch.long)[tok // PAGE_TOKENS].to(self.device)
        offs = (tok % PAGE_TOKENS).to(self.device)
        kb = k.to(device=self.device, dtype=self.dtype)
        vb = v.to(device=self.device, dtype=self.dtype)
        dims = torch.arange(ATTN_HEAD_DIM, device=self.device)
        kk, g, j = (dims % 64) // 8, dims // 64, dims % 8
        pg, of = pages[:, None], offs[:, None]
        for h in range(self.num_kv_heads):
            self.k[layer, pg, h, kk[None, :], g[None, :], of, j[None, :]] = kb[:, h, :]
            self.v[layer, pages, h, :, offs] = vb[:, h, :]

    def key_row(self, layer: int, page: int, head: int, offset: int) -> torch.Tensor:
        """The 256-dim key stored at (page, head, token offset), in dim order."""
        tile = self.k[layer, page, head]  # [8 (kk), 4 (g), 16, 8 (j)]
        return tile[:, :, offset, :].permute(1, 0, 2).reshape(ATTN_HEAD_DIM)

    def layer(self, idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.k[idx], self.v[idx]

    def bytes_per_token(self) -> int:
        return self.num_layers * 2 * self.num_kv_heads * ATTN_HEAD_DIM * 2
