"""Host-side paging: allocator, slot mapping and the K-tile layout (no GPU needed)."""

from __future__ import annotations

import pytest
import torch

from router_ia import kernels as K
from router_ia.paged_kv import PageAllocator, PagedKVCache


def test_slot_mapping_is_page_table_times_16_plus_offset() -> None:
    alloc = PageAllocator(64, 3, 8, shuffle_seed=5)
    alloc.ensure(0, 40)
    alloc.ensure(1, 1)
    alloc.ensure(2, 16)
    for row, n in ((0, 40), (1, 1), (2, 16)):
        for t in range(n):
            assert alloc.slot_of(row, t) == alloc.tables[row][t // 16] * 16 + t % 16
    used = [p for row in range(3) for p in alloc.tables[row]]
    assert len(used) == len(set(used)) == 3 + 1 + 1  # no page handed out twice


def test_shuffle_is_deterministic_and_not_identity() -> None:
    a = PageAllocator(100, 1, 100, shuffle_seed=4)
    b = PageAllocator(100, 1, 100, shuffle_seed=4)
    a.ensure(0, 1600)
    b.ensure(0, 1600)
    assert a.tables[0] == b.tables[0]
    assert sorted(a.tables[0]) == list(range(100)) and a.tables[0] != list(range(100))
    c = PageAllocator(100, 1, 100)
    c.ensure(0, 1600)
    assert c.tables[0] == list(range(100))


def test_release_returns_pages_and_errors_are_raised() -> None:
    alloc = PageAllocator(4, 2, 3)
    alloc.ensure(0, 48)
    assert alloc.free_pages == 1
    with pytest.raises(RuntimeError, match="exhausted"):
        alloc.ensure(1, 32)
    alloc.release(0)
    assert alloc.free_pages == 4 and alloc.tables[0] == []
    with pytest.raises(RuntimeError, match="page table holds"):
        alloc.ensure(1, 64)


def test_write_tokens_layout_round_trips_on_host() -> None:
    cache = PagedKVCache(2, 8, 2, 4, num_kv_heads=2, device="cpu", shuffle_seed=1)
    cache.ensure_many([37, 5])
    k = torch.randn(37, 2, 256).to(torch.bfloat16)
    v = torch.randn(37, 2, 256).to(torch.bfloat16)
    cache.write_tokens(1, 0, 0, k, v)
    for t in (0, 15, 16, 36):
        page, off = divmod(cache.alloc.slot_of(0, t), 16)
        for h in range(2):
            assert torch.equal(cache.key_row(1, page, h, off), k[t, h])
            assert torch.equal(cache.v[1, page, h, :, off], v[t, h])
    host = cache.page_table
    assert host[0, :3].tolist() == cache.alloc.tables[0] and host[0, 3].item() == -1


def test_k_tile_index_is_the_mfma_operand_order() -> None:
    # Lane l = g*16 + t of load kk reads 8 contiguous elements at (kk*64 + l)*8:
    # key dims 64*g + 8*kk .. +8 of token t.
    tile = torch.zeros(K.K_TILE_SHAPE, dtype=torch.int64)
    for t in range(16):
        for d in range(256):
            tile[K.k_tile_index(t, d)] = t * 1000 + d
    flat = tile.reshape(-1)
    for kk in range(8):
        for lane in range(64):
            t, g = lane % 16, lane // 16
            seg = flat[(kk * 64 + lane) * 8:(kk * 64 + lane) * 8 + 8].tolist()
            assert seg == [t * 1000 + 64 * g + 8 * kk + j for j in range(8)]


def _tables_tensor(cache: PagedKVCache) -> torch.Tensor:
    host = torch.full(tuple(cache.page_table.shape), -1, dtype=torch.int32)
    for row, table in enumerate(cache.alloc.tables):
        host[row, : len(table)] = torch.tensor(table, dtype=torch.int32) if table else host[row, :0]
    return host


def test_ensure_many_is_all_or_nothing_on_pool_exhaustion() -> None:
    cache = PagedKVCache(1, 10, 3, 8, num_kv_heads=2, device="cpu", shuffle_seed=3)
    cache.ensure_many([40, 16, 1])  # 3 + 1 + 1 pages
    before = [list(t) for t in cache.alloc.tables]
    free_before = cache.alloc.free_pages
    # rows 0 and 1 could grow, row 2 cannot: nothing may change
    with pytest.raises(RuntimeError, match="exhausted"):
        cache.ensure_many([64, 48, 80])
    assert [list(t) for t in cache.alloc.tables] == before
    assert cache.alloc.free_pages == free_before
    assert torch.equal(cache.page_table, _tables_tensor(cache))
    # a row whose table is too narrow fails the same way
    with pytest.raises(RuntimeError, match="page table holds"):
        cache.ensure_many([48, 200, 1])
    assert [list(t) for t in cache.alloc.tables] == before
    # a request that fits goes through, and the device table follows the host tables
    cache.ensure_many([64, 32, 17])
    assert torch.equal(cache.page_table, _tables_tensor(cache))
    assert cache.alloc.free_pages == 10 - 4 - 2 - 2
