"""The fused paged-cache validation reductions (``fat_cache_stats``) against
the torch reductions of the same quantities on the CPU copies: seq_lens
range, the page-table range over the columns the longest sequence uses
(flashattn_tile/paging.py:123-129) and the page count, including batches
above one workgroup's 1024 threads, empty and over-capacity sequences,
negative and out-of-pool ids, and a strided table."""

from __future__ import annotations

import pytest
import torch

from flashattntile_amd import PagedKVCache
from flashattntile_amd.paging import cache_stats

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cache(lens, table, page_size, num_pages=64):
    k = torch.zeros(num_pages, page_size, 1, 16, dtype=torch.float16)
    return PagedKVCache(k, k, table, torch.tensor(lens, dtype=torch.int32), page_size)


def _both(lens, table, page_size):
    cpu = _cache(lens, table, page_size)
    want = cache_stats(cpu, with_total_pages=True)
    dev = PagedKVCache(cpu.k_cache.to(DEV), cpu.v_cache.to(DEV), table.to(DEV), cpu.seq_lens.to(DEV), page_size)
    got = cache_stats(dev, with_total_pages=True)
    return got, want


@pytest.mark.parametrize("B", [1, 7, 1024, 1500, 3000])
@pytest.mark.parametrize("page_size", [1, 16, 64])
def test_cache_stats_match_the_torch_reductions(B, page_size):
    print(f"cache_stats B{B} P{page_size}", flush=True)
    g = torch.Generator().manual_seed(B + page_size)
    max_pages = 40
    lens = torch.randint(0, max_pages * page_size + 1, (B,), generator=g)
    lens[0] = 0
    table = torch.randint(-3, 70, (B, max_pages), generator=g, dtype=torch.int32)
    got, want = _both(lens.tolist(), table, page_size)
    assert got == want


def test_cache_stats_edge_cases():
    print("cache_stats edge cases", flush=True)
    table = torch.arange(12, dtype=torch.int32).view(3, 4)
    assert _both([0, 0, 0], table, 16)[0] == (0, 0, 0, -1, 0)   # nothing cached: no page range
    got, want = _both([-5, 3, 0], table, 16)                      # a negative length
    assert got == want and got[0] == -5
    got, want = _both([100, 1, 2], table, 16)                     # beyond the table's 64-token capacity
    assert got == want and got[1] == 100
    wide = torch.arange(60, dtype=torch.int32).view(3, 20) - 7
    strided = wide[:, 2:9]                                         # row stride 20, 7 columns
    got, want = _both([17, 40, 5], strided, 8)
    assert got == want and got[2] < 0
