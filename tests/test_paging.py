"""Page-table contract (behaviour of the reference's tests/test_paging.py)."""

from __future__ import annotations

import math

import pytest
import torch

from flashattntile_amd.paging import (
    PagedKVCache,
    allocate,
    append_tokens,
    gather_contiguous,
    gather_paged,
    validate_cache,
)

DTYPE = torch.float32


def _append_steps(cache, ks, vs):
    for t in range(ks.shape[0]):
        append_tokens(cache, ks[t], vs[t])


@pytest.mark.parametrize(
    "batch, lens, page_size, kv_heads, head_dim",
    [(3, [1, 5, 17], 4, 2, 8), (1, [16], 16, 1, 4), (4, [31, 32, 33, 1], 16, 2, 16), (2, [7, 8], 8, 4, 8)],
)
def test_append_then_gather_roundtrip(batch, lens, page_size, kv_heads, head_dim):
    torch.manual_seed(0)
    cache = allocate(batch, max(lens), kv_heads, head_dim, page_size, dtype=DTYPE)
    assert cache.num_pages == batch * math.ceil(max(lens) / page_size)
    steps = max(lens)
    ks = torch.randn(steps, batch, kv_heads, head_dim)
    vs = torch.randn(steps, batch, kv_heads, head_dim)
    _append_steps(cache, ks, vs)
    cache.seq_lens[:] = torch.tensor(lens, dtype=torch.int32)
    exp_k = torch.zeros(batch, steps, kv_heads, head_dim)
    exp_v = torch.zeros_like(exp_k)
    for b, n in enumerate(lens):
        exp_k[b, :n] = ks[:n, b]
        exp_v[b, :n] = vs[:n, b]
    gk, gv = gather_contiguous(cache)
    torch.testing.assert_close(gk, exp_k, rtol=0, atol=0)
    torch.testing.assert_close(gv, exp_v, rtol=0, atol=0)


def test_page_table_indirection_with_permuted_pages():
    torch.manual_seed(1)
    cache = allocate(2, 13, 2, 8, 4, dtype=DTYPE)
    perm = torch.randperm(cache.num_pages)
    cache.page_table = perm[cache.page_table.long()].to(torch.int32)
    validate_cache(cache)
    ks = torch.randn(13, 2, 2, 8)
    vs = torch.randn(13, 2, 2, 8)
    _append_steps(cache, ks, vs)
    gk, gv = gather_contiguous(cache)
    for b in range(2):
        torch.testing.assert_close(gk[b], ks[:, b], rtol=0, atol=0)
        torch.testing.assert_close(gv[b], vs[:, b], rtol=0, atol=0)


def test_append_respects_page_capacity():
    cache = allocate(1, max_seq_len=4, num_kv_heads=1, head_dim=4, page_size=2, dtype=DTYPE)
    assert cache.capacity == 4
    for _ in range(4):
        append_tokens(cache, torch.zeros(1, 1, 4), torch.zeros(1, 1, 4))
    assert cache.seq_lens.tolist() == [4]
    with pytest.raises(AssertionError, match="capacity"):
        append_tokens(cache, torch.zeros(1, 1, 4), torch.zeros(1, 1, 4))


def test_out_of_bounds_page_table_is_rejected():
    cache = allocate(2, 8, 1, 4, page_size=4, dtype=DTYPE)
    cache.seq_lens[:] = 8
    cache.page_table[0, 0] = cache.num_pages
    with pytest.raises(AssertionError, match="references page"):
        validate_cache(cache)
    with pytest.raises(AssertionError, match="page id outside"):
        gather_paged(cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, cache.page_size)
    cache.page_table[0, 0] = -1
    with pytest.raises(AssertionError, match="negative page id"):
        validate_cache(cache)


def test_validate_checks_the_reference_slice_only():
    """Entries past ceil(max_len / P) are ignored (paging.py:123-129)."""
    cache = allocate(2, 16, 1, 4, page_size=4, dtype=DTYPE)
    cache.seq_lens[:] = torch.tensor([5, 3], dtype=torch.int32)  # max 5 -> 2 pages checked
    cache.page_table[:, 2:] = -7
    assert validate_cache(cache) == (3, 5)
    cache.page_table[1, 1] = -7  # inside the checked slice for every row
    with pytest.raises(AssertionError, match="negative page id"):
        validate_cache(cache)


def test_seq_len_over_capacity_rejected():
    cache = allocate(1, 8, 1, 4, page_size=4, dtype=DTYPE)
    cache.seq_lens[0] = 9
    with pytest.raises(AssertionError, match="exceeds page-table capacity"):
        validate_cache(cache)
    cache.seq_lens[0] = -1
    with pytest.raises(AssertionError, match="non-negative"):
        validate_cache(cache)


def test_append_validates_dtype_and_shape():
    cache = allocate(2, 4, 2, 4, page_size=2, dtype=torch.float16)
    bad_dtype = torch.zeros(2, 2, 4, dtype=torch.float32)
    with pytest.raises(AssertionError, match="dtype"):
        append_tokens(cache, bad_dtype, bad_dtype)
    bad_shape = torch.zeros(2, 3, 4, dtype=torch.float16)
    with pytest.raises(AssertionError, match="new_k must be"):
        append_tokens(cache, bad_shape, bad_shape)


@pytest.mark.parametrize("bad_dtype", [torch.int64, torch.int16])
def test_page_table_dtype_is_strict(bad_dtype):
    cache = allocate(1, 4, 1, 4, page_size=2, dtype=DTYPE)
    cache.page_table = cache.page_table.to(bad_dtype)
    with pytest.raises(AssertionError, match="page_table must be int32"):
        validate_cache(cache)


def test_gather_paged_handles_zero_length_sequences():
    cache = allocate(3, 8, 2, 4, page_size=4, dtype=DTYPE)
    for t in range(5):
        append_tokens(cache, torch.full((3, 2, 4), float(t)), torch.full((3, 2, 4), float(t) + 100.0))
    cache.seq_lens[:] = torch.tensor([3, 0, 2], dtype=torch.int32)
    gk, gv = gather_contiguous(cache)
    assert gk.shape == (3, 3, 2, 4)
    assert torch.all(gk[0, :3] == torch.tensor([0.0, 1.0, 2.0]).view(3, 1, 1))
    assert torch.all(gk[1] == 0)
    assert torch.all(gk[2, :2] == torch.tensor([0.0, 1.0]).view(2, 1, 1))
    assert torch.all(gv[2, :2] == torch.tensor([100.0, 101.0]).view(2, 1, 1))


def test_cache_properties():
    cache = allocate(3, 40, 2, 16, page_size=16, dtype=torch.bfloat16)
    assert (cache.batch_size, cache.num_pages, cache.num_kv_heads, cache.head_dim) == (3, 9, 2, 16)
    assert cache.max_pages_per_seq == 3 and cache.capacity == 48
    assert isinstance(cache, PagedKVCache)
