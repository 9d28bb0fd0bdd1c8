"""The paged-cache contract on CPU tensors (flashattntile_amd/paging.py).

Behaviour and error texts follow the reference's ``flashattn_tile/paging.py``
(append ``:172-210``, gather ``:213-262``, validation ``:84-130``); the cases
here are this repo's own:

* a model-based check: random decode schedules append into caches of random
  geometry while a plain Python shadow records which token each sequence
  holds; gather must return exactly the shadow, before and after the pool is
  permuted and the sequences are cut to ragged lengths;
* a table of corruptions (bad ids, lengths, dtypes, shapes), each with the
  exception and message the contract names.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from flashattntile_amd.paging import (PagedKVCache, allocate, append_tokens, gather_contiguous, gather_paged,
                                      validate_cache)


class Shadow:
    """Tokens each sequence holds, as the list of (k, v) rows appended."""

    def __init__(self, batch: int) -> None:
        self.rows: list[list[tuple[torch.Tensor, torch.Tensor]]] = [[] for _ in range(batch)]

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        for b, seq in enumerate(self.rows):
            seq.append((k[b].clone(), v[b].clone()))

    def cut(self, lens: list[int]) -> None:
        self.rows = [seq[:n] for seq, n in zip(self.rows, lens)]

    def expected(self, heads: int, dim: int) -> tuple[torch.Tensor, torch.Tensor]:
        longest = max((len(s) for s in self.rows), default=0)
        k = torch.zeros(len(self.rows), longest, heads, dim)
        v = torch.zeros_like(k)
        for b, seq in enumerate(self.rows):
            for t, (kr, vr) in enumerate(seq):
                k[b, t], v[b, t] = kr, vr
        return k, v


def _permute_pool(cache: PagedKVCache, rng: random.Random) -> None:
    """Move every physical page to a new slot and rewrite the table to match."""
    n = cache.num_pages
    new_of_old = list(range(n))
    rng.shuffle(new_of_old)
    dst = torch.tensor(new_of_old)
    k, v = cache.k_cache.clone(), cache.v_cache.clone()
    cache.k_cache[dst] = k
    cache.v_cache[dst] = v
    cache.page_table = dst[cache.page_table.long()].to(torch.int32)


@pytest.mark.parametrize("seed", range(8))
def test_append_gather_matches_a_shadow_of_the_appends(seed):
    rng = random.Random(seed)
    batch = rng.randint(1, 5)
    page = rng.choice([1, 2, 3, 4, 8, 16])
    heads, dim = rng.choice([1, 2, 4]), rng.choice([4, 8, 16])
    max_len = rng.randint(1, 40)
    cache = allocate(batch, max_len, heads, dim, page, dtype=torch.float32)
    assert cache.num_pages == batch * math.ceil(max_len / page)
    assert cache.capacity >= max_len and cache.capacity - max_len < page
    shadow = Shadow(batch)
    g = torch.Generator().manual_seed(seed)
    steps = rng.randint(0, max_len)
    for step in range(steps):
        k = torch.randn(batch, heads, dim, generator=g)
        v = torch.randn(batch, heads, dim, generator=g)
        append_tokens(cache, k, v)
        shadow.append(k, v)
        assert cache.seq_lens.tolist() == [step + 1] * batch
        if rng.random() < 0.3:  # relocating pages changes nothing a reader sees
            _permute_pool(cache, rng)
    for phase in ("full", "ragged"):
        if phase == "ragged":
            lens = [rng.randint(0, steps) for _ in range(batch)]
            cache.seq_lens = torch.tensor(lens, dtype=torch.int32)
            shadow.cut(lens)
        want_k, want_v = shadow.expected(heads, dim)
        got_k, got_v = gather_contiguous(cache)
        assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v), (seed, phase)
        direct = gather_paged(cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, page)
        assert torch.equal(direct[0], want_k) and torch.equal(direct[1], want_v)


def test_token_lands_at_table_page_and_slot():
    """Token t of sequence b is slot t % P of page table[b, t // P]."""
    cache = allocate(2, 7, 1, 2, 3, dtype=torch.float32)
    cache.page_table = torch.tensor([[5, 0, 3], [1, 4, 2]], dtype=torch.int32)
    for t in range(7):
        vals = torch.tensor([[[10.0 + t, 0.0]], [[20.0 + t, 0.0]]])
        append_tokens(cache, vals, -vals)
    for b, base in ((0, 10.0), (1, 20.0)):
        for t in range(7):
            page = int(cache.page_table[b, t // 3])
            assert cache.k_cache[page, t % 3, 0, 0].item() == base + t
            assert cache.v_cache[page, t % 3, 0, 0].item() == -(base + t)


def test_gather_pads_with_zeros_and_skips_empty_sequences():
    cache = allocate(3, 6, 2, 4, 2, dtype=torch.float32)
    for t in range(6):
        append_tokens(cache, torch.full((3, 2, 4), t + 1.0), torch.full((3, 2, 4), -(t + 1.0)))
    cache.seq_lens = torch.tensor([0, 6, 1], dtype=torch.int32)
    k, v = gather_contiguous(cache)
    assert k.shape == (3, 6, 2, 4)
    assert torch.all(k[0] == 0) and torch.all(v[0] == 0)
    assert k[1, :, 0, 0].tolist() == [1.0, 2.0, 3.0, 4.0, 5.0, 6.0]
    assert k[2, 0, 0, 0].item() == 1.0 and torch.all(k[2, 1:] == 0) and v[2, 0, 1, 3].item() == -1.0
    cache.seq_lens = torch.zeros(3, dtype=torch.int32)
    assert gather_contiguous(cache)[0].shape == (3, 0, 2, 4)


def test_validate_reads_only_the_pages_in_use():
    """Entries past ceil(max(seq_lens) / P) are never read (paging.py:123-129),
    so garbage there is accepted; inside that slice every row is checked."""
    cache = allocate(3, 20, 1, 4, 4, dtype=torch.float32)
    cache.seq_lens = torch.tensor([2, 9, 0], dtype=torch.int32)  # 3 pages in use
    cache.page_table[:, 3:] = 10_000
    assert validate_cache(cache) == (0, 9)
    cache.page_table[2, 2] = -3  # row 2 holds no token, but the slice is shared
    with pytest.raises(AssertionError, match="negative page id"):
        validate_cache(cache)


def _corrupt(kind: str):
    """A small valid cache, then one corruption; returns (callable, exc, msg)."""
    cache = allocate(2, 8, 1, 4, 4, dtype=torch.float16)
    zeros = torch.zeros(2, 1, 4, dtype=torch.float16)
    if kind == "page id past the pool":
        cache.seq_lens[:] = 5
        cache.page_table[1, 1] = cache.num_pages + 2
        return (lambda: validate_cache(cache)), AssertionError, "references page"
    if kind == "gather with a page id past the pool":
        cache.seq_lens[:] = 5
        cache.page_table[0, 1] = cache.num_pages
        return (lambda: gather_paged(cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, 4)), \
            AssertionError, "page id outside"
    if kind == "negative page id":
        cache.seq_lens[:] = 1
        cache.page_table[0, 0] = -1
        return (lambda: validate_cache(cache)), AssertionError, "negative page id"
    if kind == "length past the table":
        cache.seq_lens[1] = cache.capacity + 1
        return (lambda: validate_cache(cache)), AssertionError, "exceeds page-table capacity"
    if kind == "negative length":
        cache.seq_lens[0] = -2
        return (lambda: validate_cache(cache)), AssertionError, "non-negative"
    if kind == "int64 page table":
        cache.page_table = cache.page_table.long()
        return (lambda: validate_cache(cache)), AssertionError, "page_table must be int32"
    if kind == "int16 page table":
        cache.page_table = cache.page_table.to(torch.int16)
        return (lambda: validate_cache(cache)), AssertionError, "page_table must be int32"
    if kind == "int64 lengths":
        cache.seq_lens = cache.seq_lens.long()
        return (lambda: validate_cache(cache)), AssertionError, "seq_lens must be int32"
    if kind == "append past capacity":
        cache.seq_lens[:] = cache.capacity
        return (lambda: append_tokens(cache, zeros, zeros)), AssertionError, "capacity"
    if kind == "append in the wrong dtype":
        return (lambda: append_tokens(cache, zeros.float(), zeros.float())), AssertionError, "dtype"
    if kind == "append of the wrong shape":
        bad = torch.zeros(2, 2, 4, dtype=torch.float16)
        return (lambda: append_tokens(cache, bad, bad)), AssertionError, "new_k must be"
    if kind == "k and v pools disagree":
        cache.v_cache = cache.v_cache[:-1]
        return (lambda: validate_cache(cache)), AssertionError, "must match"
    raise KeyError(kind)


@pytest.mark.parametrize("kind", [
    "page id past the pool", "gather with a page id past the pool", "negative page id", "length past the table",
    "negative length", "int64 page table", "int16 page table", "int64 lengths", "append past capacity",
    "append in the wrong dtype", "append of the wrong shape", "k and v pools disagree",
])
def test_contract_violations_raise_with_the_named_message(kind):
    fn, exc, msg = _corrupt(kind)
    with pytest.raises(exc, match=msg):
        fn()


def test_append_fills_to_capacity_exactly():
    """A full table accepts appends up to its capacity and no further, and a
    failed append leaves the cache untouched."""
    cache = allocate(1, 6, 1, 2, 3, dtype=torch.float32)
    for t in range(cache.capacity):
        append_tokens(cache, torch.full((1, 1, 2), float(t)), torch.zeros(1, 1, 2))
    before = cache.k_cache.clone()
    with pytest.raises(AssertionError, match="capacity"):
        append_tokens(cache, torch.ones(1, 1, 2), torch.ones(1, 1, 2))
    assert cache.seq_lens.tolist() == [6] and torch.equal(cache.k_cache, before)


def test_geometry_properties():
    cache = allocate(5, 33, 3, 8, 8, dtype=torch.bfloat16)
    assert isinstance(cache, PagedKVCache)
    assert (cache.batch_size, cache.num_pages, cache.num_kv_heads, cache.head_dim) == (5, 25, 3, 8)
    assert (cache.max_pages_per_seq, cache.page_size, cache.capacity) == (5, 8, 40)
    assert cache.page_table.tolist()[2] == [10, 11, 12, 13, 14]
    assert cache.seq_lens.tolist() == [0] * 5 and cache.k_cache.dtype == torch.bfloat16
