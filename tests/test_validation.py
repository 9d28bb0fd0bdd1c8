"""Input validation of the kernel wrappers: the reference's error types and
messages (tests/test_decode.py:197-216, tests/test_prefill.py:101-114),
raised on the host before any device work."""

from __future__ import annotations

import pytest
import torch

from flashattntile_amd.kernels.decode import paged_decode_attention, paged_decode_attention_fp8
from flashattntile_amd.kernels.prefill import prefill_attention
from flashattntile_amd.paging import allocate, append_tokens


def _cache(lens, page_size=16, kv_heads=2, head_dim=16, dtype=torch.float32):
    cache = allocate(len(lens), max(lens), kv_heads, head_dim, page_size, dtype=dtype)
    for _ in range(max(lens)):
        append_tokens(cache, torch.randn(len(lens), kv_heads, head_dim).to(dtype),
                      torch.randn(len(lens), kv_heads, head_dim).to(dtype))
    cache.seq_lens[:] = torch.tensor(lens, dtype=torch.int32)
    return cache


def test_decode_validation_errors():
    cache = _cache([5, 9])
    with pytest.raises(ValueError, match="q batch"):
        paged_decode_attention(torch.randn(3, 4, 16), cache)
    with pytest.raises(ValueError, match="divisible"):
        paged_decode_attention(torch.randn(2, 3, 16), cache)
    with pytest.raises(ValueError, match="head_dim"):
        paged_decode_attention(torch.randn(2, 4, 8), cache)
    with pytest.raises(ValueError, match="split_k"):
        paged_decode_attention(torch.randn(2, 4, 16), cache, config={"split_k": 0})
    with pytest.raises(ValueError, match="split_k"):
        paged_decode_attention(torch.randn(2, 4, 16), cache, config={"split_k": 65})
    with pytest.raises(ValueError, match="unknown decode config keys"):
        paged_decode_attention(torch.randn(2, 4, 16), cache, config={"BLOCK_N": 16})


def test_zero_length_sequence_is_rejected_for_decode():
    cache = _cache([4, 4])
    cache.seq_lens[1] = 0
    with pytest.raises(ValueError, match="at least one cached token"):
        paged_decode_attention(torch.randn(2, 4, 16), cache)


def test_decode_page_table_errors_surface():
    cache = _cache([8, 8], page_size=4)
    cache.page_table[0, 0] = cache.num_pages
    with pytest.raises(AssertionError, match="references page"):
        paged_decode_attention(torch.randn(2, 4, 16), cache)
    cache.page_table[0, 0] = -1
    with pytest.raises(AssertionError, match="negative page id"):
        paged_decode_attention(torch.randn(2, 4, 16), cache)


def test_quant_decode_validation():
    cache = _cache([5, 9])
    scales = {"k": torch.ones(cache.num_pages, 2), "v": torch.ones(cache.num_pages, 2)}
    with pytest.raises(ValueError, match="int8/float8"):
        paged_decode_attention_fp8(torch.randn(2, 4, 16), cache, scales)
    cache.k_cache = cache.k_cache.to(torch.int8)
    cache.v_cache = cache.v_cache.to(torch.int8)
    with pytest.raises(ValueError, match="scales must have shape"):
        paged_decode_attention_fp8(torch.randn(2, 4, 16), cache, {"k": torch.ones(1, 2), "v": torch.ones(1, 2)})


def _varlen(lens, h=2, hk=2, d=16):
    total = sum(lens)
    q = torch.randn(total, h, d)
    k = torch.randn(total, hk, d)
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0).tolist()), dtype=torch.int32)
    return q, k, k.clone(), cu


def test_prefill_config_validation_rejects_bad_blocks():
    q, k, v, cu = _varlen([3])
    with pytest.raises(ValueError, match="power of two"):
        prefill_attention(q, k, v, cu, cu, 3, 3, config={"BLOCK_M": 48})
    with pytest.raises(ValueError, match="unknown prefill config keys"):
        prefill_attention(q, k, v, cu, cu, 3, 3, config={"BLOCK_K": 32})


def test_prefill_invalid_offsets_rejected():
    q = torch.randn(4, 2, 16)
    bad = torch.tensor([0, 5], dtype=torch.int32)
    with pytest.raises(ValueError, match="must equal q.shape"):
        prefill_attention(q, q, q, bad, bad, 4, 4)
    with pytest.raises(ValueError, match="must be int32"):
        prefill_attention(q, q, q, bad.long(), bad.long(), 4, 4)
    cu_dec = torch.tensor([0, 3, 2, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match="non-decreasing"):
        prefill_attention(q, q, q, cu_dec, cu_dec, 4, 4)
    cq = torch.tensor([0, 4], dtype=torch.int32)
    ck = torch.tensor([0, 2], dtype=torch.int32)
    with pytest.raises(ValueError, match="kv_len >= q_len"):
        prefill_attention(q, q[:2], q[:2], cq, ck, 4, 2)


def test_prefill_max_seqlen_bounds():
    q, k, v, cu = _varlen([3, 7])
    with pytest.raises(ValueError, match="max_seqlen_q must be positive"):
        prefill_attention(q, k, v, cu, cu, 0, 7)
    with pytest.raises(ValueError, match="smaller than the longest query"):
        prefill_attention(q, k, v, cu, cu, 5, 7)
