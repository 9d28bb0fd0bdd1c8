"""Analytic work formulas (reference KATs, tests/test_autotune.py:13-50) and
the MI355X split heuristic."""

from __future__ import annotations

import pytest

from flashattntile_amd import autotune as at


def test_flops_causal_and_noncausal():
    assert at.flops_attention(1, 4, 2, 3, causal=False) == 96
    assert at.flops_attention(1, 4, 2, 3, causal=True) == 80
    assert at.flops_attention(8, 128, 1, 4096, causal=True, batch=4) == 4 * 4 * 8 * 128 * 4096


def test_flops_varlen_sums_sequences():
    total = at.flops_attention_varlen(2, 8, [1, 4], [10, 4], causal=True)
    assert total == at.flops_attention(2, 8, 1, 10, causal=True) + at.flops_attention(2, 8, 4, 4, causal=True)
    with pytest.raises(ValueError):
        at.flops_attention_varlen(2, 8, [1], [1, 2])


def test_bytes_decode_and_prefill():
    nbytes = at.bytes_attention("decode", 8, 1, 4096, 32, 8, 128, elem_bytes=2)
    assert nbytes == 8 * 4096 * 8 * 128 * 2 * 2 + 2 * 8 * 32 * 128 * 2
    assert 3.0 < at.arithmetic_intensity(at.flops_attention(32, 128, 1, 4096, True, 8), nbytes) < 5.0
    assert at.bytes_attention("prefill", 1, 1024, 1024, 32, 8, 128, 2) == 2 * (1024 * 32 * 128 * 2) + 1024 * 8 * 128 * 4
    with pytest.raises(ValueError):
        at.bytes_attention("backward", 1, 1, 1, 1, 1, 1)
    with pytest.raises(ValueError):
        at.bytes_attention("decode", 1, 2, 4, 1, 1, 1)


def test_baseline_work_numbers():
    """The roofline numerators quoted for the BASELINE configs."""
    assert at.bytes_attention("decode", 32, 1, 4096, 32, 8, 128) == 537_395_200
    assert at.bytes_decode_paged([4096] * 32, 32, 8, 128) == 537_395_200
    assert at.flops_attention(32, 128, 8192, 8192, causal=True) == 549_822_922_752
    assert at.flops_attention(32, 128, 512, 512, causal=True) == 2_151_677_952
    q = at.bytes_decode_paged([16384] * 128, 32, 8, 128, q_elem_bytes=2, kv_elem_bytes=1, page_size=16,
                              quantized=True)
    assert q == 4_305_453_056
    assert at.bytes_decode_paged([131072], 32, 8, 128) == 536_887_296


def test_split_heuristic():
    # the measured MI355X optima (32/8 heads, D128, page 16)
    assert at.decode_split_k(32, 32, 8, 256) == 1
    assert at.decode_split_k(8, 32, 8, 256) == 4
    assert at.decode_split_k(1, 32, 8, 64) == 8
    assert at.decode_split_k(1, 32, 8, 1024) == 16
    assert at.decode_split_k(1, 32, 8, 8192) == 16  # capped
    assert at.decode_split_k(128, 32, 8, 1024) == 1
    assert at.decode_split_k(1, 32, 8, 3) == 1  # partitions of at least 8 pages


def test_partition_heuristic():
    # uniform batches: same launches as decode_split_k
    assert at.decode_partition(32, 32, 8, 256, 32 * 256) == (1, 256)
    assert at.decode_partition(8, 32, 8, 256, 8 * 256) == (4, 64)
    assert at.decode_partition(1, 32, 8, 64, 64) == (8, 8)
    # capped at 16 partitions, pages re-spread over them
    assert at.decode_partition(1, 32, 8, 8192, 8192) == (16, 512)
    # skewed batch: small partitions (~16 workgroups per CU), split covers the longest sequence
    split, chunk = at.decode_partition(64, 32, 8, 4096, 40019)
    assert chunk == -(-40019 * 8 // (16 * 256)) and split == -(-4096 // chunk)
    assert split * chunk >= 4096 and split <= 64
