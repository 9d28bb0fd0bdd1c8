"""The reference's import paths resolve to this build's modules (CPU only:
nothing here launches a kernel)."""

from __future__ import annotations

import importlib

import pytest
import torch

REFERENCE_MODULES = ["flashattn_tile.kernels.decode", "flashattn_tile.kernels.prefill", "flashattn_tile.paging",
                     "flashattn_tile.quant", "flashattn_tile.backend", "flashattn_tile.ops",
                     "flashattn_tile.autotune", "flashattn_tile.native", "flashattn_tile.env"]


@pytest.mark.parametrize("name", REFERENCE_MODULES)
def test_reference_module_path_is_the_same_module(name):
    ref_style = importlib.import_module(name)
    ours = importlib.import_module(name.replace("flashattn_tile", "flashattntile_amd", 1))
    assert ref_style is ours


def test_reference_style_imports():
    from flashattn_tile import PAGED_DECODE_OP, PREFILL_OP, PagedKVCache, allocate, append_tokens, gather_contiguous
    from flashattn_tile.backend import AttentionMetadata, FlashAttnTileBackend, get_kv_cache_shape
    from flashattn_tile.kernels.decode import paged_decode_attention, paged_decode_attention_fp8
    from flashattn_tile.kernels.prefill import prefill_attention
    from flashattn_tile.ops import ops_available
    from flashattn_tile.paging import gather_paged, validate_cache
    from flashattn_tile.quant import QuantScales, kv_bytes_per_token, quantize_kv_pages

    import flashattntile_amd as impl

    assert paged_decode_attention is impl.paged_decode_attention
    assert prefill_attention is impl.prefill_attention
    assert PagedKVCache is impl.PagedKVCache and allocate is impl.allocate
    assert ops_available() and hasattr(torch.ops.flashattn_tile, "paged_decode")
    assert PAGED_DECODE_OP.startswith("flashattn_tile::paged_decode") and PREFILL_OP.startswith("flashattn_tile::")
    assert FlashAttnTileBackend(32, 8, 128, 16).get_name() == "flashattn_tile"
    assert get_kv_cache_shape(4, 16, 8, 128) == (2, 4, 16, 8, 128)
    assert kv_bytes_per_token(8, 128, "fp16", 16) == 4100
    assert callable(paged_decode_attention_fp8) and callable(gather_paged) and callable(validate_cache)
    assert callable(append_tokens) and callable(gather_contiguous) and callable(quantize_kv_pages)
    assert QuantScales is impl.QuantScales


def test_package_attribute_access():
    import flashattn_tile

    assert flashattn_tile.kernels.decode.paged_decode_attention is flashattn_tile.paged_decode_attention
    assert flashattn_tile.paging.PagedKVCache is flashattn_tile.PagedKVCache
    assert not hasattr(flashattn_tile, "reference")  # the oracle is test infrastructure, not product
