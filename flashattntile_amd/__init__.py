"""flashattntile_amd: the FlashAttnTile attention hot path, MI355X-native.

Drop-in for the reference package's operator surface
(``flashattn_tile/__init__.py:22-39``): importing registers the
``flashattn_tile::paged_decode`` / ``flashattn_tile::prefill_varlen`` custom
ops (plus the extensions ``flashattn_tile::paged_decode_quant`` and
``flashattn_tile::prefill_paged``), and the cache contract,
quantisation helpers, kernel wrappers and backend keep their names.  Every op
executes hand-written gfx950 HIP kernels (``csrc/``) through the C ABI of
``include/fat_abi.h``; there is no CPU fallback.  The reference's fp32 oracle
is test infrastructure here and lives outside the package (``oracle/``).
"""

from __future__ import annotations

__version__ = "0.1.0"

from . import ops as _ops  # noqa: F401  (registers the custom ops)
from .kernels.decode import (DecodeLaunch, paged_decode_attention, paged_decode_attention_fp8,
                             paged_decode_attention_multi)
from .kernels.prefill import paged_prefill_attention, prefill_attention
from .ops import (PAGED_DECODE_MULTI_OP, PAGED_DECODE_OP, PAGED_DECODE_QUANT_OP, PREFILL_OP, PREFILL_PAGED_OP,
                  paged_decode, paged_decode_multi, paged_decode_quant, prefill_paged, prefill_varlen)
from .paging import (AppendLaunch, PagedKVCache, allocate, append_tokens, gather_contiguous, gather_paged,
                     validate_cache)
from .quant import QuantScales, dequantize_cache, kv_bytes_per_token, quantize_cache

__all__ = [
    "__version__",
    "PAGED_DECODE_OP",
    "PREFILL_OP",
    "PAGED_DECODE_QUANT_OP",
    "PREFILL_PAGED_OP",
    "PAGED_DECODE_MULTI_OP",
    "paged_decode",
    "prefill_varlen",
    "paged_decode_quant",
    "prefill_paged",
    "paged_decode_multi",
    "paged_prefill_attention",
    "paged_decode_attention",
    "paged_decode_attention_fp8",
    "paged_decode_attention_multi",
    "DecodeLaunch",
    "prefill_attention",
    "PagedKVCache",
    "allocate",
    "append_tokens",
    "AppendLaunch",
    "gather_contiguous",
    "gather_paged",
    "validate_cache",
    "QuantScales",
    "quantize_cache",
    "dequantize_cache",
    "kv_bytes_per_token",
]
