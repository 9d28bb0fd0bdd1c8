"""INT8 / OCP-FP8 (e4m3fn) KV-cache quantisation with per-(page, KV-head) scales.

Drop-in for ``flashattn_tile/quant.py`` (same names and semantics):

* one fp32 scale per ``(page, kv_head)``, shape ``[num_pages, num_kv_heads]``,
  ``scale = max(absmax over (slot, dim) / {127 | 448}, 1e-8)``; the absmax
  covers every slot of the page (``quant.py:114-117``);
* int8: ``clamp(round_half_even(x / scale), -127, 127)`` (``quant.py:122-124``);
* fp8: ``clamp(x / scale, -448, 448).to(float8_e4m3fn)`` (``quant.py:125-127``);
* dequantise: ``(float(x) * scale).to(out_dtype)`` (``quant.py:145-161``).

On ROCm tensors the quantisation itself is the HIP kernel ``fat_quantize_pages``
(one pass over the pages, bit-exact to the formulas above); CPU tensors take
the torch expressions.  The HIP decode kernels apply the dequantisation in
registers (with fp16 queries: K staged as its exact 8-bit values and k_scale
applied to the fp32 scores, as the reference's quantised kernel does,
``kernels/decode.py:419-429``), so a quantised cache costs 1 byte per element
of HBM traffic plus 8 bytes of scales per (page, KV head).  On gfx950 float8_e4m3fn is the OCP encoding the hardware
converts natively (v_cvt_pk_f32_fp8), which is why it is the default format
whenever a ROCm device is present.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .paging import PagedKVCache, validate_cache

__all__ = [
    "FP8_DTYPE",
    "FP8_MAX",
    "INT8_MAX",
    "QuantScales",
    "available_quant_modes",
    "default_quant_mode",
    "quantize_kv_pages",
    "dequantize_kv_pages",
    "quantize_cache",
    "dequantize_cache",
    "kv_bytes_per_token",
]

FP8_DTYPE = getattr(torch, "float8_e4m3fn", None)
FP8_MAX = 448.0
INT8_MAX = 127.0
FP8_MIN_SCALE = 1e-8
INT8_MIN_SCALE = 1e-8


@dataclass
class QuantScales:
    """Per-(page, KV-head) dequantisation scales (``quant.py:36-48``)."""

    k: torch.Tensor
    v: torch.Tensor
    mode: str
    granularity: str = "per_page_per_head"

    def as_dict(self) -> dict:
        return {"k": self.k, "v": self.v, "mode": self.mode, "granularity": self.granularity}


def available_quant_modes() -> list[str]:
    modes = ["int8"]
    if FP8_DTYPE is not None:
        modes.insert(0, "float8_e4m3fn")
    return modes


def default_quant_mode() -> str:
    """``float8_e4m3fn`` when the dtype exists and a ROCm device is present
    (the gfx950 kernel consumes it), else ``int8`` (``quant.py:56-65``)."""
    if FP8_DTYPE is not None and torch.cuda.is_available():
        return "float8_e4m3fn"
    return "int8"


def _resolve_mode(mode: str) -> str:
    return default_quant_mode() if mode == "auto" else mode


def _quant_dtype(mode: str) -> torch.dtype:
    mode = _resolve_mode(mode)
    if mode == "int8":
        return torch.int8
    if mode in ("float8_e4m3fn", "fp8"):
        if FP8_DTYPE is None:
            raise RuntimeError("this PyTorch build has no torch.float8_e4m3fn")
        return FP8_DTYPE
    raise ValueError(f"unknown quantisation mode {mode!r}; expected 'int8' or 'float8_e4m3fn'")


def quantize_kv_pages(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    mode: str = "auto",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, dict]:
    """Quantise ``[num_pages, page_size, kv_heads, dim]`` float pages.

    Returns ``(qk, qv, scale_k, scale_v, info)`` (``quant.py:84-142``).
    """
    if k_cache.shape != v_cache.shape:
        raise ValueError(f"k/v shape mismatch: {tuple(k_cache.shape)} vs {tuple(v_cache.shape)}")
    if k_cache.dim() != 4:
        raise ValueError("cache must be [num_pages, page_size, num_kv_heads, head_dim]")
    if not k_cache.is_floating_point():
        raise ValueError(f"quantize_kv_pages expects a float cache, got {k_cache.dtype}")
    mode = _resolve_mode(mode)
    dtype = _quant_dtype(mode)
    is_int8 = mode == "int8"
    max_val = INT8_MAX if is_int8 else FP8_MAX
    min_scale = INT8_MIN_SCALE if is_int8 else FP8_MIN_SCALE
    _, page_size, kv_heads, head_dim = k_cache.shape

    if k_cache.is_cuda:
        from . import _hip

        def one(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
            # fat_quantize_pages (HIP): fp16/bf16/fp32 pages in, codes and
            # fp32 scales out; other float types are rounded to fp32 first,
            # as quant.py:111-112 does.
            src = x.detach()
            if src.dtype not in (torch.float16, torch.bfloat16, torch.float32):
                src = src.to(torch.float32)
            if src.stride(3) != 1:
                src = src.contiguous()
            codes = torch.empty(x.shape, dtype=dtype, device=x.device)
            scale = torch.empty(x.shape[0], x.shape[2], dtype=torch.float32, device=x.device)
            _hip.quantize_pages(src, codes, scale)
            return codes, scale
    else:
        def one(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
            xf = x.detach().to(torch.float32)
            scale = (xf.abs().amax(dim=(1, 3)) / max_val).clamp_min(min_scale)
            y = xf / scale[:, None, :, None]
            if is_int8:
                y = torch.round(y)
            return y.clamp(-max_val, max_val).to(dtype), scale

    qk, k_scale = one(k_cache)
    qv, v_scale = one(v_cache)
    if k_scale.numel():
        scale_min, scale_max = (float(x) for x in torch.stack([k_scale.min(), k_scale.max()]).cpu().tolist())
    else:
        scale_min = scale_max = 0.0
    info = {
        "mode": mode,
        "dtype": str(qk.dtype),
        "max_representable": max_val,
        "granularity": "per_page_per_head",
        "page_size": int(page_size),
        "num_kv_heads": int(kv_heads),
        "head_dim": int(head_dim),
        "scale_dtype": str(k_scale.dtype),
        "scale_min": scale_min,
        "scale_max": scale_max,
        "rounding": "round-to-nearest" if is_int8 else "cast-to-fp8",
    }
    return qk, qv, k_scale, v_scale, info


def dequantize_kv_pages(
    qk: torch.Tensor,
    qv: torch.Tensor,
    scale_k: torch.Tensor,
    scale_v: torch.Tensor,
    out_dtype: torch.dtype = torch.float16,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(float(x) * scale).to(out_dtype)`` per element (``quant.py:145-161``)."""
    if qk.shape != qv.shape:
        raise ValueError("quantised k/v shapes must match")
    if scale_k.shape != (qk.shape[0], qk.shape[2]):
        raise ValueError(f"scale_k shape {tuple(scale_k.shape)} must be [{qk.shape[0]}, {qk.shape[2]}]")
    k = qk.to(torch.float32) * scale_k.to(torch.float32)[:, None, :, None]
    v = qv.to(torch.float32) * scale_v.to(torch.float32)[:, None, :, None]
    return k.to(out_dtype), v.to(out_dtype)


def quantize_cache(cache: PagedKVCache, mode: str = "auto") -> tuple[PagedKVCache, QuantScales]:
    """New cache holding quantised K/V (same table and lengths) plus scales."""
    validate_cache(cache)
    qk, qv, sk, sv, info = quantize_kv_pages(cache.k_cache, cache.v_cache, mode=mode)
    quantized = PagedKVCache(k_cache=qk, v_cache=qv, page_table=cache.page_table,
                             seq_lens=cache.seq_lens, page_size=cache.page_size)
    return quantized, QuantScales(k=sk, v=sv, mode=info["mode"])


def dequantize_cache(cache: PagedKVCache, scales: QuantScales | dict,
                     out_dtype: torch.dtype = torch.float16) -> PagedKVCache:
    """Float copy of a quantised cache (debug/reference utility)."""
    sk = scales["k"] if isinstance(scales, dict) else scales.k
    sv = scales["v"] if isinstance(scales, dict) else scales.v
    k, v = dequantize_kv_pages(cache.k_cache, cache.v_cache, sk, sv, out_dtype=out_dtype)
    return PagedKVCache(k_cache=k, v_cache=v, page_table=cache.page_table,
                        seq_lens=cache.seq_lens, page_size=cache.page_size)


def kv_bytes_per_token(num_kv_heads: int, head_dim: int, storage: str = "fp16", page_size: int = 16) -> float:
    """Bytes of K+V per cached token including the fp32 scale overhead
    (``quant.py:194-208``): ``2*Hkv*D*elem + 2*Hkv*4/page_size``."""
    elem = {"fp16": 2, "bf16": 2, "fp32": 4, "int8": 1, "fp8": 1}[storage]
    return float(2 * num_kv_heads * head_dim * elem + 2 * num_kv_heads * 4 / page_size)
