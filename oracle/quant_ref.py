"""KV-cache quantisation restated for the oracle -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module.

Restates ``flashattn_tile/quant.py`` (read, not run):

``quantize_pages``  (quant.py:84-142)
    per-(page, kv_head) ``scale = max(absmax / qmax, 1e-8)`` with qmax 127
    (int8, round-half-even then clamp) or 448 (fp8 e4m3fn: clamp then cast).
``dequantize_pages``  (quant.py:145-161)
    ``(float(x) * scale).to(out_dtype)``.
``fp8_e4m3fn_value``
    the OCP e4m3fn decoding from its bit fields (1 sign, 4 exponent bits with
    bias 7, 3 mantissa bits; exponent 0 is subnormal; S.1111.111 is NaN; no
    infinities).  Pinned exhaustively, all 256 codes, against torch's
    float8_e4m3fn -> float32 conversion (tests/test_quant.py); the gfx950
    kernel's v_cvt_pk_f32_fp8 decoding is then checked against this table on
    the GPU through the quantised-decode parity tests.

Pinning of quantize/dequantize: closed-form KATs (a page whose absmax is
127 * s quantises to integers exactly; round-half-even ties; clamping at the
range ends; the 1e-8 floor on all-zero pages).
"""

from __future__ import annotations

import math

import torch

FP8_DTYPE = getattr(torch, "float8_e4m3fn", None)
INT8_QMAX = 127.0
FP8_QMAX = 448.0
MIN_SCALE = 1e-8


def fp8_e4m3fn_value(code: int) -> float:
    """Real value of one OCP e4m3fn byte."""
    sign = -1.0 if code & 0x80 else 1.0
    exp = (code >> 3) & 0xF
    man = code & 0x7
    if exp == 0xF and man == 0x7:
        return math.nan
    if exp == 0:
        return sign * (man / 8.0) * 2.0 ** (1 - 7)
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


def fp8_table() -> torch.Tensor:
    """float32 values of all 256 codes (index = code)."""
    return torch.tensor([fp8_e4m3fn_value(c) for c in range(256)], dtype=torch.float32)


def quantize_pages(x: torch.Tensor, mode: str) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise ``[pages, P, Hkv, D]`` float pages; returns (q, scale [pages, Hkv])."""
    qmax = INT8_QMAX if mode == "int8" else FP8_QMAX
    xf = x.detach().cpu().float()
    scale = (xf.abs().amax(dim=(1, 3)) / qmax).clamp_min(MIN_SCALE)
    y = xf / scale[:, None, :, None]
    if mode == "int8":
        return torch.round(y).clamp(-qmax, qmax).to(torch.int8), scale
    if FP8_DTYPE is None:
        raise RuntimeError("torch has no float8_e4m3fn")
    return y.clamp(-qmax, qmax).to(FP8_DTYPE), scale


def dequantize_pages(q: torch.Tensor, scale: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """``(float(x) * scale).to(out_dtype)``; fp8 bytes decode through
    :func:`fp8_table` so the oracle does not depend on the cast it checks."""
    qc = q.detach().cpu()
    if qc.dtype == torch.int8:
        xf = qc.float()
    else:
        xf = fp8_table()[qc.view(torch.uint8).long()]
    return (xf * scale.detach().cpu().float()[:, None, :, None]).to(out_dtype)
