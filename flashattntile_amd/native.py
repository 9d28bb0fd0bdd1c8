"""Availability of the native (HIP) kernel library.

Mirror of ``flashattn_tile/native.py:54-84``: ``is_available()`` and
``unavailable_reason()`` never raise; :func:`paged_decode_attention` calls the
native decode directly (no validation beyond the C ABI's own checks) and
raises ``RuntimeError`` when the library is missing.  On MI355X the native
library *is* the product path -- every op routes through it.
"""

from __future__ import annotations

import torch

from . import _hip


def is_available() -> bool:
    """True when libfat_hip.so loaded and a ROCm device is visible."""
    return _hip.is_loaded() and torch.cuda.is_available()


def unavailable_reason() -> str:
    if not _hip.is_loaded():
        return _hip.load_error()
    if not torch.cuda.is_available():
        return "no ROCm device detected"
    return ""


def paged_decode_attention(q, k_cache, v_cache, page_table, seq_lens, page_size, softmax_scale=None):
    """Decode through the HIP kernel without split-K (``native.py:68-84``)."""
    if not is_available():
        raise RuntimeError(f"native HIP path unavailable: {unavailable_reason()}")
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    q = q.contiguous()
    out = torch.empty_like(q)
    _hip.paged_decode(q, k_cache, v_cache, page_table, seq_lens, out, int(page_size), float(softmax_scale), 1)
    return out
