"""The native decode entry: the reference's ``paged_decode_cuda`` contract on
the HIP library.

Mirror of ``flashattn_tile/native.py:54-84``: ``is_available()`` and
``unavailable_reason()`` never raise, and :func:`paged_decode_attention` takes
the raw tensors (no :class:`~flashattntile_amd.paging.PagedKVCache`) with the
argument checks, error type and messages of the reference's C++ binding
(``csrc/paged_decode.cu:306-323``, ``TORCH_CHECK`` -> ``RuntimeError``), made
on the host before anything is enqueued.  What the binding accepts, this does:

* fp16, bf16 and fp32 queries with a cache of the same dtype;
* ``page_size`` 1..32, power of two or not (pages may hold more slots than
  ``page_size``; only the first ``page_size`` of each are read);
* head_dim 64 or 128;
* sequences of length <= 0 give zeros (``paged_decode.cu:135-143``) instead
  of the Python wrappers' error.

The library picks the kernel: the VALU/MFMA decode where it takes the shape,
the generic decode (fp32, pages below the fast kernels' floor or not a power
of two) otherwise.  The launch needs no device synchronisation: the split-K
partition comes from the page table's width, not from the lengths.
"""

from __future__ import annotations

import torch

from . import _hip
from .autotune import decode_partition

__all__ = ["is_available", "unavailable_reason", "paged_decode_attention"]

_NATIVE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def is_available() -> bool:
    """True when libfat_hip.so loaded and a ROCm device is visible."""
    return _hip.is_loaded() and torch.cuda.is_available()


def unavailable_reason() -> str:
    """Why the native path is unusable ('' when it is usable)."""
    if not _hip.is_loaded():
        return _hip.load_error()
    if not torch.cuda.is_available():
        return "no ROCm device detected"
    return ""


def _check(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _check_args(q, k_cache, v_cache, page_table, seq_lens, page_size: int) -> None:
    """The binding's checks (``paged_decode.cu:306-323``), in its order, plus
    the ones a raw-pointer launch needs: one device, 2-D table, 1-D lengths,
    and no page_size past the cache's page dimension."""
    _check(q.is_cuda, "q must be a CUDA tensor")
    _check(k_cache.is_cuda and v_cache.is_cuda, "KV cache must be CUDA tensors")
    _check(page_table.is_cuda and seq_lens.is_cuda, "metadata must be CUDA tensors")
    _check(q.dim() == 3, "q must be [batch, heads, head_dim]")
    _check(k_cache.dim() == 4 and v_cache.dim() == 4, "cache must be [pages, page, kv, dim]")
    _check(q.is_contiguous(), "q must be contiguous")
    _check(k_cache.is_contiguous() and v_cache.is_contiguous(), "cache must be contiguous")
    _check(page_table.dtype == torch.int32, "page_table must be int32")
    _check(seq_lens.dtype == torch.int32, "seq_lens must be int32")
    _check(q.dtype == k_cache.dtype and q.dtype == v_cache.dtype, "q and cache dtypes must match")
    _check(k_cache.shape == v_cache.shape, "k/v cache shapes must match")
    _check(q.shape[2] == k_cache.shape[3], "q head_dim must match cache head_dim")
    _check(0 < page_size <= 32, "page_size must be in [1, 32]")
    _check(page_table.dim() == 2 and seq_lens.dim() == 1, "page_table must be [batch, pages], seq_lens [batch]")
    _check(page_table.shape[0] == q.shape[0], "page_table batch must match q")
    _check(seq_lens.shape[0] == q.shape[0], "seq_lens batch must match q")
    _check(q.shape[1] % k_cache.shape[2] == 0, "heads must be divisible by KV heads")
    _check(q.dtype in _NATIVE_DTYPES, "native paged decode supports fp16, bf16 and fp32")
    _check(q.shape[2] in (64, 128), "native paged decode supports head_dim 64 or 128")
    _check(page_size <= k_cache.shape[1], f"page_size {page_size} exceeds the cache's page dimension "
                                          f"{k_cache.shape[1]}")
    dev = q.device
    _check(all(t.device == dev for t in (k_cache, v_cache, page_table, seq_lens)),
           "q, the cache and its metadata must live on one device")


def paged_decode_attention(q, k_cache, v_cache, page_table, seq_lens, page_size, softmax_scale=None):
    """Decode through the HIP library (``native.py:68-84``).

    ``q`` ``[batch, heads, head_dim]``; ``k_cache``/``v_cache``
    ``[pages, page_slots, kv_heads, head_dim]``; ``page_table`` int32
    ``[batch, max_pages]``; ``seq_lens`` int32 ``[batch]``.  Token t of
    sequence b is slot ``t % page_size`` of page ``page_table[b, t //
    page_size]``.  Returns ``[batch, heads, head_dim]`` in ``q.dtype``.
    """
    if not is_available():
        raise RuntimeError(f"native HIP path unavailable: {unavailable_reason()}")
    page_size = int(page_size)
    _check_args(q, k_cache, v_cache, page_table, seq_lens, page_size)
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    out = torch.empty_like(q)
    batch, heads = int(q.shape[0]), int(q.shape[1])
    if batch == 0 or heads == 0:
        return out
    table = page_table if page_table.stride(-1) == 1 else page_table.contiguous()
    max_pages = int(table.shape[1])
    if max_pages == 0:
        return out.zero_()  # no page can hold a token: every sequence is empty
    split, chunk = decode_partition(batch, heads, int(k_cache.shape[2]), max_pages, batch * max_pages)
    workspace = None
    if split > 1:
        need = _hip.decode_workspace_bytes(batch, heads, int(q.shape[2]), split)
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _hip.paged_decode(q, k_cache, v_cache, table, seq_lens.contiguous(), out, page_size, float(softmax_scale),
                      split, workspace=workspace, pages_per_split=chunk)
    return out
