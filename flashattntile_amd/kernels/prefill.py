"""Varlen (packed) prefill attention on MI355X: host side of ``csrc/prefill.hip``.

Keeps the reference signature, config keys and validation
(``flashattn_tile/kernels/prefill.py:145-326``).  The HIP kernel runs QK^T
and PV on CDNA4 MFMA (v_mfma_f32_32x32x16_{f16,bf16}) with fp32
accumulation; the Triton tile knobs (BLOCK_M/BLOCK_N/num_warps/num_stages)
are validated as in the reference but the gfx950 kernels use their own fixed
tiling.  The one gfx950 knob is ``kernel``: ``"pingpong"`` (8 waves, 256 query
rows per workgroup), ``"wide"`` (8 waves of 64 query rows, 512 per workgroup;
packed prefill at head_dim 128), ``"4wave"`` (128 rows), ``"4wave_split"`` (8
waves, 128 rows, the two 4-wave groups taking alternate key tiles),
``"generic"`` (an fp32 VALU kernel, 32 query rows per workgroup) or None
(chosen from the grid size and the longest key chain).  With
``config=None`` the stored winner for the shape is used
(:func:`flashattntile_amd.autotune.best_config`, the reference's lookup at
``prefill.py:167-191``).  There is no CPU fallback: non-ROCm tensors raise.
fp32 inputs, and head_dim 16 or 512, always run on ``"generic"`` (the
reference sends fp32 to its fp32 torch path, ``prefill.py:286-290``);
forcing ``"generic"`` runs it on any shape.

``paged_prefill_attention`` is the paged (chunked) form the reference lacks:
the queries of each sequence attend to that sequence's keys in a
:class:`PagedKVCache` (its own new tokens appended first), read through the
page table by the same gfx950 kernels.
"""

from __future__ import annotations

import torch

from .. import _hip
from ..autotune import best_config, prefill_paged_signature, prefill_signature
from ..paging import PagedKVCache, _check_layout

__all__ = ["DEFAULT_CONFIG", "PAGED_CONFIG", "prefill_attention", "prefill_launch", "paged_prefill_attention",
           "paged_prefill_launch"]

DEFAULT_CONFIG = {"BLOCK_M": 64, "BLOCK_N": 64, "num_warps": 4, "num_stages": 3, "kernel": None}

_KERNEL_CODES = {None: _hip.KERNEL_AUTO, "pingpong": _hip.KERNEL_PREFILL_PINGPONG,
                 "4wave": _hip.KERNEL_PREFILL_4WAVE, "4wave_split": _hip.KERNEL_PREFILL_4WAVE_SPLIT,
                 "wide": _hip.KERNEL_PREFILL_WIDE, "generic": _hip.KERNEL_PREFILL_GENERIC}

_PREFILL_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# Paged prefill's one extra knob: how K/V rows are addressed (None = the
# fastest form the page size allows; "wide" = wave-uniform page ids with
# 64-bit row addresses; "lane" = per-lane page ids).  All give identical bits.
PAGED_CONFIG = {**DEFAULT_CONFIG, "rows": None}
_ROWS_CODES = {None: _hip.ROWS_AUTO, "wide": _hip.ROWS_WIDE, "lane": _hip.ROWS_LANE}


def _resolve_config(config: dict | None, kind: str | None = None, signature: str | None = None,
                    defaults: dict = DEFAULT_CONFIG) -> dict:
    """``prefill.py:167-191``: an explicit config, else the stored winner for
    ``kind:signature`` (when given), else the defaults."""
    resolved = dict(defaults)
    if config is None:
        stored = best_config(kind, signature) if kind and signature else None
        if stored and stored.get("kernel", None) in _KERNEL_CODES:
            resolved["kernel"] = stored.get("kernel")
    else:
        unknown = set(config) - set(defaults)
        if unknown:
            raise ValueError(f"unknown prefill config keys: {sorted(unknown)}")
        resolved.update(config)
    if resolved.get("rows") not in _ROWS_CODES:
        raise ValueError(f"rows must be None, 'wide' or 'lane', got {resolved['rows']!r}")
    if resolved["kernel"] not in _KERNEL_CODES:
        raise ValueError(f"kernel must be None, 'pingpong', 'wide', '4wave', '4wave_split' or 'generic', "
                         f"got {resolved['kernel']!r}")
    for key in ("BLOCK_M", "BLOCK_N"):
        val = resolved[key]
        if val <= 0 or val & (val - 1):
            raise ValueError(f"{key} must be a positive power of two, got {val}")
    if resolved["num_warps"] not in (1, 2, 4, 8, 16, 32):
        raise ValueError(f"num_warps must be a power of two <= 32, got {resolved['num_warps']}")
    if resolved["num_stages"] < 1:
        raise ValueError(f"num_stages must be >= 1, got {resolved['num_stages']}")
    return resolved


def _validate_inputs(q, k, v, cu_seqlens_q, cu_seqlens_k, causal) -> tuple[int, int]:
    """``prefill.py:194-233`` with the device-side checks in one sync.

    Returns the longest query and key sequence lengths."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be 3-D [tokens, heads, head_dim]")
    if k.shape != v.shape:
        raise ValueError(f"k shape {tuple(k.shape)} != v shape {tuple(v.shape)}")
    if q.shape[-1] != k.shape[-1]:
        raise ValueError(f"q head_dim {q.shape[-1]} != k head_dim {k.shape[-1]}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(f"dtype mismatch: q {q.dtype}, k {k.dtype}, v {v.dtype}")
    if not q.is_floating_point():
        raise ValueError(f"expected floating point inputs, got {q.dtype}")
    if q.device != k.device or k.device != v.device:
        raise ValueError("q, k, v must live on the same device")
    if cu_seqlens_q.dim() != 1 or cu_seqlens_k.dim() != 1:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must be 1-D")
    if cu_seqlens_q.shape[0] != cu_seqlens_k.shape[0]:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have the same batch dimension")
    if cu_seqlens_q.numel() < 2:
        raise ValueError("cu_seqlens must contain at least batch + 1 entries")
    if cu_seqlens_q.dtype != torch.int32 or cu_seqlens_k.dtype != torch.int32:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must be int32")
    if cu_seqlens_q.device != q.device or cu_seqlens_k.device != q.device:
        raise ValueError("cu_seqlens must live on the same device as q")
    cq = cu_seqlens_q.to(torch.int64)
    ck = cu_seqlens_k.to(torch.int64)
    lq = cq[1:] - cq[:-1]
    lk = ck[1:] - ck[:-1]
    keyless = (lk == 0) & (lq > 0)
    first_keyless = keyless.to(torch.int64).argmax()
    stats = torch.stack([
        cq[0], ck[0], cq[-1], ck[-1],
        (lq < 0).any().to(torch.int64), (lk < 0).any().to(torch.int64),
        (lk < lq).any().to(torch.int64), lq.max(), lk.max(),
        keyless.any().to(torch.int64), first_keyless, lq[first_keyless],
    ]).cpu().tolist()
    q0, k0, q_end, k_end, q_dec, k_dec, short_kv, max_q, max_k, any_keyless, kl_b, kl_q = (int(x) for x in stats)
    if q0 != 0 or k0 != 0:
        raise ValueError("cu_seqlens must start at 0")
    if q_end != q.shape[0]:
        raise ValueError("cu_seqlens_q[-1] must equal q.shape[0]")
    if k_end != k.shape[0]:
        raise ValueError("cu_seqlens_k[-1] must equal k.shape[0]")
    if q_dec:
        raise ValueError("cu_seqlens_q must be non-decreasing")
    if k_dec:
        raise ValueError("cu_seqlens_k must be non-decreasing")
    if causal and short_kv:
        raise ValueError("causal bottom-right alignment requires kv_len >= q_len per sequence")
    if any_keyless:  # reference.py:115-116 (the kernels would write zeros)
        raise ValueError(f"sequence {kl_b} has {kl_q} queries but no keys")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError(f"num_heads ({q.shape[1]}) must be divisible by num_kv_heads ({k.shape[1]})")
    return max_q, max_k


def prefill_launch(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    causal: bool,
    softmax_scale: float,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    kernel: str | None = None,
) -> torch.Tensor:
    """Enqueue the HIP prefill without validation or synchronisation.

    ``q``/``k``/``v`` must have a contiguous head_dim axis; ``max_seqlen_*``
    must bound every sequence (they size the launch grid).  ``kernel``:
    None (library's choice), ``"pingpong"``, ``"wide"``, ``"4wave"``, ``"4wave_split"`` or ``"generic"``.
    """
    if q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("q, k, v need a contiguous head_dim axis")
    if out is None:
        out = torch.empty_like(q)
    # The kernels read cu_seqlens densely.
    cu_seqlens_q = cu_seqlens_q if cu_seqlens_q.is_contiguous() else cu_seqlens_q.contiguous()
    cu_seqlens_k = cu_seqlens_k if cu_seqlens_k.is_contiguous() else cu_seqlens_k.contiguous()
    a = _hip.prefill_args(q, k, v, cu_seqlens_q, cu_seqlens_k, out, max_seqlen_q, max_seqlen_k, causal,
                          softmax_scale, workspace=None, kernel=_KERNEL_CODES[kernel])
    # Long bf16 launches on the large-grid kernel stage an fp16 copy of V from
    # a workspace; the library says how much this launch uses (0 for fp16 and
    # every other launch), so nothing is allocated that it would not use.
    need = _hip.prefill_varlen_workspace_bytes(a)
    if need:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        a.workspace = workspace.data_ptr()
    _hip.prefill_varlen_with_args(a, _hip.current_stream_handle(q.device))
    return out


def prefill_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    causal: bool = True,
    softmax_scale: float | None = None,
    config: dict | None = None,
) -> torch.Tensor:
    """Fused varlen prefill attention (``prefill.py:236-326``).

    ``q``: ``[total_q, num_heads, head_dim]``; ``k``/``v``:
    ``[total_k, num_kv_heads, head_dim]``; ``cu_seqlens_*`` int32 ``[B + 1]``
    on the same ROCm device; causal masking is bottom-right aligned.  Returns
    ``[total_q, num_heads, head_dim]`` in ``q.dtype``.
    """
    longest_q, longest_k = _validate_inputs(q, k, v, cu_seqlens_q, cu_seqlens_k, causal)
    scale = float(softmax_scale) if softmax_scale is not None else q.shape[-1] ** -0.5
    if max_seqlen_q <= 0:
        raise ValueError(f"max_seqlen_q must be positive, got {max_seqlen_q}")
    if max_seqlen_k <= 0:
        raise ValueError(f"max_seqlen_k must be positive, got {max_seqlen_k}")
    # The grid is sized from max_seqlen_q; a smaller bound would leave rows
    # uncomputed, so it is checked against cu_seqlens (no extra sync).
    if max_seqlen_q < longest_q:
        raise ValueError(f"max_seqlen_q {max_seqlen_q} is smaller than the longest query sequence {longest_q}")
    if max_seqlen_k < longest_k:
        raise ValueError(f"max_seqlen_k {max_seqlen_k} is smaller than the longest key sequence {longest_k}")
    sig = prefill_signature(cu_seqlens_q.shape[0] - 1, q.shape[1], k.shape[1], q.shape[2], int(max_seqlen_q),
                            int(max_seqlen_k), causal)
    cfg = _resolve_config(config, "prefill", sig)
    if not all(t.is_cuda for t in (q, k, v, cu_seqlens_q, cu_seqlens_k)):
        raise RuntimeError("prefill_attention: inputs must be ROCm device tensors; this build runs the gfx950 "
                           "HIP kernel only (no CPU or reference fallback)")
    if q.dtype not in _PREFILL_DTYPES:
        raise ValueError(f"prefill_attention: dtype {q.dtype} is not fp16/bf16/fp32 (the HIP kernels' types)")
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    return prefill_launch(q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), int(max_seqlen_k),
                          bool(causal), scale, kernel=cfg["kernel"])


def _validate_paged(q, cache: PagedKVCache, cu_seqlens_q, causal) -> int:
    """Shape/dtype checks plus the device-side ones (cu_seqlens_q monotone
    and ending at q.shape[0]; lengths within the table; used pages inside the
    pool; kv_len >= q_len when causal) in one synchronisation.  The messages
    are those of ``prefill.py:194-233`` and ``paging.py:84-130``.  Returns the
    longest query sequence."""
    if not isinstance(cache, PagedKVCache):
        raise TypeError("cache must be a PagedKVCache")
    _check_layout(cache)
    if q.dim() != 3:
        raise ValueError("q must be 3-D [tokens, heads, head_dim]")
    if q.shape[-1] != cache.head_dim:
        raise ValueError(f"q head_dim {q.shape[-1]} != cache head_dim {cache.head_dim}")
    if q.dtype != cache.k_cache.dtype:
        raise ValueError(f"q dtype {q.dtype} != cache dtype {cache.k_cache.dtype}")
    if q.shape[1] % cache.num_kv_heads != 0:
        raise ValueError(f"num_heads ({q.shape[1]}) must be divisible by num_kv_heads ({cache.num_kv_heads})")
    if cu_seqlens_q.dim() != 1 or cu_seqlens_q.dtype != torch.int32:
        raise ValueError("cu_seqlens_q must be a 1-D int32 tensor")
    if cu_seqlens_q.shape[0] != cache.batch_size + 1:
        raise ValueError(f"cu_seqlens_q must have batch + 1 = {cache.batch_size + 1} entries, "
                         f"got {cu_seqlens_q.shape[0]}")
    dev = q.device
    if any(t.device != dev for t in (cache.k_cache, cache.page_table, cache.seq_lens, cu_seqlens_q)):
        raise ValueError("q, the cache, its page table, seq_lens and cu_seqlens_q must live on one device")
    cq = cu_seqlens_q.to(torch.int64)
    lq = cq[1:] - cq[:-1]
    sl = cache.seq_lens.to(torch.int64)
    P = cache.page_size
    need = torch.div(sl.max() + (P - 1), P, rounding_mode="floor")
    pt = cache.page_table
    used = (torch.arange(pt.shape[1], device=dev) < need).unsqueeze(0).expand_as(pt)
    big, small = torch.iinfo(torch.int32).max, torch.iinfo(torch.int32).min
    lo = torch.where(used, pt, torch.full_like(pt, big)).min().to(torch.int64) if pt.numel() else sl.max() * 0
    hi = torch.where(used, pt, torch.full_like(pt, small)).max().to(torch.int64) if pt.numel() else sl.max() * 0
    keyless = (sl <= 0) & (lq > 0)
    first_keyless = keyless.to(torch.int64).argmax()
    stats = torch.stack([
        cq[0], cq[-1], (lq < 0).any().to(torch.int64), lq.max(), (sl < lq).any().to(torch.int64),
        sl.min(), sl.max(), lo, hi, keyless.any().to(torch.int64), first_keyless, lq[first_keyless],
    ]).cpu().tolist()
    q0, q_end, q_dec, max_q, short_kv, min_len, max_len, lo, hi, any_keyless, kl_b, kl_q = (int(x) for x in stats)
    if q0 != 0:
        raise ValueError("cu_seqlens must start at 0")
    if q_end != q.shape[0]:
        raise ValueError("cu_seqlens_q[-1] must equal q.shape[0]")
    if q_dec:
        raise ValueError("cu_seqlens_q must be non-decreasing")
    if min_len < 0:
        raise AssertionError("seq_lens must be non-negative")
    if max_len > cache.capacity:
        raise AssertionError(f"seq_len {max_len} exceeds page-table capacity {cache.capacity}")
    if max_len > 0 and lo != big:
        if lo < 0:
            raise AssertionError("page_table contains a negative page id")
        if hi >= cache.num_pages:
            raise AssertionError(f"page_table references page {hi} but cache has {cache.num_pages} pages")
    if causal and short_kv:
        raise ValueError("causal bottom-right alignment requires kv_len >= q_len per sequence")
    if any_keyless:  # reference.py:115-116, as for packed prefill
        raise ValueError(f"sequence {kl_b} has {kl_q} queries but no keys")
    return max_q


def paged_prefill_launch(q: torch.Tensor, cache: PagedKVCache, cu_seqlens_q: torch.Tensor, max_seqlen_q: int,
                         causal: bool, softmax_scale: float, out: torch.Tensor | None = None,
                         kernel: str | None = None, rows: str | None = None,
                         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Enqueue ``fat_prefill_paged`` without validation or synchronisation
    (``kernel`` as for :func:`prefill_launch`; ``rows``: None, ``"wide"`` or
    ``"lane"``, the row addressing of ``PAGED_CONFIG``).  ``workspace``: a
    uint8 device buffer of at least ``fat_prefill_paged_workspace_bytes`` of
    the launch (long chunks copy their K/V rows there for the wide kernel);
    None or too small allocates one, so a caller that must not allocate
    (graph capture) passes its own."""
    if q.stride(-1) != 1 or cache.k_cache.stride(-1) != 1 or cache.v_cache.stride(-1) != 1:
        raise ValueError("q and the cache need a contiguous head_dim axis")
    if out is None:
        out = torch.empty_like(q)
    pt = cache.page_table if cache.page_table.stride(-1) == 1 else cache.page_table.contiguous()
    sl = cache.seq_lens if cache.seq_lens.is_contiguous() else cache.seq_lens.contiguous()
    cu = cu_seqlens_q if cu_seqlens_q.is_contiguous() else cu_seqlens_q.contiguous()
    a = _hip.prefill_paged_args(q, cache.k_cache, cache.v_cache, pt, sl, cu, out, cache.page_size,
                                int(max_seqlen_q), bool(causal), float(softmax_scale),
                                kernel=_KERNEL_CODES[kernel], rows=_ROWS_CODES[rows])
    # Long chunks run on the packed wide kernel through copies of their K/V
    # rows: allocate the workspace the library asks for (0 for the others).
    need = _hip.prefill_paged_workspace_bytes(a)
    if need:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        a.workspace = workspace.data_ptr()
    _hip.prefill_paged_with_args(a, _hip.current_stream_handle(q.device))
    return out


def paged_prefill_attention(
    q: torch.Tensor,
    cache: PagedKVCache,
    cu_seqlens_q: torch.Tensor,
    max_seqlen_q: int,
    causal: bool = True,
    softmax_scale: float | None = None,
    config: dict | None = None,
) -> torch.Tensor:
    """Paged (chunked) prefill: ``q`` ``[total_q, num_heads, head_dim]`` packed
    by ``cu_seqlens_q`` (int32 ``[B + 1]``) attends, per sequence b, to keys
    ``0 .. seq_lens[b] - 1`` of ``cache`` (which already holds the chunk's
    own K/V).  Causal masking is bottom-right aligned, as in
    :func:`prefill_attention`, so query i of a q_len-token chunk sees keys
    ``j <= i + seq_lens[b] - q_len``.  ``config`` as for
    :func:`prefill_attention` plus ``rows`` (store kind ``prefill_paged``).
    Returns ``q``'s shape and dtype.
    """
    longest_q = _validate_paged(q, cache, cu_seqlens_q, causal)
    if max_seqlen_q <= 0:
        raise ValueError(f"max_seqlen_q must be positive, got {max_seqlen_q}")
    if max_seqlen_q < longest_q:
        raise ValueError(f"max_seqlen_q {max_seqlen_q} is smaller than the longest query sequence {longest_q}")
    if not q.is_cuda:
        raise RuntimeError("paged_prefill_attention: inputs must be ROCm device tensors; this build runs the "
                           "gfx950 HIP kernel only (no CPU or reference fallback)")
    if q.dtype not in _PREFILL_DTYPES:
        raise ValueError(f"paged_prefill_attention: dtype {q.dtype} is not fp16/bf16/fp32 (the HIP kernels' types)")
    sig = prefill_paged_signature(cache.batch_size, q.shape[1], cache.num_kv_heads, cache.head_dim,
                                  cache.page_size, int(max_seqlen_q), causal)
    cfg = _resolve_config(config, "prefill_paged", sig, defaults=PAGED_CONFIG)
    scale = float(softmax_scale) if softmax_scale is not None else q.shape[-1] ** -0.5
    q = q if q.stride(-1) == 1 else q.contiguous()
    return paged_prefill_launch(q, cache, cu_seqlens_q, int(max_seqlen_q), bool(causal), scale,
                                kernel=cfg["kernel"], rows=cfg["rows"])
