"""Paged decode on MI355X: host side of the HIP kernels in ``csrc/decode.hip``.

Public functions keep the reference signatures and validation
(``flashattn_tile/kernels/decode.py:474-704``):

* :func:`paged_decode_attention` (fp16/bf16 cache, ``decode.py:533``);
* :func:`paged_decode_attention_fp8` (int8 / float8_e4m3fn cache with
  per-(page, KV-head) scales, ``decode.py:645``);

plus :func:`paged_decode_attention_multi`, the multi-token (speculative)
decode the reference lacks (its decode takes one query per sequence,
``decode.py:548-553``).

Differences, all deliberate:

* there is no CPU or Triton fallback: non-ROCm tensors, or a dtype the HIP
  kernels do not take, raise instead of silently running the fp32 reference
  (the oracle lives outside the product, under ``oracle/``);
* the quantised path supports split-K as well;
* ``config=None`` takes the launch stored for this shape in the gfx950
  tuned-config store (:func:`flashattntile_amd.autotune.best_config`, keyed by
  :func:`~flashattntile_amd.autotune.decode_signature`) and otherwise the
  MI355X partition heuristic (:func:`~flashattntile_amd.autotune.decode_partition`);
  an explicit ``split_k`` is honoured exactly;
* validation costs one device->host synchronisation instead of ~6.

:func:`paged_decode_launch` is the sync-free entry below the validation, for
callers (benchmarks, CUDA-graph-style capture loops) that validated once.
"""

from __future__ import annotations

import warnings

import torch

from .. import _hip
from ..autotune import best_config, decode_partition, decode_signature, is_ragged
from ..paging import PagedKVCache, _check_layout, cache_stats

__all__ = [
    "DEFAULT_CONFIG",
    "paged_decode_attention",
    "paged_decode_attention_fp8",
    "paged_decode_attention_multi",
    "paged_decode_launch",
    "resolve_decode_config",
    "DecodeLaunch",
]

# split_k None -> MI355X partition heuristic (split_k and pages_per_split from
# the batch's lengths); an explicit split_k keeps the reference's partitioning
# (ceil(pages / split_k) per sequence) unless pages_per_split is also given.
# num_warps is the number of 64-lane waves per workgroup (4 or 8; None lets the
# library choose from the grid size); num_stages is accepted for signature
# compatibility with the reference's Triton knob and validated the same way,
# but the HIP kernel's pipeline depth is fixed (one 16-token unit prefetched
# per wave).  kernel None lets the library choose the kernel family; "valu",
# "mfma" or "generic" forces one (what a tuning run stores for its shape; the
# generic kernel is the library's own choice only for the shapes the other
# two do not take: fp32, page sizes below their floor or not a power of two,
# head_dim 32 or 256).
DEFAULT_CONFIG = {"split_k": None, "num_warps": None, "num_stages": 2, "pages_per_split": None, "kernel": None}

_KERNEL_CODES = {None: _hip.KERNEL_AUTO, "valu": _hip.KERNEL_DECODE_VALU, "mfma": _hip.KERNEL_DECODE_MFMA,
                 "generic": _hip.KERNEL_DECODE_GENERIC}

# Element types the HIP decode kernels take for q (and for a cache of the same
# type); int8 / float8_e4m3fn caches take fp16 / bf16 queries.
_DECODE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

_QUANT_DTYPES = tuple(d for d in (torch.int8, getattr(torch, "float8_e4m3fn", None)) if d is not None)


def _resolve_config(config: dict | None, q: torch.Tensor, cache: PagedKVCache, max_len: int,
                    total_pages: int, q_len: int = 1) -> dict:
    """``decode.py:474-500``: an explicit config, else the stored winner for
    this shape, else the heuristic.  A stored entry the checks below reject
    is ignored with a warning.  Needs no device synchronisation."""
    if config is None:
        sig = decode_signature(int(q.shape[0]), int(q.shape[-2]), cache.num_kv_heads, cache.head_dim,
                               cache.page_size, max_len, total_pages, cache.k_cache.dtype, q_len)
        stored = best_config("decode", sig)
        if stored:
            try:
                return _merge_config({k: v for k, v in stored.items() if k in DEFAULT_CONFIG}, q, cache, max_len,
                                     total_pages, q_len)
            except ValueError as exc:
                warnings.warn(f"ignoring the stored decode config for {sig}: {exc}", RuntimeWarning, stacklevel=3)
        return _merge_config({}, q, cache, max_len, total_pages, q_len)
    unknown = set(config) - set(DEFAULT_CONFIG)
    if unknown:
        raise ValueError(f"unknown decode config keys: {sorted(unknown)}")
    return _merge_config(config, q, cache, max_len, total_pages, q_len)


def resolve_decode_config(q: torch.Tensor, cache: PagedKVCache, max_len: int, total_pages: int,
                          config: dict | None = None, q_len: int = 1) -> dict:
    """The launch the decode wrappers make for these inputs: ``config`` if
    given, else the stored winner for the shape, else the heuristic.  Host
    work only; ``max_len`` and ``total_pages`` are the batch's longest
    sequence and its page count.  For callers of :func:`paged_decode_launch`
    (benchmarks, capture loops) that validated once."""
    return _resolve_config(config, q, cache, max_len, total_pages, q_len)


def _merge_config(config: dict, q: torch.Tensor, cache: PagedKVCache, max_len: int, total_pages: int,
                  q_len: int) -> dict:
    resolved = dict(DEFAULT_CONFIG)
    resolved.update(config)
    if resolved["split_k"] is None:
        max_pages = -(-max_len // cache.page_size)
        split, chunk = decode_partition(int(q.shape[0]), int(q.shape[-2]), cache.num_kv_heads, max_pages,
                                        total_pages, quantized=cache.k_cache.dtype in _QUANT_DTYPES, q_len=q_len)
        resolved["split_k"] = split
        if resolved["pages_per_split"] is None:
            resolved["pages_per_split"] = chunk
        # A skewed batch runs 4-wave workgroups: the library's own choice (8
        # waves for partitions of >= 1024 keys, measured on uniform batches)
        # was 1.04-1.4x slower on the skewed batches of decode_partition.
        if resolved["num_warps"] is None and is_ragged(int(q.shape[0]), max_pages, total_pages):
            resolved["num_warps"] = 4
    if resolved["pages_per_split"] is None:
        resolved["pages_per_split"] = 0
    split_k = resolved["split_k"]
    if not isinstance(split_k, int) or isinstance(split_k, bool) or split_k < 1:
        raise ValueError(f"split_k must be a positive integer, got {split_k}")
    if split_k > 64:
        raise ValueError(f"split_k must be <= 64, got {split_k}")
    pps = resolved["pages_per_split"]
    if not isinstance(pps, int) or isinstance(pps, bool) or pps < 0:
        raise ValueError(f"pages_per_split must be a non-negative integer, got {pps}")
    if resolved["num_warps"] not in (None, 1, 2, 4, 8, 16, 32):
        raise ValueError(f"num_warps must be a power of two <= 32, got {resolved['num_warps']}")
    if resolved["num_warps"] not in (None, 4, 8):
        raise ValueError(f"num_warps must be 4 or 8 waves per workgroup on MI355X, got {resolved['num_warps']}")
    if resolved["num_stages"] < 1:
        raise ValueError(f"num_stages must be >= 1, got {resolved['num_stages']}")
    if resolved["kernel"] not in _KERNEL_CODES:
        raise ValueError(f"kernel must be None, 'valu', 'mfma' or 'generic', got {resolved['kernel']!r}")
    if resolved["kernel"] in ("valu", "generic") and q_len > 1:
        raise ValueError(f"kernel {resolved['kernel']!r} takes one query per sequence; multi-token decode runs "
                         "on 'mfma'")
    if (resolved["kernel"] == "valu" and cache.k_cache.dtype in _QUANT_DTYPES
            and q.shape[-2] // cache.num_kv_heads >= 8):
        raise ValueError("kernel 'valu' takes int8/float8 caches only for GQA groups below 8; use 'mfma'")
    return resolved


def _validate_decode_inputs(q: torch.Tensor, cache: PagedKVCache, multi: bool = False) -> tuple[int, int]:
    """``decode.py:503-522`` + ``paging.validate_cache``, with one sync.

    ``multi``: ``q`` is ``[batch, q_len, heads, head_dim]`` and every sequence
    must already hold its q_len new tokens.  Returns ``(max_len,
    total_pages)`` for the partition heuristic."""
    if not isinstance(cache, PagedKVCache):
        raise TypeError("cache must be a PagedKVCache")
    _check_layout(cache)
    if multi:
        if q.dim() != 4:
            raise ValueError(f"q must be [batch, q_len, heads, head_dim], got {tuple(q.shape)}")
    elif q.dim() != 3:
        raise ValueError(f"q must be [batch, heads, head_dim], got {tuple(q.shape)}")
    if q.shape[0] != cache.batch_size:
        raise ValueError(f"q batch {q.shape[0]} != cache batch {cache.batch_size}")
    if q.shape[-1] != cache.head_dim:
        raise ValueError(f"q head_dim {q.shape[-1]} != cache head_dim {cache.head_dim}")
    if q.shape[-2] % cache.num_kv_heads != 0:
        raise ValueError(f"num_heads {q.shape[-2]} must be divisible by num_kv_heads {cache.num_kv_heads}")
    if q.device != cache.k_cache.device:
        raise ValueError("q and cache must live on the same device")
    if not q.is_floating_point():
        raise ValueError(f"q must be floating point, got {q.dtype}")
    min_len, max_len, lo, hi, total_pages = cache_stats(cache, with_total_pages=True)
    if min_len < 0:
        raise AssertionError("seq_lens must be non-negative")
    capacity = cache.capacity
    if max_len > capacity:
        raise AssertionError(f"seq_len {max_len} exceeds page-table capacity {capacity}")
    if max_len > 0:
        if lo < 0:
            raise AssertionError("page_table contains a negative page id")
        if hi >= cache.num_pages:
            raise AssertionError(f"page_table references page {hi} but cache has {cache.num_pages} pages")
    if min_len <= 0:
        raise ValueError("decode requires every sequence to hold at least one cached token")
    if multi and min_len < q.shape[1]:
        raise ValueError(f"multi-token decode requires every sequence to hold its {q.shape[1]} new tokens "
                         f"(shortest seq_len {min_len})")
    return max_len, total_pages


def _require_rocm(q: torch.Tensor, cache: PagedKVCache, what: str) -> None:
    tensors = (q, cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens)
    if not all(t.is_cuda for t in tensors):
        raise RuntimeError(
            f"{what}: inputs must be ROCm device tensors; this build runs the gfx950 HIP kernel only "
            "(no CPU or reference fallback)"
        )


# Split-K merge counters of the one-call decode paths: one zeroed int32
# buffer per (device, stream), grown on demand.  Every launch leaves its
# counters zero, so launches in one stream's order share them; launches on
# other streams get their own.
_MERGE_COUNTERS: dict[tuple[int, int], torch.Tensor] = {}


def merge_counters(q: torch.Tensor, split_k: int) -> torch.Tensor | None:
    """Zeroed merge counters for a split-K launch of ``q`` on torch's current
    stream (None when ``split_k`` is 1): the decode kernels then merge the
    partitions themselves instead of a second kernel."""
    if split_k <= 1:
        return None
    rows = q.shape[0] * (q.shape[1] if q.dim() == 4 else 1)
    n = rows * q.shape[-2]  # fat_paged_decode_counters_bytes / 4: one int32 per (query row, head)
    key = (q.device.index if q.device.index is not None else torch.cuda.current_device(),
           _hip.current_stream_handle(q.device))
    t = _MERGE_COUNTERS.get(key)
    if t is None or t.numel() < n:
        t = torch.zeros(max(n, 4096), dtype=torch.int32, device=q.device)
        _MERGE_COUNTERS[key] = t
    return t


def paged_decode_launch(
    q: torch.Tensor,
    cache: PagedKVCache,
    softmax_scale: float,
    split_k: int,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    scales=None,
    waves_per_group: int | None = None,
    pages_per_split: int = 0,
    kernel: str | None = None,
    counters: torch.Tensor | None = None,
) -> torch.Tensor:
    """Enqueue the HIP decode without validation or synchronisation.

    ``q`` (``[B, H, D]``, or ``[B, T, H, D]`` for multi-token decode) must be
    contiguous fp16/bf16 on the cache's device; ``out`` (default
    ``empty_like(q)``) and ``workspace`` (default: allocated) may be passed in
    to avoid allocations.  ``kernel``: None (library's choice), ``"valu"`` or
    ``"mfma"``.  ``counters``: zeroed int32 split-K merge counters
    (:func:`merge_counters`, or any buffer of ``decode_counters_bytes`` that
    only this stream's launches use); the decode launch then merges its
    partitions itself.  None: a second kernel merges.
    """
    if cache.k_cache.stride(-1) != 1 or cache.v_cache.stride(-1) != 1:
        raise ValueError("k_cache and v_cache need a contiguous head_dim axis")
    if out is None:
        out = torch.empty_like(q)
    # The kernels read page_table rows with a unit column stride and seq_lens
    # densely (the reference honours any strides, kernels/decode.py:89).
    pt = cache.page_table if cache.page_table.stride(-1) == 1 else cache.page_table.contiguous()
    sl = cache.seq_lens if cache.seq_lens.is_contiguous() else cache.seq_lens.contiguous()
    rows = q.shape[0] * (q.shape[1] if q.dim() == 4 else 1)
    need = _hip.decode_workspace_bytes(rows, q.shape[-2], q.shape[-1], split_k)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    k_scale = v_scale = None
    if scales is not None:
        k_scale = scales["k"] if isinstance(scales, dict) else scales.k
        v_scale = scales["v"] if isinstance(scales, dict) else scales.v
    # fat_paged_decode_counters_bytes: one int32 per (query row, head)
    if counters is not None and counters.numel() * counters.element_size() < 4 * rows * q.shape[-2]:
        raise ValueError("paged_decode_launch: counters smaller than decode_counters_bytes(rows, num_heads)")
    _hip.paged_decode(q, cache.k_cache, cache.v_cache, pt, sl, out,
                      cache.page_size, softmax_scale, split_k, workspace=workspace,
                      k_scale=k_scale, v_scale=v_scale, waves_per_group=waves_per_group or 0,
                      pages_per_split=pages_per_split, kernel=_KERNEL_CODES[kernel], counters=counters)
    return out


def paged_decode_attention(
    q: torch.Tensor,
    cache: PagedKVCache,
    softmax_scale: float | None = None,
    config: dict | None = None,
    grouped: bool = False,
) -> torch.Tensor:
    """Paged decode attention, one query per sequence (``decode.py:533-642``).

    ``q``: ``[batch, num_heads, head_dim]`` fp16/bf16/fp32 on a ROCm device;
    the cache holds the same dtype (fp32 runs on the HIP kernel too, where the
    reference falls back to its fp32 oracle, ``decode.py:569-576``).  ``softmax_scale`` defaults to
    ``head_dim ** -0.5``.  ``config``: ``split_k`` (1 = no split; default from
    the MI355X heuristic), ``num_warps``, ``num_stages``.  ``grouped`` is
    accepted for compatibility: the HIP kernel always reads each K/V page
    once per GQA group.  Returns ``[batch, num_heads, head_dim]`` in
    ``q.dtype``.
    """
    del grouped  # every launch is grouped on MI355X
    max_len, total_pages = _validate_decode_inputs(q, cache)
    scale = float(softmax_scale) if softmax_scale is not None else q.shape[-1] ** -0.5
    cfg = _resolve_config(config, q, cache, max_len, total_pages)
    _require_rocm(q, cache, "paged_decode_attention")
    if q.dtype not in _DECODE_DTYPES:
        raise ValueError(f"paged_decode_attention: dtype {q.dtype} is not fp16/bf16/fp32 (the HIP kernels' types)")
    if cache.k_cache.dtype != q.dtype:
        raise ValueError(f"q dtype {q.dtype} must match cache dtype {cache.k_cache.dtype}")
    q = q.contiguous()
    return paged_decode_launch(q, cache, scale, cfg["split_k"], waves_per_group=cfg["num_warps"],
                               pages_per_split=cfg["pages_per_split"], kernel=cfg["kernel"],
                               counters=merge_counters(q, cfg["split_k"]))


def paged_decode_attention_fp8(
    q: torch.Tensor,
    cache: PagedKVCache,
    scales,
    softmax_scale: float | None = None,
    config: dict | None = None,
) -> torch.Tensor:
    """Decode against an int8 / float8_e4m3fn cache (``decode.py:645-704``).

    ``scales`` is a :class:`~flashattntile_amd.quant.QuantScales` (or a dict
    with ``"k"``/``"v"``), fp32 ``[num_pages, num_kv_heads]``.  Pages are
    dequantised in registers as ``(float(x) * scale).to(q.dtype)``.
    """
    max_len, total_pages = _validate_decode_inputs(q, cache)
    k_scale = scales["k"] if isinstance(scales, dict) else scales.k
    v_scale = scales["v"] if isinstance(scales, dict) else scales.v
    quant_dtype = cache.k_cache.dtype
    if quant_dtype not in _QUANT_DTYPES:
        raise ValueError(f"expected int8/float8 cache, got {quant_dtype}")
    expected = (cache.num_pages, cache.num_kv_heads)
    if tuple(k_scale.shape) != expected or tuple(v_scale.shape) != expected:
        raise ValueError(f"scales must have shape {expected}, got {tuple(k_scale.shape)}")
    scale = float(softmax_scale) if softmax_scale is not None else q.shape[-1] ** -0.5
    cfg = _resolve_config(config, q, cache, max_len, total_pages)
    _require_rocm(q, cache, "paged_decode_attention_fp8")
    if not (k_scale.is_cuda and v_scale.is_cuda):
        raise RuntimeError("paged_decode_attention_fp8: scales must be ROCm device tensors")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"quantised decode requires fp16/bf16 queries, got {q.dtype}")
    if k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
        raise ValueError("scales must be float32")
    q = q.contiguous()
    return paged_decode_launch(q, cache, scale, cfg["split_k"],
                               scales={"k": k_scale.contiguous(), "v": v_scale.contiguous()},
                               waves_per_group=cfg["num_warps"], pages_per_split=cfg["pages_per_split"],
                               kernel=cfg["kernel"], counters=merge_counters(q, cfg["split_k"]))


def paged_decode_attention_multi(
    q: torch.Tensor,
    cache: PagedKVCache,
    softmax_scale: float | None = None,
    config: dict | None = None,
    scales=None,
) -> torch.Tensor:
    """Multi-token (speculative) decode: ``q`` ``[batch, q_len, num_heads,
    head_dim]`` holds the last q_len tokens of each sequence, whose K/V are
    already in ``cache`` (``seq_lens[b] >= q_len``).  Token t of sequence b
    attends keys ``j <= seq_lens[b] - q_len + t`` -- the bottom-right causal
    convention of :func:`~flashattntile_amd.kernels.prefill.prefill_attention`
    -- and every K/V page is read once per KV head (per 32 (head, token)
    rows) by the MFMA decode kernel.  ``scales`` (QuantScales or
    ``{"k", "v"}``) selects an int8/float8_e4m3fn cache.  ``config`` as for
    :func:`paged_decode_attention`.  Returns ``q``'s shape and dtype.
    """
    max_len, total_pages = _validate_decode_inputs(q, cache, multi=True)
    q_len = int(q.shape[1])
    if q_len > 64:
        raise ValueError(f"multi-token decode takes at most 64 tokens per sequence, got {q_len}")
    quantized = cache.k_cache.dtype in _QUANT_DTYPES
    if quantized != (scales is not None):
        raise ValueError("an int8/float8 cache needs scales, and only such a cache takes them")
    scale = float(softmax_scale) if softmax_scale is not None else q.shape[-1] ** -0.5
    cfg = _resolve_config(config, q, cache, max_len, total_pages, q_len=q_len)
    _require_rocm(q, cache, "paged_decode_attention_multi")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"paged_decode_attention_multi: dtype {q.dtype} is not fp16/bf16")
    sc = None
    if quantized:
        k_scale = scales["k"] if isinstance(scales, dict) else scales.k
        v_scale = scales["v"] if isinstance(scales, dict) else scales.v
        expected = (cache.num_pages, cache.num_kv_heads)
        if tuple(k_scale.shape) != expected or tuple(v_scale.shape) != expected:
            raise ValueError(f"scales must have shape {expected}, got {tuple(k_scale.shape)}")
        if k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
            raise ValueError("scales must be float32")
        sc = {"k": k_scale.contiguous(), "v": v_scale.contiguous()}
    elif cache.k_cache.dtype != q.dtype:
        raise ValueError(f"q dtype {q.dtype} must match cache dtype {cache.k_cache.dtype}")
    q = q.contiguous()
    return paged_decode_launch(q, cache, scale, cfg["split_k"], scales=sc,
                               waves_per_group=cfg["num_warps"], pages_per_split=cfg["pages_per_split"],
                               kernel=cfg["kernel"], counters=merge_counters(q, cfg["split_k"]))


class DecodeLaunch:
    """A decode launch prepared once and run every step (plan / run).

    Construction validates ``q`` and ``cache`` (one synchronisation, as
    :func:`paged_decode_attention` does, unless ``max_len`` and
    ``total_pages`` are given), resolves the launch (``config``, else the
    tuned store, else the heuristic), allocates the split-K workspace and
    fills the ``fat_decode_args`` block.  :meth:`run` then only writes the
    query and output addresses into that block and enqueues
    ``fat_paged_decode``: no validation, synchronisation or allocation, about
    the cost of one ctypes call.  The page table and seq_lens are read on the
    device at every run, so the serving engine updates them in place.  ``q``
    and ``out`` passed to :meth:`run` must have the dtype, shape and strides
    of the ``q`` given here (``out``: contiguous).  ``q`` is ``[B, H, D]`` or
    ``[B, T, H, D]`` (multi-token decode); ``scales`` selects an int8 /
    float8_e4m3fn cache.
    """

    def __init__(self, q: torch.Tensor, cache: PagedKVCache, softmax_scale: float | None = None,
                 config: dict | None = None, scales=None, max_len: int | None = None,
                 total_pages: int | None = None) -> None:
        multi = q.dim() == 4
        if max_len is None or total_pages is None:
            max_len, total_pages = _validate_decode_inputs(q, cache, multi=multi)
        q_len = int(q.shape[1]) if multi else 1
        cfg = _resolve_config(config, q, cache, max_len, total_pages, q_len=q_len)
        _require_rocm(q, cache, "DecodeLaunch")
        quantized = cache.k_cache.dtype in _QUANT_DTYPES
        if q.dtype not in (_DECODE_DTYPES[:2] if quantized else _DECODE_DTYPES):
            raise ValueError(f"DecodeLaunch: q dtype {q.dtype} is not one the HIP decode takes for a "
                             f"{cache.k_cache.dtype} cache")
        if quantized != (scales is not None):
            raise ValueError("an int8/float8 cache needs scales, and only such a cache takes them")
        if not quantized and cache.k_cache.dtype != q.dtype:
            raise ValueError(f"q dtype {q.dtype} must match cache dtype {cache.k_cache.dtype}")
        if not q.is_contiguous():
            raise ValueError("DecodeLaunch: q must be contiguous")
        k_scale = v_scale = None
        if quantized:
            k_scale = (scales["k"] if isinstance(scales, dict) else scales.k).contiguous()
            v_scale = (scales["v"] if isinstance(scales, dict) else scales.v).contiguous()
            expected = (cache.num_pages, cache.num_kv_heads)
            if tuple(k_scale.shape) != expected or tuple(v_scale.shape) != expected:
                raise ValueError(f"scales must have shape {expected}, got {tuple(k_scale.shape)}")
            if k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
                raise ValueError("scales must be float32")
        if cache.k_cache.stride(-1) != 1 or cache.v_cache.stride(-1) != 1:
            raise ValueError("k_cache and v_cache need a contiguous head_dim axis")
        # The argument block points at the engine's own table and lengths,
        # which it updates in place: they cannot be copied to a dense layout.
        if cache.page_table.stride(-1) != 1 or not cache.seq_lens.is_contiguous():
            raise ValueError("DecodeLaunch: page_table rows and seq_lens must be contiguous")
        self.config = cfg
        self.softmax_scale = float(softmax_scale) if softmax_scale is not None else q.shape[-1] ** -0.5
        rows = q.shape[0] * q_len
        need = _hip.decode_workspace_bytes(rows, q.shape[-2], q.shape[-1], cfg["split_k"])
        self.workspace = torch.empty(max(1, need), dtype=torch.uint8, device=q.device) if need else None
        # Zeroed split-K merge counters of this launch (each run leaves them
        # zero): the decode kernel merges its partitions itself.  Runs of one
        # DecodeLaunch share them, as they share the workspace.
        self.counters = (torch.zeros(_hip.decode_counters_bytes(rows, q.shape[-2]) // 4, dtype=torch.int32,
                                     device=q.device) if cfg["split_k"] > 1 else None)
        self._keep = (cache, k_scale, v_scale)  # the argument block points into these
        self._shape, self._dtype = tuple(q.shape), q.dtype
        self._device = q.device
        self._args = _hip.decode_args(q, cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, q,
                                      cache.page_size, self.softmax_scale, cfg["split_k"],
                                      workspace=self.workspace, k_scale=k_scale, v_scale=v_scale,
                                      waves_per_group=cfg["num_warps"] or 0,
                                      pages_per_split=cfg["pages_per_split"], kernel=_KERNEL_CODES[cfg["kernel"]],
                                      counters=self.counters)

    def run(self, q: torch.Tensor, out: torch.Tensor | None = None, stream: int | None = None) -> torch.Tensor:
        """Decode ``q`` into ``out`` (default: a new tensor) on ``stream``
        (a hipStream_t handle; default torch's current stream)."""
        if tuple(q.shape) != self._shape or q.dtype != self._dtype or not q.is_contiguous():
            raise ValueError(f"DecodeLaunch.run: q must be a contiguous {self._dtype} tensor of shape {self._shape}")
        if out is None:
            out = torch.empty_like(q)
        elif tuple(out.shape) != self._shape or out.dtype != self._dtype or not out.is_contiguous():
            raise ValueError(f"DecodeLaunch.run: out must be a contiguous {self._dtype} tensor of shape {self._shape}")
        a = self._args
        a.q = q.data_ptr()
        a.out = out.data_ptr()
        _hip.decode_with_args(a, _hip.current_stream_handle(self._device) if stream is None else stream)
        return out
