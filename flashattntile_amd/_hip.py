"""ctypes binding of ``libfat_hip.so`` (the C ABI declared in ``include/fat_abi.h``).

This is the MI355X replacement of the reference's lazy nvcc build
(``flashattn_tile/native.py:17-51``): the HIP library is compiled ahead of
time (``flashattntile_amd/csrc/build.py``) and loaded here once, under a lock.
Nothing here falls back to a CPU path: if the library cannot be loaded every
entry point raises ``RuntimeError`` naming the reason.

Tensors cross the boundary as raw device pointers, element strides and sizes;
kernels are enqueued on torch's current HIP stream.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libfat_hip.so"
ABI_VERSION = 14

# enum fat_dtype
DT_F16 = 0
DT_BF16 = 1
DT_I8 = 2
DT_FP8E4M3 = 3
DT_F32 = 4

# enum fat_kernel (the `kernel` field of the decode and prefill arguments)
KERNEL_AUTO = 0
KERNEL_DECODE_VALU = 1
KERNEL_DECODE_MFMA = 2
KERNEL_DECODE_GENERIC = 3
KERNEL_PREFILL_PINGPONG = 1
KERNEL_PREFILL_4WAVE = 2
KERNEL_PREFILL_4WAVE_SPLIT = 3
KERNEL_PREFILL_WIDE = 4
KERNEL_PREFILL_GENERIC = 5

# enum fat_rows (the `rows` field of the paged prefill arguments)
ROWS_AUTO = 0
ROWS_WIDE = 1
ROWS_LANE = 2

EXPORTED_SYMBOLS = (
    "fat_abi_version",
    "fat_last_error",
    "fat_paged_decode_workspace_bytes",
    "fat_paged_decode_counters_bytes",
    "fat_paged_decode",
    "fat_paged_decode_noalloc",
    "fat_prefill_workspace_bytes",
    "fat_prefill_varlen_workspace_bytes",
    "fat_prefill_varlen",
    "fat_prefill_paged_workspace_bytes",
    "fat_prefill_paged",
    "fat_quantize_pages",
    "fat_append_kv",
    "fat_cache_stats",
)

_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32
_c_vp = ctypes.c_void_p


class DecodeArgs(ctypes.Structure):
    """Mirror of ``fat_decode_args``."""

    _fields_ = [
        ("q", _c_vp),
        ("k_cache", _c_vp),
        ("v_cache", _c_vp),
        ("k_scale", _c_vp),
        ("v_scale", _c_vp),
        ("page_table", _c_vp),
        ("seq_lens", _c_vp),
        ("out", _c_vp),
        ("workspace", _c_vp),
        ("q_stride_b", _c_i64),
        ("q_stride_h", _c_i64),
        ("k_stride_page", _c_i64),
        ("k_stride_slot", _c_i64),
        ("k_stride_head", _c_i64),
        ("v_stride_page", _c_i64),
        ("v_stride_slot", _c_i64),
        ("v_stride_head", _c_i64),
        ("scale_stride_page", _c_i64),
        ("scale_stride_head", _c_i64),
        ("page_table_stride", _c_i64),
        ("out_stride_b", _c_i64),
        ("out_stride_h", _c_i64),
        ("batch", _c_i32),
        ("num_heads", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("page_size", _c_i32),
        ("num_pages", _c_i32),
        ("max_pages", _c_i32),
        ("split_k", _c_i32),
        ("waves_per_group", _c_i32),
        ("q_dtype", _c_i32),
        ("kv_dtype", _c_i32),
        ("pages_per_split", _c_i32),
        ("softmax_scale", ctypes.c_float),
        ("q_stride_t", _c_i64),
        ("out_stride_t", _c_i64),
        ("q_len", _c_i32),
        ("kernel", _c_i32),
        ("merge_counters", _c_vp),
    ]


class PrefillArgs(ctypes.Structure):
    """Mirror of ``fat_prefill_args``."""

    _fields_ = [
        ("q", _c_vp),
        ("k", _c_vp),
        ("v", _c_vp),
        ("cu_seqlens_q", _c_vp),
        ("cu_seqlens_k", _c_vp),
        ("out", _c_vp),
        ("workspace", _c_vp),
        ("q_stride_t", _c_i64),
        ("q_stride_h", _c_i64),
        ("k_stride_t", _c_i64),
        ("k_stride_h", _c_i64),
        ("v_stride_t", _c_i64),
        ("v_stride_h", _c_i64),
        ("out_stride_t", _c_i64),
        ("out_stride_h", _c_i64),
        ("batch", _c_i32),
        ("total_q", _c_i32),
        ("total_k", _c_i32),
        ("num_heads", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("max_seqlen_q", _c_i32),
        ("max_seqlen_k", _c_i32),
        ("causal", _c_i32),
        ("dtype", _c_i32),
        ("softmax_scale", ctypes.c_float),
        ("kernel", _c_i32),
    ]


class PrefillPagedArgs(ctypes.Structure):
    """Mirror of ``fat_prefill_paged_args``."""

    _fields_ = [
        ("q", _c_vp),
        ("k_cache", _c_vp),
        ("v_cache", _c_vp),
        ("page_table", _c_vp),
        ("seq_lens", _c_vp),
        ("cu_seqlens_q", _c_vp),
        ("out", _c_vp),
        ("q_stride_t", _c_i64),
        ("q_stride_h", _c_i64),
        ("k_stride_page", _c_i64),
        ("k_stride_slot", _c_i64),
        ("k_stride_head", _c_i64),
        ("v_stride_page", _c_i64),
        ("v_stride_slot", _c_i64),
        ("v_stride_head", _c_i64),
        ("page_table_stride", _c_i64),
        ("out_stride_t", _c_i64),
        ("out_stride_h", _c_i64),
        ("batch", _c_i32),
        ("total_q", _c_i32),
        ("num_heads", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("page_size", _c_i32),
        ("num_pages", _c_i32),
        ("max_pages", _c_i32),
        ("max_seqlen_q", _c_i32),
        ("causal", _c_i32),
        ("dtype", _c_i32),
        ("softmax_scale", ctypes.c_float),
        ("kernel", _c_i32),
        ("rows", _c_i32),
        ("workspace", _c_vp),
    ]


class QuantizeArgs(ctypes.Structure):
    """Mirror of ``fat_quantize_args``."""

    _fields_ = [
        ("src", _c_vp),
        ("dst", _c_vp),
        ("scale", _c_vp),
        ("src_stride_page", _c_i64),
        ("src_stride_slot", _c_i64),
        ("src_stride_head", _c_i64),
        ("dst_stride_page", _c_i64),
        ("dst_stride_slot", _c_i64),
        ("dst_stride_head", _c_i64),
        ("scale_stride_page", _c_i64),
        ("scale_stride_head", _c_i64),
        ("num_pages", _c_i32),
        ("page_size", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("src_dtype", _c_i32),
        ("dst_dtype", _c_i32),
    ]


class AppendArgs(ctypes.Structure):
    """Mirror of ``fat_append_args``."""

    _fields_ = [
        ("new_k", _c_vp),
        ("new_v", _c_vp),
        ("k_cache", _c_vp),
        ("v_cache", _c_vp),
        ("quant_k_cache", _c_vp),
        ("quant_v_cache", _c_vp),
        ("k_scale", _c_vp),
        ("v_scale", _c_vp),
        ("page_table", _c_vp),
        ("seq_lens", _c_vp),
        ("new_k_stride_b", _c_i64),
        ("new_k_stride_h", _c_i64),
        ("new_v_stride_b", _c_i64),
        ("new_v_stride_h", _c_i64),
        ("k_stride_page", _c_i64),
        ("k_stride_slot", _c_i64),
        ("k_stride_head", _c_i64),
        ("v_stride_page", _c_i64),
        ("v_stride_slot", _c_i64),
        ("v_stride_head", _c_i64),
        ("qk_stride_page", _c_i64),
        ("qk_stride_slot", _c_i64),
        ("qk_stride_head", _c_i64),
        ("qv_stride_page", _c_i64),
        ("qv_stride_slot", _c_i64),
        ("qv_stride_head", _c_i64),
        ("scale_stride_page", _c_i64),
        ("scale_stride_head", _c_i64),
        ("page_table_stride", _c_i64),
        ("batch", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("page_size", _c_i32),
        ("num_pages", _c_i32),
        ("max_pages", _c_i32),
        ("dtype", _c_i32),
        ("quant_dtype", _c_i32),
        ("advance", _c_i32),
    ]


class CacheStatsArgs(ctypes.Structure):
    """Mirror of ``fat_cache_stats_args``."""

    _fields_ = [
        ("seq_lens", _c_vp),
        ("page_table", _c_vp),
        ("page_table_stride", _c_i64),
        ("batch", _c_i32),
        ("max_pages", _c_i32),
        ("page_size", _c_i32),
        ("out", _c_vp),
    ]


_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None
_ERROR: str | None = None
_TRIED = False


def _load() -> None:
    global _LIB, _ERROR, _TRIED
    with _LOCK:
        if _TRIED:
            return
        _TRIED = True
        path = Path(os.environ.get("FAT_HIP_LIB", str(LIB_PATH)))
        if not path.exists():
            _ERROR = f"{path} not found; build it with `python -m flashattntile_amd.csrc.build`"
            return
        try:
            # torch's HIP runtime is already loaded (import torch above), so the
            # library binds to the same libamdhip64 instance.
            lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
        except OSError as exc:
            _ERROR = f"cannot load {path}: {exc}"
            return
        lib.fat_abi_version.restype = ctypes.c_int
        version = lib.fat_abi_version()
        if version != ABI_VERSION:  # before binding: an old build lacks newer symbols
            _ERROR = f"{path} has ABI version {version}, expected {ABI_VERSION}; rebuild it"
            return
        lib.fat_last_error.restype = ctypes.c_char_p
        lib.fat_paged_decode_workspace_bytes.restype = ctypes.c_size_t
        lib.fat_paged_decode_workspace_bytes.argtypes = [_c_i32, _c_i32, _c_i32, _c_i32]
        lib.fat_paged_decode.restype = ctypes.c_int
        lib.fat_paged_decode.argtypes = [ctypes.POINTER(DecodeArgs), _c_vp]
        lib.fat_paged_decode_noalloc.restype = ctypes.c_int
        lib.fat_paged_decode_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), _c_vp]
        lib.fat_prefill_workspace_bytes.restype = ctypes.c_size_t
        lib.fat_prefill_workspace_bytes.argtypes = [_c_i32, _c_i32, _c_i32]
        lib.fat_prefill_varlen_workspace_bytes.restype = ctypes.c_size_t
        lib.fat_prefill_varlen_workspace_bytes.argtypes = [ctypes.POINTER(PrefillArgs)]
        lib.fat_prefill_varlen.restype = ctypes.c_int
        lib.fat_prefill_varlen.argtypes = [ctypes.POINTER(PrefillArgs), _c_vp]
        lib.fat_prefill_paged_workspace_bytes.restype = ctypes.c_size_t
        lib.fat_prefill_paged_workspace_bytes.argtypes = [ctypes.POINTER(PrefillPagedArgs)]
        lib.fat_prefill_paged.restype = ctypes.c_int
        lib.fat_prefill_paged.argtypes = [ctypes.POINTER(PrefillPagedArgs), _c_vp]
        lib.fat_quantize_pages.restype = ctypes.c_int
        lib.fat_quantize_pages.argtypes = [ctypes.POINTER(QuantizeArgs), _c_vp]
        lib.fat_append_kv.restype = ctypes.c_int
        lib.fat_append_kv.argtypes = [ctypes.POINTER(AppendArgs), _c_vp]
        lib.fat_cache_stats.restype = ctypes.c_int
        lib.fat_cache_stats.argtypes = [ctypes.POINTER(CacheStatsArgs), _c_vp]
        _LIB = lib


def is_loaded() -> bool:
    """Load the library once; True if it is usable."""
    _load()
    return _LIB is not None


def load_error() -> str:
    """Why the library is unusable ('' when it loaded)."""
    _load()
    return "" if _LIB is not None else (_ERROR or "libfat_hip.so not loaded")


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError (no fallback) when unavailable."""
    _load()
    if _LIB is None:
        raise RuntimeError(f"HIP kernel library unavailable: {_ERROR}")
    return _LIB


def cache_stats(seq_lens: torch.Tensor, page_table: torch.Tensor, page_size: int) -> list[int]:
    """``fat_cache_stats`` on the current stream, then one copy back:
    ``[min_len, max_len, min_page, max_page, total_pages]`` (the page range
    over the columns the longest sequence uses; INT32_MAX / INT32_MIN when
    none).  ``seq_lens`` int32 [B] contiguous, ``page_table`` int32 [B, M]
    with a contiguous last axis."""
    out = torch.empty(5, dtype=torch.int64, device=seq_lens.device)
    a = CacheStatsArgs()
    a.seq_lens = _ptr(seq_lens)
    a.page_table = _ptr(page_table)
    a.page_table_stride = page_table.stride(0)
    a.batch = seq_lens.shape[0]
    a.max_pages = page_table.shape[1]
    a.page_size = int(page_size)
    a.out = _ptr(out)
    stream = torch.cuda.current_stream(seq_lens.device)
    _check(lib().fat_cache_stats(ctypes.byref(a), _c_vp(int(stream.cuda_stream))), "fat_cache_stats")
    host = torch.empty(5, dtype=torch.int64, pin_memory=True)
    host.copy_(out, non_blocking=True)
    stream.synchronize()
    return host.tolist()


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return DT_F16
    if dtype == torch.bfloat16:
        return DT_BF16
    if dtype == torch.int8:
        return DT_I8
    if dtype == getattr(torch, "float8_e4m3fn", None):
        return DT_FP8E4M3
    if dtype == torch.float32:
        return DT_F32
    raise TypeError(f"no HIP kernel element type for {dtype}")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().fat_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def current_stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def decode_workspace_bytes(batch: int, num_heads: int, head_dim: int, split_k: int) -> int:
    return int(lib().fat_paged_decode_workspace_bytes(batch, num_heads, head_dim, split_k))


def decode_counters_bytes(rows: int, num_heads: int) -> int:
    """Bytes of the split-K merge counters for ``rows`` = batch * q_len."""
    return int(lib().fat_paged_decode_counters_bytes(rows, num_heads))


def prefill_workspace_bytes(total_k: int, num_kv_heads: int, head_dim: int) -> int:
    return int(lib().fat_prefill_workspace_bytes(total_k, num_kv_heads, head_dim))


def prefill_varlen_workspace_bytes(a: PrefillArgs) -> int:
    """Workspace bytes the launch of ``a`` uses (0: it runs without one)."""
    return int(lib().fat_prefill_varlen_workspace_bytes(ctypes.byref(a)))


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())


def paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    out: torch.Tensor,
    page_size: int,
    softmax_scale: float,
    split_k: int,
    workspace: torch.Tensor | None = None,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    stream: int | None = None,
    waves_per_group: int = 0,
    pages_per_split: int = 0,
    kernel: int = KERNEL_AUTO,
    counters: torch.Tensor | None = None,
) -> None:
    """Enqueue ``fat_paged_decode`` for already-validated device tensors.

    ``q``/``out`` are ``[B, H, D]`` (one query per sequence) or
    ``[B, T, H, D]`` (multi-token decode, ``q_len = T``).  ``counters``:
    zeroed int32 merge counters (``decode_counters_bytes``) for the split-K
    merge inside the decode launch, or None (a second kernel merges)."""
    a = decode_args(q, k_cache, v_cache, page_table, seq_lens, out, page_size, softmax_scale, split_k,
                    workspace=workspace, k_scale=k_scale, v_scale=v_scale, waves_per_group=waves_per_group,
                    pages_per_split=pages_per_split, kernel=kernel, counters=counters)
    handle = current_stream_handle(q.device) if stream is None else stream
    _check(lib().fat_paged_decode(ctypes.byref(a), _c_vp(handle)), "fat_paged_decode")


def decode_args(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    out: torch.Tensor,
    page_size: int,
    softmax_scale: float,
    split_k: int,
    workspace: torch.Tensor | None = None,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    waves_per_group: int = 0,
    pages_per_split: int = 0,
    kernel: int = KERNEL_AUTO,
    counters: torch.Tensor | None = None,
) -> DecodeArgs:
    """The ``fat_decode_args`` block of a decode launch (see paged_decode)."""
    multi = q.dim() == 4
    a = DecodeArgs()
    a.q = _ptr(q)
    a.k_cache = _ptr(k_cache)
    a.v_cache = _ptr(v_cache)
    a.k_scale = _ptr(k_scale)
    a.v_scale = _ptr(v_scale)
    a.page_table = _ptr(page_table)
    a.seq_lens = _ptr(seq_lens)
    a.out = _ptr(out)
    a.workspace = _ptr(workspace)
    if multi:
        a.q_stride_b, a.q_stride_t, a.q_stride_h = q.stride(0), q.stride(1), q.stride(2)
        a.out_stride_t = out.stride(1)
        a.q_len = q.shape[1]
    else:
        a.q_stride_b, a.q_stride_h = q.stride(0), q.stride(1)
    a.k_stride_page, a.k_stride_slot, a.k_stride_head = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.v_stride_page, a.v_stride_slot, a.v_stride_head = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    if k_scale is not None:
        a.scale_stride_page, a.scale_stride_head = k_scale.stride(0), k_scale.stride(1)
    a.page_table_stride = page_table.stride(0)
    a.out_stride_b, a.out_stride_h = out.stride(0), out.stride(2 if multi else 1)
    a.batch = q.shape[0]
    a.num_heads = q.shape[-2]
    a.num_kv_heads = k_cache.shape[2]
    a.head_dim = q.shape[-1]
    a.page_size = int(page_size)
    a.num_pages = k_cache.shape[0]
    a.max_pages = page_table.shape[1]
    a.split_k = int(split_k)
    a.waves_per_group = int(waves_per_group)
    a.q_dtype = dtype_code(q.dtype)
    a.kv_dtype = dtype_code(k_cache.dtype)
    a.pages_per_split = int(pages_per_split)
    a.softmax_scale = float(softmax_scale)
    a.kernel = int(kernel)
    a.merge_counters = _ptr(counters)
    return a


def decode_with_args(a: DecodeArgs, stream: int) -> None:
    """Enqueue ``fat_paged_decode`` with a prepared argument block."""
    _check(lib().fat_paged_decode(ctypes.byref(a), _c_vp(stream)), "fat_paged_decode")


# FAT_DECODE_NOALLOC_MAX_WORKSPACE of include/fat_abi.h
NOALLOC_MAX_WORKSPACE = 32 << 20


def decode_noalloc_with_args(a: DecodeArgs, stream: int) -> None:
    """Enqueue ``fat_paged_decode_noalloc`` (split-K workspace inside the
    library; ``a.workspace`` is ignored) with a prepared argument block."""
    _check(lib().fat_paged_decode_noalloc(ctypes.byref(a), _c_vp(stream)), "fat_paged_decode_noalloc")


def prefill_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    out: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    causal: bool,
    softmax_scale: float,
    workspace: torch.Tensor | None = None,
    stream: int | None = None,
    kernel: int = KERNEL_AUTO,
) -> None:
    """Enqueue ``fat_prefill_varlen`` for already-validated device tensors."""
    a = prefill_args(q, k, v, cu_seqlens_q, cu_seqlens_k, out, max_seqlen_q, max_seqlen_k, causal,
                     softmax_scale, workspace=workspace, kernel=kernel)
    prefill_varlen_with_args(a, current_stream_handle(q.device) if stream is None else stream)


def prefill_varlen_with_args(a: PrefillArgs, stream: int) -> None:
    """Enqueue ``fat_prefill_varlen`` from a filled argument block."""
    _check(lib().fat_prefill_varlen(ctypes.byref(a), _c_vp(stream)), "fat_prefill_varlen")


def prefill_args(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    out: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    causal: bool,
    softmax_scale: float,
    workspace: torch.Tensor | None = None,
    kernel: int = KERNEL_AUTO,
) -> PrefillArgs:
    """The ``fat_prefill_args`` block of a packed prefill launch (see
    prefill_varlen).  It holds the tensors' addresses: they must stay alive
    and in place while the block is used."""
    a = PrefillArgs()
    a.q = _ptr(q)
    a.k = _ptr(k)
    a.v = _ptr(v)
    a.cu_seqlens_q = _ptr(cu_seqlens_q)
    a.cu_seqlens_k = _ptr(cu_seqlens_k)
    a.out = _ptr(out)
    a.workspace = _ptr(workspace)
    a.q_stride_t, a.q_stride_h = q.stride(0), q.stride(1)
    a.k_stride_t, a.k_stride_h = k.stride(0), k.stride(1)
    a.v_stride_t, a.v_stride_h = v.stride(0), v.stride(1)
    a.out_stride_t, a.out_stride_h = out.stride(0), out.stride(1)
    a.batch = cu_seqlens_q.shape[0] - 1
    a.total_q = q.shape[0]
    a.total_k = k.shape[0]
    a.num_heads = q.shape[1]
    a.num_kv_heads = k.shape[1]
    a.head_dim = q.shape[2]
    a.max_seqlen_q = int(max_seqlen_q)
    a.max_seqlen_k = int(max_seqlen_k)
    a.causal = 1 if causal else 0
    a.dtype = dtype_code(q.dtype)
    a.softmax_scale = float(softmax_scale)
    a.kernel = int(kernel)
    return a


def prefill_paged_workspace_bytes(a: PrefillPagedArgs) -> int:
    """Workspace bytes the paged launch of ``a`` uses (0: it runs without one)."""
    return int(lib().fat_prefill_paged_workspace_bytes(ctypes.byref(a)))


def prefill_paged_with_args(a: PrefillPagedArgs, stream: int) -> None:
    _check(lib().fat_prefill_paged(ctypes.byref(a), _c_vp(stream)), "fat_prefill_paged")


def prefill_paged(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    out: torch.Tensor,
    page_size: int,
    max_seqlen_q: int,
    causal: bool,
    softmax_scale: float,
    stream: int | None = None,
    kernel: int = KERNEL_AUTO,
    rows: int = ROWS_AUTO,
    workspace: torch.Tensor | None = None,
) -> None:
    """Enqueue ``fat_prefill_paged`` for already-validated device tensors
    (``workspace``: None, or at least :func:`prefill_paged_workspace_bytes`
    of the launch, 256-byte aligned)."""
    a = prefill_paged_args(q, k_cache, v_cache, page_table, seq_lens, cu_seqlens_q, out, page_size, max_seqlen_q,
                           causal, softmax_scale, kernel, rows, workspace)
    handle = current_stream_handle(q.device) if stream is None else stream
    prefill_paged_with_args(a, handle)


def prefill_paged_args(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    out: torch.Tensor,
    page_size: int,
    max_seqlen_q: int,
    causal: bool,
    softmax_scale: float,
    kernel: int = KERNEL_AUTO,
    rows: int = ROWS_AUTO,
    workspace: torch.Tensor | None = None,
) -> PrefillPagedArgs:
    """The ``fat_prefill_paged_args`` block of a launch."""
    a = PrefillPagedArgs()
    a.q = _ptr(q)
    a.k_cache = _ptr(k_cache)
    a.v_cache = _ptr(v_cache)
    a.page_table = _ptr(page_table)
    a.seq_lens = _ptr(seq_lens)
    a.cu_seqlens_q = _ptr(cu_seqlens_q)
    a.out = _ptr(out)
    a.q_stride_t, a.q_stride_h = q.stride(0), q.stride(1)
    a.k_stride_page, a.k_stride_slot, a.k_stride_head = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.v_stride_page, a.v_stride_slot, a.v_stride_head = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    a.page_table_stride = page_table.stride(0)
    a.out_stride_t, a.out_stride_h = out.stride(0), out.stride(1)
    a.batch = cu_seqlens_q.shape[0] - 1
    a.total_q = q.shape[0]
    a.num_heads = q.shape[1]
    a.num_kv_heads = k_cache.shape[2]
    a.head_dim = q.shape[2]
    a.page_size = int(page_size)
    a.num_pages = k_cache.shape[0]
    a.max_pages = page_table.shape[1]
    a.max_seqlen_q = int(max_seqlen_q)
    a.causal = 1 if causal else 0
    a.dtype = dtype_code(q.dtype)
    a.softmax_scale = float(softmax_scale)
    a.kernel = int(kernel)
    a.rows = int(rows)
    a.workspace = _ptr(workspace)
    return a


def quantize_pages(src: torch.Tensor, dst: torch.Tensor, scale: torch.Tensor, stream: int | None = None) -> None:
    """Enqueue ``fat_quantize_pages``: ``src`` [pages, P, Hkv, D] fp16/bf16/fp32
    into int8/fp8 codes ``dst`` (same shape) and fp32 ``scale`` [pages, Hkv]."""
    a = QuantizeArgs()
    a.src = _ptr(src)
    a.dst = _ptr(dst)
    a.scale = _ptr(scale)
    a.src_stride_page, a.src_stride_slot, a.src_stride_head = src.stride(0), src.stride(1), src.stride(2)
    a.dst_stride_page, a.dst_stride_slot, a.dst_stride_head = dst.stride(0), dst.stride(1), dst.stride(2)
    a.scale_stride_page, a.scale_stride_head = scale.stride(0), scale.stride(1)
    a.num_pages, a.page_size, a.num_kv_heads, a.head_dim = (int(x) for x in src.shape)
    a.src_dtype = dtype_code(src.dtype)
    a.dst_dtype = dtype_code(dst.dtype)
    handle = current_stream_handle(src.device) if stream is None else stream
    _check(lib().fat_quantize_pages(ctypes.byref(a), _c_vp(handle)), "fat_quantize_pages")


def append_kv(
    new_k: torch.Tensor,
    new_v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    page_size: int,
    quant_k: torch.Tensor | None = None,
    quant_v: torch.Tensor | None = None,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    advance: bool = True,
    stream: int | None = None,
) -> None:
    """Enqueue ``fat_append_kv`` for already-validated device tensors."""
    a = append_args(new_k, new_v, k_cache, v_cache, page_table, seq_lens, page_size, quant_k=quant_k,
                    quant_v=quant_v, k_scale=k_scale, v_scale=v_scale, advance=advance)
    handle = current_stream_handle(k_cache.device) if stream is None else stream
    _check(lib().fat_append_kv(ctypes.byref(a), _c_vp(handle)), "fat_append_kv")


def append_args(
    new_k: torch.Tensor,
    new_v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    page_size: int,
    quant_k: torch.Tensor | None = None,
    quant_v: torch.Tensor | None = None,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    advance: bool = True,
) -> AppendArgs:
    """The ``fat_append_args`` block of an append (see append_kv)."""
    a = AppendArgs()
    a.new_k = _ptr(new_k)
    a.new_v = _ptr(new_v)
    a.k_cache = _ptr(k_cache)
    a.v_cache = _ptr(v_cache)
    a.quant_k_cache = _ptr(quant_k)
    a.quant_v_cache = _ptr(quant_v)
    a.k_scale = _ptr(k_scale)
    a.v_scale = _ptr(v_scale)
    a.page_table = _ptr(page_table)
    a.seq_lens = _ptr(seq_lens)
    a.new_k_stride_b, a.new_k_stride_h = new_k.stride(0), new_k.stride(1)
    a.new_v_stride_b, a.new_v_stride_h = new_v.stride(0), new_v.stride(1)
    a.k_stride_page, a.k_stride_slot, a.k_stride_head = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.v_stride_page, a.v_stride_slot, a.v_stride_head = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    if quant_k is not None:
        a.qk_stride_page, a.qk_stride_slot, a.qk_stride_head = quant_k.stride(0), quant_k.stride(1), quant_k.stride(2)
        a.quant_dtype = dtype_code(quant_k.dtype)
    if quant_v is not None:
        a.qv_stride_page, a.qv_stride_slot, a.qv_stride_head = quant_v.stride(0), quant_v.stride(1), quant_v.stride(2)
    if k_scale is not None:
        a.scale_stride_page, a.scale_stride_head = k_scale.stride(0), k_scale.stride(1)
    a.page_table_stride = page_table.stride(0)
    a.batch = new_k.shape[0]
    a.num_kv_heads = k_cache.shape[2]
    a.head_dim = k_cache.shape[3]
    a.page_size = int(page_size)
    a.num_pages = k_cache.shape[0]
    a.max_pages = page_table.shape[1]
    a.dtype = dtype_code(k_cache.dtype)
    a.advance = 1 if advance else 0
    return a


def append_with_args(a: AppendArgs, stream: int) -> None:
    """Enqueue ``fat_append_kv`` with a prepared argument block."""
    _check(lib().fat_append_kv(ctypes.byref(a), _c_vp(stream)), "fat_append_kv")
