"""Paged KV-cache contract: NHD pages, an int32 block table and int32 lengths.

Drop-in for ``flashattn_tile/paging.py`` (same names, fields, error types and
messages; reference lines cited per function).  The kernels read exactly this
layout:

``k_cache`` / ``v_cache``
    ``[num_pages, page_size, num_kv_heads, head_dim]``; head_dim contiguous.
    A quantised cache stores ``int8`` or ``float8_e4m3fn`` elements.
``page_table``
    ``int32 [batch, max_pages_per_seq]``: ``page_table[b, i]`` is the physical
    page holding logical block ``i`` of sequence ``b``; entries past
    ``ceil(seq_lens[b] / page_size)`` are never read.
``seq_lens``
    ``int32 [batch]`` valid tokens; token ``t`` of sequence ``b`` lives in page
    ``page_table[b, t // page_size]`` at slot ``t % page_size``.

On MI355X the whole pool is one allocation in HBM (288 GB per GPU holds e.g.
a 32-sequence x 4096-token fp16 cache of 32 KiB pages in 512 MiB); pages are
addressed through the table so a serving engine may permute them freely.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

__all__ = [
    "PagedKVCache",
    "validate_cache",
    "allocate",
    "append_tokens",
    "AppendLaunch",
    "gather_paged",
    "gather_contiguous",
]


@dataclass
class PagedKVCache:
    """Paged K/V cache plus its page table (``paging.py:30-76``)."""

    k_cache: torch.Tensor
    v_cache: torch.Tensor
    page_table: torch.Tensor
    seq_lens: torch.Tensor
    page_size: int

    @property
    def batch_size(self) -> int:
        return int(self.seq_lens.shape[0])

    @property
    def num_pages(self) -> int:
        return int(self.k_cache.shape[0])

    @property
    def num_kv_heads(self) -> int:
        return int(self.k_cache.shape[2])

    @property
    def head_dim(self) -> int:
        return int(self.k_cache.shape[3])

    @property
    def max_pages_per_seq(self) -> int:
        return int(self.page_table.shape[1])

    @property
    def capacity(self) -> int:
        """Maximum tokens per sequence addressable by the page table."""
        return self.max_pages_per_seq * self.page_size


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise AssertionError(message)


def _check_layout(cache: PagedKVCache) -> None:
    """Host-only shape/dtype/device checks (no device synchronisation)."""
    _require(isinstance(cache, PagedKVCache), "cache must be a PagedKVCache")
    k, v = cache.k_cache, cache.v_cache
    _require(k.dim() == 4, f"k_cache must be 4-D [pages, page_size, kv_heads, dim], got {tuple(k.shape)}")
    _require(k.shape == v.shape, f"k_cache {tuple(k.shape)} and v_cache {tuple(v.shape)} must match")
    _require(k.dtype == v.dtype, f"k_cache dtype {k.dtype} != v_cache dtype {v.dtype}")
    _require(k.device == v.device, "k_cache and v_cache must live on the same device")
    _require(cache.page_size > 0, "page_size must be positive")
    _require(k.shape[1] == cache.page_size, f"k_cache page dim {k.shape[1]} != page_size {cache.page_size}")
    pt, sl = cache.page_table, cache.seq_lens
    _require(pt.dtype == torch.int32, f"page_table must be int32, got {pt.dtype}")
    _require(sl.dtype == torch.int32, f"seq_lens must be int32, got {sl.dtype}")
    _require(pt.dim() == 2, "page_table must be [batch, max_pages_per_seq]")
    _require(sl.dim() == 1, "seq_lens must be [batch]")
    _require(pt.shape[0] == sl.shape[0], "page_table and seq_lens batch dimensions disagree")
    _require(pt.device == sl.device, "page_table and seq_lens must live on the same device")


def cache_stats(cache: PagedKVCache, with_total_pages: bool = False) -> tuple[int, ...]:
    """``(min_len, max_len, min_page, max_page)`` in ONE device->host copy
    (ROCm tensors: one ``fat_cache_stats`` launch; otherwise torch reductions).

    The page range covers ``page_table[:, :ceil(max_len / page_size)]`` for every
    row, the same entries ``paging.py:123-129`` inspects.  With no cached token
    the page range is reported as ``(0, -1)``.  ``with_total_pages`` appends
    ``sum_b ceil(seq_lens[b] / page_size)`` (same copy).
    """
    sl = cache.seq_lens
    pt = cache.page_table
    if sl.numel() == 0:
        return (0, 0, 0, -1, 0) if with_total_pages else (0, 0, 0, -1)
    big = torch.iinfo(torch.int32).max
    if sl.is_cuda and pt.is_cuda and sl.dtype == torch.int32 and pt.dtype == torch.int32 and \
            sl.is_contiguous() and pt.dim() == 2 and pt.stride(-1) == 1:
        from . import _hip

        if _hip.is_loaded():  # one fused launch and one copy back (fat_cache_stats)
            stats = _hip.cache_stats(sl, pt, cache.page_size)
            if stats[2] == big:
                stats[2], stats[3] = 0, -1
            return tuple(stats) if with_total_pages else tuple(stats[:4])
    max_len = sl.max()
    need = torch.div(max_len + (cache.page_size - 1), cache.page_size, rounding_mode="floor")
    cols = torch.arange(pt.shape[1], device=pt.device)
    used = (cols < need).unsqueeze(0).expand_as(pt)
    small = torch.iinfo(torch.int32).min
    if pt.numel():
        min_page = torch.where(used, pt, torch.full_like(pt, big)).min()
        max_page = torch.where(used, pt, torch.full_like(pt, small)).max()
    else:
        min_page = torch.tensor(big, dtype=torch.int32, device=pt.device)
        max_page = torch.tensor(small, dtype=torch.int32, device=pt.device)
    parts = [sl.min().to(torch.int64), max_len.to(torch.int64), min_page.to(torch.int64),
             max_page.to(torch.int64)]
    if with_total_pages:
        pages = torch.div(sl.to(torch.int64).clamp_min(0) + (cache.page_size - 1), cache.page_size,
                          rounding_mode="floor")
        parts.append(pages.sum())
    stats = [int(x) for x in torch.stack(parts).cpu().tolist()]
    if stats[2] == big:
        stats[2], stats[3] = 0, -1
    return tuple(stats)


def validate_cache(cache: PagedKVCache, *, check_pages: bool = True) -> tuple[int, int]:
    """Validate shapes, dtypes, page bounds and lengths (``paging.py:84-130``).

    Raises ``AssertionError`` naming the offending field.  Returns
    ``(min_len, max_len)`` so callers need no further synchronisation.
    """
    _check_layout(cache)
    min_len, max_len, lo, hi = cache_stats(cache)
    _require(min_len >= 0, "seq_lens must be non-negative")
    capacity = cache.max_pages_per_seq * cache.page_size
    _require(max_len <= capacity, f"seq_len {max_len} exceeds page-table capacity {capacity}")
    if check_pages and max_len > 0:
        _require(lo >= 0, "page_table contains a negative page id")
        _require(hi < cache.num_pages, f"page_table references page {hi} but cache has {cache.num_pages} pages")
    return min_len, max_len


def allocate(
    batch: int,
    max_seq_len: int,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    dtype: torch.dtype = torch.float16,
    device: torch.device | str = "cpu",
) -> PagedKVCache:
    """Zeroed cache with the contiguous mapping ``page_table[b, i] = b * pages + i``
    (``paging.py:133-169``)."""
    _require(batch > 0, "batch must be positive")
    _require(max_seq_len > 0, "max_seq_len must be positive")
    _require(num_kv_heads > 0 and head_dim > 0, "num_kv_heads and head_dim must be positive")
    _require(page_size > 0, "page_size must be positive")
    allowed = {torch.float16, torch.bfloat16, torch.float32, torch.int8}
    if getattr(torch, "float8_e4m3fn", None) is not None:
        allowed.add(torch.float8_e4m3fn)
    _require(dtype in allowed, f"unsupported cache dtype {dtype}")
    pages_per_seq = math.ceil(max_seq_len / page_size)
    num_pages = batch * pages_per_seq
    shape = (num_pages, page_size, num_kv_heads, head_dim)
    cache = PagedKVCache(
        k_cache=torch.zeros(shape, dtype=dtype, device=device),
        v_cache=torch.zeros(shape, dtype=dtype, device=device),
        page_table=torch.arange(num_pages, dtype=torch.int32, device=device).view(batch, pages_per_seq),
        seq_lens=torch.zeros(batch, dtype=torch.int32, device=device),
        page_size=page_size,
    )
    validate_cache(cache)
    return cache


def _quant_pair(cache: PagedKVCache, quantized) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Check an int8/fp8 copy ``(qcache, scales)`` of ``cache`` and return
    ``(qk, qv, k_scale, v_scale)``."""
    qcache, scales = quantized
    qk, qv = qcache.k_cache, qcache.v_cache
    sk = scales["k"] if isinstance(scales, dict) else scales.k
    sv = scales["v"] if isinstance(scales, dict) else scales.v
    fp8 = getattr(torch, "float8_e4m3fn", None)
    shape = tuple(cache.k_cache.shape)
    _require(tuple(qk.shape) == shape and tuple(qv.shape) == shape,
             f"quantised pages {tuple(qk.shape)} / {tuple(qv.shape)} must match the cache {shape}")
    _require(qk.dtype in (torch.int8, fp8) and qv.dtype == qk.dtype,
             f"quantised pages must be int8 or float8_e4m3fn, got {qk.dtype} / {qv.dtype}")
    want = (shape[0], shape[2])
    _require(tuple(sk.shape) == want and tuple(sv.shape) == want,
             f"scales must be [{want[0]}, {want[1]}], got {tuple(sk.shape)} / {tuple(sv.shape)}")
    _require(sk.dtype == torch.float32 and sv.dtype == torch.float32, "scales must be float32")
    dev = cache.k_cache.device
    _require(all(t.device == dev for t in (qk, qv, sk, sv)), "the quantised copy must live on the cache device")
    return qk, qv, sk, sv


def append_tokens(cache: PagedKVCache, new_k: torch.Tensor, new_v: torch.Tensor, quantized=None, *,
                  validate: bool = True) -> None:
    """Write one token per sequence at position ``seq_lens[b]`` through the page
    table, then increment ``seq_lens`` in place (``paging.py:172-210``).

    ``quantized``: optional ``(qcache, scales)`` from ``quant.quantize_cache``
    -- an int8/fp8 copy of this cache under the same page table.  Each
    (page, KV head) that receives a token is requantised from the updated
    pages, so the copy stays equal to ``quantize_cache`` of the updated cache
    (the reference has no incremental form; it requantises the whole cache).

    On a ROCm cache the write (and the requantisation) is the HIP kernel
    ``fat_append_kv``; the bounds checks cost one device synchronisation.
    ``validate=False`` skips them (ROCm only): an entry whose position or page
    id is out of range is then skipped on the device and its length kept.
    """
    _check_layout(cache)
    expect = (cache.batch_size, cache.num_kv_heads, cache.head_dim)
    _require(new_k.shape == expect,
             f"new_k must be [{expect[0]}, {expect[1]}, {expect[2]}], got {tuple(new_k.shape)}")
    _require(new_v.shape == new_k.shape, f"new_v shape {tuple(new_v.shape)} != new_k shape {tuple(new_k.shape)}")
    _require(new_k.dtype == cache.k_cache.dtype, f"new_k dtype {new_k.dtype} != cache dtype {cache.k_cache.dtype}")
    _require(new_v.dtype == cache.k_cache.dtype, f"new_v dtype {new_v.dtype} != cache dtype {cache.k_cache.dtype}")
    _require(new_k.device == cache.k_cache.device, "new_k must be on the cache device")
    _require(new_v.device == cache.k_cache.device, "new_v must be on the cache device")
    mirror = _quant_pair(cache, quantized) if quantized is not None else None
    if cache.k_cache.is_cuda:
        _append_hip(cache, new_k, new_v, mirror, validate)
        return

    validate_cache(cache, check_pages=False)
    pos = cache.seq_lens.long()
    if pos.numel() == 0:
        return
    block = torch.div(pos, cache.page_size, rounding_mode="floor")
    rows = torch.arange(cache.batch_size, device=cache.page_table.device)
    safe_block = block.clamp(max=cache.max_pages_per_seq - 1)
    phys = cache.page_table[rows, safe_block].long()
    # One synchronisation for all bounds checks.
    max_pos, max_block, lo, hi = (int(x) for x in torch.stack(
        [pos.max(), block.max(), phys.min(), phys.max()]).cpu().tolist())
    _require(max_pos < cache.capacity, f"append would exceed page-table capacity {cache.capacity}")
    _require(max_block < cache.max_pages_per_seq, "append would index past the page table")
    _require(lo >= 0 and hi < cache.num_pages, f"page_table maps to a page outside [0, {cache.num_pages})")
    slots = (pos % cache.page_size).to(cache.k_cache.device)
    phys = phys.to(cache.k_cache.device)
    cache.k_cache[phys, slots] = new_k
    cache.v_cache[phys, slots] = new_v
    if mirror is not None:
        from .quant import quantize_kv_pages

        qk, qv, sk, sv = mirror
        touched = torch.unique(phys)
        mode = "int8" if qk.dtype == torch.int8 else "float8_e4m3fn"
        nk, nv, nsk, nsv, _ = quantize_kv_pages(cache.k_cache[touched], cache.v_cache[touched], mode=mode)
        qk[touched], qv[touched], sk[touched], sv[touched] = nk, nv, nsk, nsv
    cache.seq_lens += 1


def _append_hip(cache: PagedKVCache, new_k: torch.Tensor, new_v: torch.Tensor, mirror, validate: bool) -> None:
    """ROCm path of :func:`append_tokens`: bounds checks in one copy, then
    ``fat_append_kv`` on the current stream."""
    from . import _hip

    dev = cache.k_cache.device
    _require(cache.page_table.device == dev and cache.seq_lens.device == dev,
             "page_table and seq_lens must live on the cache device")
    _require(cache.k_cache.stride(3) == 1 and cache.v_cache.stride(3) == 1, "the head_dim axis must be contiguous")
    _require(cache.seq_lens.is_contiguous(), "seq_lens must be contiguous (it is advanced in place)")
    if mirror is not None:
        _require(mirror[0].stride(3) == 1 and mirror[1].stride(3) == 1,
                 "the head_dim axis of the quantised pages must be contiguous")
        _require(mirror[2].stride() == mirror[3].stride(), "k and v scales must share strides")
    if cache.batch_size == 0:
        return
    pt = cache.page_table if cache.page_table.stride(1) == 1 else cache.page_table.contiguous()
    if validate:
        pos = cache.seq_lens.long()
        block = torch.div(pos, cache.page_size, rounding_mode="floor")
        rows = torch.arange(cache.batch_size, device=dev)
        phys = pt[rows, block.clamp(0, cache.max_pages_per_seq - 1)]
        min_len, max_pos, lo, hi = (int(x) for x in torch.stack(
            [pos.min(), pos.max(), phys.min().long(), phys.max().long()]).cpu().tolist())
        # Same checks, order and messages as validate_cache + paging.py:192-205.
        _require(min_len >= 0, "seq_lens must be non-negative")
        _require(max_pos <= cache.capacity, f"seq_len {max_pos} exceeds page-table capacity {cache.capacity}")
        _require(max_pos < cache.capacity, f"append would exceed page-table capacity {cache.capacity}")
        _require(lo >= 0 and hi < cache.num_pages, f"page_table maps to a page outside [0, {cache.num_pages})")
    nk = new_k if new_k.stride(2) == 1 else new_k.contiguous()
    nv = new_v if new_v.stride(2) == 1 else new_v.contiguous()
    qk = qv = sk = sv = None
    if mirror is not None:
        qk, qv, sk, sv = mirror
    _hip.append_kv(nk, nv, cache.k_cache, cache.v_cache, pt, cache.seq_lens, cache.page_size,
                   quant_k=qk, quant_v=qv, k_scale=sk, v_scale=sv, advance=True)


class AppendLaunch:
    """An append prepared once and run every decode step (plan / run).

    Construction checks the cache (and its int8/fp8 copy ``quantized``, as
    :func:`append_tokens` takes it) and fills the ``fat_append_args`` block;
    :meth:`run` writes the two new-token addresses and enqueues
    ``fat_append_kv`` on the stream: one ctypes call, no synchronisation, no
    host bounds check (entries past the table or a bad page id are skipped
    by the kernel and their lengths left, as ``append_tokens(...,
    validate=False)`` does).  ``new_k`` / ``new_v`` passed to :meth:`run` must
    be contiguous ``[batch, num_kv_heads, head_dim]`` in the cache dtype.
    ROCm tensors only.
    """

    def __init__(self, cache: PagedKVCache, quantized=None) -> None:
        from . import _hip

        _check_layout(cache)
        if not cache.k_cache.is_cuda:
            raise RuntimeError("AppendLaunch: the cache must live on a ROCm device (the HIP kernels run there)")
        dev = cache.k_cache.device
        _require(cache.page_table.device == dev and cache.seq_lens.device == dev,
                 "page_table and seq_lens must live on the cache device")
        _require(cache.k_cache.stride(3) == 1 and cache.v_cache.stride(3) == 1, "the head_dim axis must be contiguous")
        _require(cache.seq_lens.is_contiguous(), "seq_lens must be contiguous (it is advanced in place)")
        _require(cache.page_table.stride(1) == 1, "page_table rows must be contiguous")
        mirror = _quant_pair(cache, quantized) if quantized is not None else None
        qk = qv = sk = sv = None
        if mirror is not None:
            qk, qv, sk, sv = mirror
            _require(qk.stride(3) == 1 and qv.stride(3) == 1,
                     "the head_dim axis of the quantised pages must be contiguous")
            _require(sk.stride() == sv.stride(), "k and v scales must share strides")
        self._shape = (cache.batch_size, cache.num_kv_heads, cache.head_dim)
        self._dtype = cache.k_cache.dtype
        self._device = dev
        self._keep = (cache, mirror)
        tmpl = torch.empty(self._shape, dtype=self._dtype, device="meta")
        self._args = _hip.append_args(tmpl, tmpl, cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens,
                                      cache.page_size, quant_k=qk, quant_v=qv, k_scale=sk, v_scale=sv, advance=True)

    def run(self, new_k: torch.Tensor, new_v: torch.Tensor, stream: int | None = None) -> None:
        """Append ``new_k`` / ``new_v`` at ``seq_lens`` and advance it, on
        ``stream`` (a hipStream_t handle; default torch's current stream)."""
        from . import _hip

        for t in (new_k, new_v):
            if tuple(t.shape) != self._shape or t.dtype != self._dtype or not t.is_contiguous() \
                    or t.device != self._device:
                raise ValueError(f"AppendLaunch.run: new_k / new_v must be contiguous {self._dtype} "
                                 f"{self._shape} tensors on {self._device}")
        if self._shape[0] == 0:
            return
        a = self._args
        a.new_k = new_k.data_ptr()
        a.new_v = new_v.data_ptr()
        _hip.append_with_args(a, _hip.current_stream_handle(self._device) if stream is None else stream)


def gather_paged(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    page_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Padded contiguous copy ``[batch, max_len, kv_heads, dim]``; rows past a
    sequence's length are zero (``paging.py:213-256``).  A debugging/reference
    utility; the kernels never gather."""
    _require(k_cache.shape == v_cache.shape, "k_cache and v_cache shapes must match")
    _require(page_table.dtype == torch.int32, "page_table must be int32")
    _require(seq_lens.dtype == torch.int32, "seq_lens must be int32")
    _require(page_table.dim() == 2 and seq_lens.dim() == 1, "expected page_table [B, P] and seq_lens [B]")
    _require(page_table.shape[0] == seq_lens.shape[0], "page_table / seq_lens batch mismatch")
    _require(k_cache.shape[1] == page_size, "k_cache page dim != page_size")

    batch = int(seq_lens.shape[0])
    lens = [int(x) for x in seq_lens.cpu().tolist()]
    max_len = max(lens) if batch else 0
    hk, d = k_cache.shape[2], k_cache.shape[3]
    out_k = k_cache.new_zeros((batch, max_len, hk, d))
    out_v = v_cache.new_zeros((batch, max_len, hk, d))
    if max_len == 0:
        return out_k, out_v
    capacity = int(page_table.shape[1]) * page_size
    _require(max_len <= capacity, f"seq_len {max_len} exceeds page-table capacity {capacity}")

    num_pages = int(k_cache.shape[0])
    table = page_table.cpu()
    for b, length in enumerate(lens):
        if length == 0:
            continue
        ids = table[b, : math.ceil(length / page_size)].long()
        _require(int(ids.min()) >= 0 and int(ids.max()) < num_pages,
                 f"sequence {b} page id outside [0, {num_pages})")
        ids = ids.to(k_cache.device)
        out_k[b, :length] = k_cache.index_select(0, ids).reshape(-1, hk, d)[:length]
        out_v[b, :length] = v_cache.index_select(0, ids).reshape(-1, hk, d)[:length]
    return out_k, out_v


def gather_contiguous(cache: PagedKVCache) -> tuple[torch.Tensor, torch.Tensor]:
    """Validate, then gather ``cache`` into padded contiguous K/V."""
    validate_cache(cache)
    return gather_paged(cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, cache.page_size)
