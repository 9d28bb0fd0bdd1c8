"""vLLM-shaped attention backend routing prefill and decode to the HIP kernels.

Mirror of ``flashattn_tile/backend.py:37-175`` (same class, method names,
metadata fields and errors):

* ``get_name()`` -> ``"flashattn_tile"``;
* ``get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_dim)`` ->
  ``(2, num_blocks, block_size, num_kv_heads, head_dim)``;
* ``forward(query, kv_cache, attn_metadata)`` runs causal varlen prefill when
  ``attn_metadata.is_prefill`` and paged decode otherwise.

Two extension fields the reference backend lacks:
* ``kv_scales``: an int8/fp8 :class:`PagedKVCache` is routed to the quantised
  decode kernel when it carries the cache's scales;
* ``paged_prefill``: prefill reads K/V from ``kv_cache`` through the page
  table (chunked prefill; the chunk's own K/V already appended) instead of
  from the packed ``k``/``v`` the reference requires (``backend.py:158-162``).

and one extension of the decode route: a ``[batch, q_len, heads, head_dim]``
query with ``q_len > 1`` (speculative verification, the tokens' K/V already
appended) runs multi-token decode; ``q_len == 1`` is squeezed as in the
reference.
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from .kernels.decode import paged_decode_attention, paged_decode_attention_fp8, paged_decode_attention_multi
from .kernels.prefill import paged_prefill_attention, prefill_attention
from .paging import PagedKVCache, allocate


@dataclass
class AttentionMetadata:
    """Per-step metadata for :meth:`FlashAttnTileBackend.forward`."""

    page_table: torch.Tensor | None = None
    seq_lens: torch.Tensor | None = None
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    is_prefill: bool = False
    max_seqlen_q: int | None = None
    max_seqlen_k: int | None = None
    # Packed K/V of the tokens being prefilled ([total_k, num_kv_heads, head_dim]).
    k: torch.Tensor | None = None
    v: torch.Tensor | None = None
    softmax_scale: float | None = None
    # Scales of a quantised cache (QuantScales or {"k": ..., "v": ...}).
    kv_scales: object | None = None
    # Prefill from the paged cache (chunk K/V already appended) instead of k/v.
    paged_prefill: bool = False


def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                       head_dim: int) -> tuple[int, int, int, int, int]:
    """vLLM-style cache shape ``(2, blocks, block_size, kv_heads, head_dim)``."""
    return (2, int(num_blocks), int(block_size), int(num_kv_heads), int(head_dim))


def _longest(cu_seqlens: torch.Tensor, given: int | None) -> int:
    """``given`` or the longest sequence of ``cu_seqlens`` (one host read)."""
    if given is not None:
        return int(given)
    return int((cu_seqlens[1:] - cu_seqlens[:-1]).max())


class FlashAttnTileBackend:
    """Paged attention backend for the MI355X kernels.

    :meth:`forward` first names the route a call takes (:meth:`route`), then
    checks the query against it and runs it; every route is one HIP launch
    behind the wrappers of :mod:`flashattntile_amd.kernels`.
    """

    ROUTES = ("decode", "decode_quant", "decode_multi", "prefill", "prefill_paged")

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                 dtype: torch.dtype | None = None, device: torch.device | str | None = None) -> None:
        if num_heads % num_kv_heads != 0:
            raise ValueError(f"num_heads {num_heads} must be divisible by num_kv_heads {num_kv_heads}")
        if page_size <= 0:
            raise ValueError("page_size must be positive")
        self.num_heads = int(num_heads)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.page_size = int(page_size)
        self.dtype = dtype
        self.device = device

    def get_name(self) -> str:
        return "flashattn_tile"

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                           head_dim: int) -> tuple[int, int, int, int, int]:
        return get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_dim)

    @staticmethod
    def get_kv_cache_shape_per_tensor(num_blocks: int, block_size: int, num_kv_heads: int,
                                      head_dim: int) -> tuple[int, int, int, int]:
        return (int(num_blocks), int(block_size), int(num_kv_heads), int(head_dim))

    def allocate_kv_cache(self, batch: int, max_seq_len: int, dtype: torch.dtype = torch.float16,
                          device: torch.device | str = "cuda") -> PagedKVCache:
        return allocate(batch=batch, max_seq_len=max_seq_len, num_kv_heads=self.num_kv_heads,
                        head_dim=self.head_dim, page_size=self.page_size, dtype=dtype, device=device)

    # -- routing ---------------------------------------------------------
    @staticmethod
    def route(query: torch.Tensor, attn_metadata: AttentionMetadata) -> str:
        """The route ``forward`` takes (one of :attr:`ROUTES`):

        * prefill metadata -> ``prefill`` (packed K/V, ``backend.py:155-173``)
          or ``prefill_paged`` (K/V read through the page table);
        * decode with a ``[batch, q_len > 1, heads, head_dim]`` query ->
          ``decode_multi``;
        * other decode calls -> ``decode_quant`` when the metadata carries
          the cache's scales, else ``decode`` (``backend.py:175``).
        """
        meta = attn_metadata
        if meta.is_prefill:
            return "prefill_paged" if meta.paged_prefill else "prefill"
        if query.dim() == 4 and query.shape[1] > 1:
            return "decode_multi"
        return "decode" if meta.kv_scales is None else "decode_quant"

    def _check_heads(self, heads: int) -> None:
        if heads != self.num_heads:
            raise ValueError(f"query has {heads} heads, backend expects {self.num_heads}")

    @staticmethod
    def _with_metadata(kv_cache: PagedKVCache, meta: AttentionMetadata) -> PagedKVCache:
        """The cache under this step's page table / lengths where the metadata
        supplies them (``backend.py:119-130``)."""
        changes = {}
        if meta.page_table is not None:
            changes["page_table"] = meta.page_table
        if meta.seq_lens is not None:
            changes["seq_lens"] = meta.seq_lens
        return replace(kv_cache, **changes) if changes else kv_cache

    def forward(self, query: torch.Tensor, kv_cache: PagedKVCache, attn_metadata: AttentionMetadata) -> torch.Tensor:
        """Run ``query`` on the route :meth:`route` names (``backend.py:132-175``).

        A ``[batch, 1, heads, head_dim]`` decode query is squeezed to 3-D, as
        in the reference; every other route takes a 3-D query (packed tokens
        for prefill)."""
        if not isinstance(kv_cache, PagedKVCache):
            raise TypeError("kv_cache must be a PagedKVCache")
        meta = attn_metadata
        cache = self._with_metadata(kv_cache, meta)
        way = self.route(query, meta)
        scale = meta.softmax_scale
        if way == "decode_multi":
            self._check_heads(query.shape[2])
            return paged_decode_attention_multi(query, cache, softmax_scale=scale, scales=meta.kv_scales)
        if not meta.is_prefill and query.dim() == 4:
            query = query.squeeze(1)
        if query.dim() != 3:
            raise ValueError(f"query must be 3-D, got {tuple(query.shape)}")
        self._check_heads(query.shape[1])
        if way == "decode":
            return paged_decode_attention(query, cache, softmax_scale=scale)
        if way == "decode_quant":
            return paged_decode_attention_fp8(query, cache, meta.kv_scales, softmax_scale=scale)
        if way == "prefill_paged":
            if meta.cu_seqlens_q is None:
                raise ValueError("paged prefill routing requires cu_seqlens_q")
            return paged_prefill_attention(query, cache, meta.cu_seqlens_q, _longest(meta.cu_seqlens_q,
                                                                                     meta.max_seqlen_q),
                                           causal=True, softmax_scale=scale)
        # way == "prefill": packed K/V of the tokens being prefilled, always causal
        if meta.cu_seqlens_q is None or meta.cu_seqlens_k is None:
            raise ValueError("prefill routing requires cu_seqlens_q and cu_seqlens_k")
        max_q = _longest(meta.cu_seqlens_q, meta.max_seqlen_q)
        max_k = _longest(meta.cu_seqlens_k, meta.max_seqlen_k)
        if meta.k is None or meta.v is None:
            raise ValueError("prefill routing requires attn_metadata.k and attn_metadata.v "
                             "(packed [total_k, num_kv_heads, head_dim])")
        return prefill_attention(query, meta.k, meta.v, meta.cu_seqlens_q, meta.cu_seqlens_k, max_q, max_k,
                                 causal=True, softmax_scale=scale)
