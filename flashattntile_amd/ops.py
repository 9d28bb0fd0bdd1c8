"""``torch.library`` custom ops -- the drop-in operator boundary.

Same namespace, names and schemas as ``flashattn_tile/ops.py:35-122``:

``flashattn_tile::paged_decode``
    ``(Tensor q, Tensor k_cache, Tensor v_cache, Tensor page_table,
    Tensor seq_lens, SymInt page_size, float softmax_scale, SymInt split_k)
    -> Tensor``
``flashattn_tile::prefill_varlen``
    ``(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, Tensor cu_seqlens_k,
    SymInt max_seqlen_q, SymInt max_seqlen_k, bool causal,
    float softmax_scale) -> Tensor``

plus three extensions the reference lacks (its quantised decode had no op,
its prefill needs packed K/V, and its decode takes one query):

``flashattn_tile::paged_decode_quant``
    ``(Tensor q, Tensor k_cache, Tensor v_cache, Tensor k_scale,
    Tensor v_scale, Tensor page_table, Tensor seq_lens, SymInt page_size,
    float softmax_scale, SymInt split_k) -> Tensor``
``flashattn_tile::prefill_paged``
    ``(Tensor q, Tensor k_cache, Tensor v_cache, Tensor page_table,
    Tensor seq_lens, Tensor cu_seqlens_q, SymInt max_seqlen_q,
    SymInt page_size, bool causal, float softmax_scale) -> Tensor``
``flashattn_tile::paged_decode_multi``
    ``(Tensor q, Tensor k_cache, Tensor v_cache, Tensor page_table,
    Tensor seq_lens, SymInt page_size, float softmax_scale, SymInt split_k,
    Tensor? k_scale=None, Tensor? v_scale=None) -> Tensor`` -- multi-token
    (speculative) decode, q ``[batch, q_len, heads, head_dim]``; the
    reference's decode takes one query per sequence (``decode.py:548-553``).

The real implementations call the gfx950 HIP kernels through the C ABI; the
fake implementations touch metadata only, so ``torch.compile(fullgraph=True)``
graphs hold the ops without graph breaks.
"""

from __future__ import annotations

import torch

from .kernels.decode import paged_decode_attention, paged_decode_attention_fp8, paged_decode_attention_multi
from .kernels.prefill import paged_prefill_attention, prefill_attention
from .paging import PagedKVCache

__all__ = [
    "paged_decode",
    "prefill_varlen",
    "paged_decode_quant",
    "prefill_paged",
    "paged_decode_multi",
    "ops_available",
    "PAGED_DECODE_OP",
    "PREFILL_OP",
    "PAGED_DECODE_QUANT_OP",
    "PREFILL_PAGED_OP",
    "PAGED_DECODE_MULTI_OP",
]

PAGED_DECODE_OP = "flashattn_tile::paged_decode"
PREFILL_OP = "flashattn_tile::prefill_varlen"
PAGED_DECODE_QUANT_OP = "flashattn_tile::paged_decode_quant"
PREFILL_PAGED_OP = "flashattn_tile::prefill_paged"
PAGED_DECODE_MULTI_OP = "flashattn_tile::paged_decode_multi"


@torch.library.custom_op(PAGED_DECODE_OP, mutates_args=())
def paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    page_size: int,
    softmax_scale: float,
    split_k: int,
) -> torch.Tensor:
    """Paged decode attention (``ops.py:35-55``); ``split_k`` is honoured exactly."""
    cache = PagedKVCache(k_cache=k_cache, v_cache=v_cache, page_table=page_table,
                         seq_lens=seq_lens, page_size=int(page_size))
    return paged_decode_attention(q, cache, softmax_scale=softmax_scale, config={"split_k": int(split_k)})


@paged_decode.register_fake
def _paged_decode_fake(q, k_cache, v_cache, page_table, seq_lens, page_size, softmax_scale, split_k):
    torch._check(q.dim() == 3, lambda: f"q must be 3-D, got {q.dim()}")
    torch._check(q.shape[0] == seq_lens.shape[0], lambda: "q batch must match seq_lens")
    torch._check(q.shape[2] == k_cache.shape[3], lambda: "q head_dim must match cache")
    torch._check(q.shape[1] % k_cache.shape[2] == 0, lambda: "heads must be divisible by KV heads")
    return q.new_empty(q.shape)


@torch.library.custom_op(PREFILL_OP, mutates_args=())
def prefill_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    causal: bool,
    softmax_scale: float,
) -> torch.Tensor:
    """Packed varlen prefill attention (``ops.py:76-99``)."""
    return prefill_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), int(max_seqlen_k),
                             causal=bool(causal), softmax_scale=softmax_scale)


@prefill_varlen.register_fake
def _prefill_varlen_fake(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal, softmax_scale):
    torch._check(q.dim() == 3, lambda: f"q must be 3-D, got {q.dim()}")
    torch._check(k.shape == v.shape, lambda: "k and v shapes must match")
    torch._check(q.shape[2] == k.shape[2], lambda: "q and k head_dim must match")
    torch._check(q.shape[1] % k.shape[1] == 0, lambda: "heads must be divisible by KV heads")
    return q.new_empty(q.shape)


@torch.library.custom_op(PAGED_DECODE_QUANT_OP, mutates_args=())
def paged_decode_quant(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    page_size: int,
    softmax_scale: float,
    split_k: int,
) -> torch.Tensor:
    """Paged decode over an int8 / float8_e4m3fn cache with per-(page, KV-head)
    fp32 scales (extension of ``decode.py:645-704``)."""
    cache = PagedKVCache(k_cache=k_cache, v_cache=v_cache, page_table=page_table,
                         seq_lens=seq_lens, page_size=int(page_size))
    return paged_decode_attention_fp8(q, cache, {"k": k_scale, "v": v_scale}, softmax_scale=softmax_scale,
                                      config={"split_k": int(split_k)})


@paged_decode_quant.register_fake
def _paged_decode_quant_fake(q, k_cache, v_cache, k_scale, v_scale, page_table, seq_lens, page_size,
                             softmax_scale, split_k):
    torch._check(q.dim() == 3, lambda: f"q must be 3-D, got {q.dim()}")
    torch._check(q.shape[0] == seq_lens.shape[0], lambda: "q batch must match seq_lens")
    torch._check(q.shape[2] == k_cache.shape[3], lambda: "q head_dim must match cache")
    torch._check(q.shape[1] % k_cache.shape[2] == 0, lambda: "heads must be divisible by KV heads")
    return q.new_empty(q.shape)


@torch.library.custom_op(PREFILL_PAGED_OP, mutates_args=())
def prefill_paged(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    max_seqlen_q: int,
    page_size: int,
    causal: bool,
    softmax_scale: float,
) -> torch.Tensor:
    """Paged (chunked) prefill: packed queries against each sequence's
    ``seq_lens[b]`` keys in the paged cache (extension of ``ops.py:76-99``)."""
    cache = PagedKVCache(k_cache=k_cache, v_cache=v_cache, page_table=page_table,
                         seq_lens=seq_lens, page_size=int(page_size))
    return paged_prefill_attention(q, cache, cu_seqlens_q, int(max_seqlen_q), causal=bool(causal),
                                   softmax_scale=softmax_scale)


@prefill_paged.register_fake
def _prefill_paged_fake(q, k_cache, v_cache, page_table, seq_lens, cu_seqlens_q, max_seqlen_q, page_size, causal,
                        softmax_scale):
    torch._check(q.dim() == 3, lambda: f"q must be 3-D, got {q.dim()}")
    torch._check(cu_seqlens_q.shape[0] == seq_lens.shape[0] + 1, lambda: "cu_seqlens_q must have batch + 1 entries")
    torch._check(q.shape[2] == k_cache.shape[3], lambda: "q head_dim must match cache")
    torch._check(q.shape[1] % k_cache.shape[2] == 0, lambda: "heads must be divisible by KV heads")
    return q.new_empty(q.shape)


@torch.library.custom_op(PAGED_DECODE_MULTI_OP, mutates_args=())
def paged_decode_multi(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    page_size: int,
    softmax_scale: float,
    split_k: int,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
) -> torch.Tensor:
    """Multi-token decode: token t of sequence b attends keys
    ``j <= seq_lens[b] - q_len + t``.  ``split_k`` >= 1 is honoured; 0 takes
    the library's launch (tuned store, else heuristic).  ``k_scale`` /
    ``v_scale`` select an int8 / float8_e4m3fn cache."""
    cache = PagedKVCache(k_cache=k_cache, v_cache=v_cache, page_table=page_table,
                         seq_lens=seq_lens, page_size=int(page_size))
    if (k_scale is None) != (v_scale is None):
        raise ValueError("k_scale and v_scale must be given together")
    scales = None if k_scale is None else {"k": k_scale, "v": v_scale}
    config = None if int(split_k) == 0 else {"split_k": int(split_k)}
    return paged_decode_attention_multi(q, cache, softmax_scale=softmax_scale, config=config, scales=scales)


@paged_decode_multi.register_fake
def _paged_decode_multi_fake(q, k_cache, v_cache, page_table, seq_lens, page_size, softmax_scale, split_k,
                             k_scale=None, v_scale=None):
    torch._check(q.dim() == 4, lambda: f"q must be 4-D [batch, q_len, heads, head_dim], got {q.dim()}")
    torch._check(q.shape[0] == seq_lens.shape[0], lambda: "q batch must match seq_lens")
    torch._check(q.shape[3] == k_cache.shape[3], lambda: "q head_dim must match cache")
    torch._check(q.shape[2] % k_cache.shape[2] == 0, lambda: "heads must be divisible by KV heads")
    return q.new_empty(q.shape)


def ops_available() -> bool:
    """True when the custom ops are registered in this process."""
    return all(hasattr(torch.ops.flashattn_tile, name)
               for name in ("paged_decode", "prefill_varlen", "paged_decode_quant", "prefill_paged",
                            "paged_decode_multi"))
