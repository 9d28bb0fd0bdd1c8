"""fp32 CPU restatement of the FlashAttnTile reference attention -- TEST INFRASTRUCTURE.

This module is the parity oracle and the CPU baseline.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it, and only as the checker / the timed CPU baseline; the product
package (``flashattntile_amd``) never imports it and has no CPU fallback.

It restates ``flashattn_tile/reference.py`` (read, not run): the score matrix
is materialised in fp32, softmaxed in fp32, and the result is cast back to
the input dtype only at the end.

Functions and what pins them (tests/test_oracle.py, tests/test_quant.py):

``ref_attention_varlen``  (reference.py:50-142)
    validation order and messages of reference.py:78-121; causal masking is
    bottom-right aligned, key j visible to query i iff j <= i + kv_len - q_len
    (reference.py:19-22, 132-137).  Pinned by an independent pure-Python
    loop on tiny inputs, by torch's SDPA math routine on GQA-expanded K/V, by
    closed forms (q = 0 -> mean of the visible values; one key -> that value;
    first causal row -> v[0]) and by the GQA head-mapping KAT [1, 1, 2, 2]
    (tests/test_paging.py:116-136 of the reference).
``ref_attention_paged``  (reference.py:145-194)
    gathers pages through the table, then varlen with one query per
    sequence.  Pinned by page-table permutation invariance and by equality
    with varlen on the contiguous gather.
``ref_attention_dense``  (reference.py:197-219)
    token-major transpose wrapper; pinned against per-batch varlen.
``ref_attention_paged_prefill``  (no reference counterpart: the chunked
    prefill the reference's backend lacks, backend.py:158-162)
    gathers each sequence's seq_lens[b] keys through the table (as
    reference.py:177-186), then varlen with the packed queries.  Pinned by
    equality with ref_attention_paged when every chunk is one query, with
    ref_attention_varlen when the pool holds the packed K/V in order, by
    page-table permutation invariance, and by the chunking identity: a causal
    sequence prefilled as two chunks gives the rows of the one-shot prefill.
``lse_partials`` / ``lse_merge``  (docs/kernel_design.md:84-94,
    kernels/decode.py:316-356)
    split-K restatement used to check the merge algebra: merging any
    partition of the keys equals the unsplit result; empty partitions are
    neutral.
"""

from __future__ import annotations

import math

import torch

__all__ = [
    "ref_attention_varlen",
    "ref_attention_paged",
    "ref_attention_dense",
    "gather_pages",
    "lse_partials",
    "lse_merge",
]


def _offsets(cu_seqlens, name: str) -> list[int]:
    """``reference.py:34-47``: 1-D, >= 2 entries, starts at 0, non-decreasing."""
    if isinstance(cu_seqlens, torch.Tensor):
        if cu_seqlens.dim() != 1:
            raise ValueError(f"{name} must be 1-D, got shape {tuple(cu_seqlens.shape)}")
        vals = [int(x) for x in cu_seqlens.detach().cpu().tolist()]
    else:
        vals = [int(x) for x in cu_seqlens]
    if len(vals) < 2:
        raise ValueError(f"{name} must have at least 2 entries (batch + 1)")
    if vals[0] != 0:
        raise ValueError(f"{name} must start at 0, got {vals[0]}")
    for a, b in zip(vals, vals[1:]):
        if b < a:
            raise ValueError(f"{name} must be non-decreasing, got {vals}")
    return vals


def _attend_one(qb: torch.Tensor, kb: torch.Tensor, vb: torch.Tensor, group: int, causal: bool,
                scale: float) -> torch.Tensor:
    """fp32 attention of one sequence: q [Lq, H, D], k/v [Lk, Hkv, D] -> [Lq, H, D]."""
    q_len, kv_len = qb.shape[0], kb.shape[0]
    kf = kb.float().repeat_interleave(group, dim=1)  # [Lk, H, D]
    vf = vb.float().repeat_interleave(group, dim=1)
    qf = qb.float()
    # scores[h, i, j] = scale * q[i, h] . k[j, h]
    scores = torch.bmm(qf.transpose(0, 1), kf.permute(1, 2, 0).contiguous()) * scale
    if causal:
        shift = kv_len - q_len
        rows = torch.arange(q_len).unsqueeze(1) + shift
        cols = torch.arange(kv_len).unsqueeze(0)
        scores = scores.masked_fill((cols > rows).unsqueeze(0), float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    return torch.bmm(probs, vf.transpose(0, 1).contiguous()).transpose(0, 1)  # [Lq, H, D]


def ref_attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, causal: bool = True,
                         softmax_scale: float | None = None, return_fp32: bool = False) -> torch.Tensor:
    """Packed varlen attention; ``q [Tq, H, D]``, ``k/v [Tk, Hkv, D]``.

    Returns ``q``'s dtype (the reference's output) or, with
    ``return_fp32=True``, the fp32 result before that final cast.
    """
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be 3-D [tokens, heads, head_dim]")
    if q.shape[-1] != k.shape[-1] or k.shape != v.shape:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(f"dtype mismatch: q {q.dtype}, k {k.dtype}, v {v.dtype}")
    if not q.is_floating_point():
        raise ValueError(f"expected floating point inputs, got {q.dtype}")
    if q.device != k.device or k.device != v.device:
        raise ValueError("q, k, v must live on the same device")
    if q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("the last dimension of q, k, v must be contiguous")
    heads, kv_heads = q.shape[1], k.shape[1]
    if heads % kv_heads != 0:
        raise ValueError(f"num_heads ({heads}) must be divisible by num_kv_heads ({kv_heads})")
    group = heads // kv_heads
    cu_q = _offsets(cu_seqlens_q, "cu_seqlens_q")
    cu_k = _offsets(cu_seqlens_k, "cu_seqlens_k")
    if len(cu_q) != len(cu_k):
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have the same length")
    if cu_q[-1] != q.shape[0]:
        raise ValueError(f"cu_seqlens_q ends at {cu_q[-1]} but q has {q.shape[0]} tokens")
    if cu_k[-1] != k.shape[0]:
        raise ValueError(f"cu_seqlens_k ends at {cu_k[-1]} but k has {k.shape[0]} tokens")
    scale = float(softmax_scale) if softmax_scale is not None else q.shape[-1] ** -0.5

    qc, kc, vc = q.detach().cpu(), k.detach().cpu(), v.detach().cpu()
    out = torch.zeros(q.shape, dtype=torch.float32)
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        q_len, kv_len = qe - qs, ke - ks
        if q_len == 0:
            continue
        if kv_len == 0:
            raise ValueError(f"sequence {b} has {q_len} queries but no keys")
        if causal and kv_len < q_len:
            raise ValueError(f"causal bottom-right alignment requires kv_len >= q_len (sequence {b}: "
                             f"{kv_len} < {q_len})")
        out[qs:qe] = _attend_one(qc[qs:qe], kc[ks:ke], vc[ks:ke], group, causal, scale)
    if return_fp32:
        return out
    return out.to(q.dtype)


def gather_pages(k_cache, v_cache, page_table, seq_lens) -> tuple[list[torch.Tensor], list[torch.Tensor]]:
    """Per-sequence contiguous K/V through the page table (own restatement of
    ``paging.gather_paged``, ``paging.py:213-256``)."""
    page_size = int(k_cache.shape[1])
    table = page_table.detach().cpu().long()
    lens = [int(x) for x in seq_lens.detach().cpu().tolist()]
    kc, vc = k_cache.detach().cpu(), v_cache.detach().cpu()
    ks, vs = [], []
    for b, n in enumerate(lens):
        pages = table[b, : math.ceil(n / page_size)] if n > 0 else table[b, :0]
        if n > 0 and (int(pages.min()) < 0 or int(pages.max()) >= kc.shape[0]):
            raise ValueError(f"sequence {b} page id outside [0, {kc.shape[0]})")
        ks.append(kc[pages].reshape(-1, kc.shape[2], kc.shape[3])[:n])
        vs.append(vc[pages].reshape(-1, vc.shape[2], vc.shape[3])[:n])
    return ks, vs


def ref_attention_paged(q, k_cache, v_cache, page_table, seq_lens, causal: bool = True,
                        softmax_scale: float | None = None, return_fp32: bool = False) -> torch.Tensor:
    """One decode query per sequence over a paged cache (``reference.py:145-194``).

    Quantised caches must be dequantised first (``oracle.quant_ref``).
    """
    if q.dim() != 3:
        raise ValueError(f"q must be [batch, heads, head_dim], got {tuple(q.shape)}")
    if q.shape[0] != seq_lens.shape[0]:
        raise ValueError(f"q batch {q.shape[0]} != seq_lens batch {seq_lens.shape[0]}")
    if q.shape[-1] != k_cache.shape[-1]:
        raise ValueError(f"q head_dim {q.shape[-1]} != cache head_dim {k_cache.shape[-1]}")
    if q.shape[1] % k_cache.shape[2] != 0:
        raise ValueError(f"num_heads {q.shape[1]} not divisible by num_kv_heads {k_cache.shape[2]}")
    if not k_cache.is_floating_point():
        raise ValueError(f"reference attention needs a dequantized float cache, got {k_cache.dtype}; "
                         "dequantize it first")
    if q.dtype != k_cache.dtype:
        raise ValueError(f"q dtype {q.dtype} != cache dtype {k_cache.dtype}")
    ks, vs = gather_pages(k_cache, v_cache, page_table, seq_lens)
    lens = [t.shape[0] for t in ks]
    if len(lens) == 0 or sum(lens) == 0:
        raise ValueError("ref_attention_paged requires at least one cached token")
    k_packed = torch.cat(ks, dim=0)
    v_packed = torch.cat(vs, dim=0)
    cu_k = [0]
    for n in lens:
        cu_k.append(cu_k[-1] + n)
    cu_q = list(range(len(lens) + 1))
    return ref_attention_varlen(q.detach().cpu(), k_packed, v_packed, cu_q, cu_k, causal=causal,
                                softmax_scale=softmax_scale, return_fp32=return_fp32)


def ref_attention_paged_prefill(q, k_cache, v_cache, page_table, seq_lens, cu_seqlens_q, causal: bool = True,
                                softmax_scale: float | None = None, return_fp32: bool = False) -> torch.Tensor:
    """Packed queries ``q [total_q, H, D]`` (offsets ``cu_seqlens_q``) against
    the first ``seq_lens[b]`` keys of each sequence in a paged cache."""
    if q.dim() != 3:
        raise ValueError(f"q must be [tokens, heads, head_dim], got {tuple(q.shape)}")
    if not k_cache.is_floating_point():
        raise ValueError(f"reference attention needs a dequantized float cache, got {k_cache.dtype}; "
                         "dequantize it first")
    ks, vs = gather_pages(k_cache, v_cache, page_table, seq_lens)
    cu_k = [0]
    for t in ks:
        cu_k.append(cu_k[-1] + t.shape[0])
    k_packed = torch.cat(ks, dim=0)
    v_packed = torch.cat(vs, dim=0)
    return ref_attention_varlen(q.detach().cpu(), k_packed, v_packed, cu_seqlens_q, cu_k, causal=causal,
                                softmax_scale=softmax_scale, return_fp32=return_fp32)


def ref_attention_dense(q, k, v, causal: bool = True, softmax_scale: float | None = None) -> torch.Tensor:
    """``[B, H, L, D]`` wrapper over varlen (``reference.py:197-219``)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D [batch, heads, seq, head_dim]")
    batch, heads, q_len, d = q.shape
    kv_len = k.shape[2]
    qt = q.transpose(1, 2).reshape(batch * q_len, heads, d).contiguous()
    kt = k.transpose(1, 2).reshape(batch * kv_len, k.shape[1], d).contiguous()
    vt = v.transpose(1, 2).reshape(batch * kv_len, v.shape[1], d).contiguous()
    cu_q = [i * q_len for i in range(batch + 1)]
    cu_k = [i * kv_len for i in range(batch + 1)]
    out = ref_attention_varlen(qt, kt, vt, cu_q, cu_k, causal=causal, softmax_scale=softmax_scale)
    return out.reshape(batch, q_len, heads, d).transpose(1, 2).contiguous()


def lse_partials(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bounds: list[tuple[int, int]],
                 scale: float) -> list[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
    """Split-K partials of one decode query: q [H, D], k/v [L, H, D] (already
    GQA-expanded).  For each key range returns (acc [H, D], m [H], l [H]) with
    m = max score, l = sum exp(s - m), acc = sum exp(s - m) v; an empty range
    gives (0, -inf, 0) (docs/kernel_design.md:92-94)."""
    parts = []
    qf, kf, vf = q.float(), k.float(), v.float()
    for lo, hi in bounds:
        if hi <= lo:
            parts.append((torch.zeros_like(qf), torch.full((qf.shape[0],), float("-inf")),
                          torch.zeros(qf.shape[0])))
            continue
        s = torch.einsum("hd,lhd->hl", qf, kf[lo:hi]) * scale
        m = s.max(dim=1).values
        p = torch.exp(s - m[:, None])
        parts.append((torch.einsum("hl,lhd->hd", p, vf[lo:hi]), m, p.sum(dim=1)))
    return parts


def lse_merge(parts) -> torch.Tensor:
    """``m* = max m_s; w_s = exp(m_s - m*); o = sum acc_s w_s / sum l_s w_s``."""
    m_all = torch.stack([m for _, m, _ in parts])  # [S, H]
    m_star = m_all.max(dim=0).values
    num = 0
    den = 0
    for acc, m, l in parts:
        w = torch.where(torch.isinf(m), torch.zeros_like(m), torch.exp(m - m_star))
        num = num + acc * w[:, None]
        den = den + l * w
    return num / den[:, None]
