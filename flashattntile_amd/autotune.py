"""Analytic work accounting and the MI355X launch heuristics.

The FLOP and byte formulas are the reference's roofline numerators
(``flashattn_tile/autotune.py:31-106``) so achieved-throughput figures are
comparable:

* ``flops = 4 * B * H * D * pairs`` (QK^T and PV, 2 FLOP per MAC; softmax
  excluded), ``pairs = q*kv`` or, causal bottom-right,
  ``q*(kv - q) + q*(q + 1)/2``;
* decode bytes = q + K + V + o; prefill bytes = q + k + v + o.

The Triton knob search of the reference (BLOCK_M/N, num_warps, num_stages and
its JSON store) has no meaning for the HIP kernels.  What does matter on
MI355X is how many workgroups a decode launch puts on the 256 CUs, so the
split-K count is derived from the shape and the CU count instead
(:func:`decode_split_k`).
"""

from __future__ import annotations

import math

__all__ = [
    "flops_attention",
    "flops_attention_varlen",
    "bytes_attention",
    "bytes_decode_paged",
    "arithmetic_intensity",
    "decode_split_k",
    "decode_partition",
    "decode_heads_per_workgroup",
    "MI355X_CUS",
]

MI355X_CUS = 256


def _causal_pairs(q_len: int, kv_len: int) -> int:
    """Query/key pairs visible under bottom-right causal alignment."""
    if q_len <= 0 or kv_len <= 0:
        return 0
    if kv_len < q_len:
        raise ValueError("causal accounting requires kv_len >= q_len")
    return q_len * (kv_len - q_len) + q_len * (q_len + 1) // 2


def flops_attention(num_heads: int, head_dim: int, q_len: int, kv_len: int,
                    causal: bool = False, batch: int = 1) -> int:
    """``4 * batch * H * D * pairs`` (``autotune.py:40-55``)."""
    pairs = _causal_pairs(q_len, kv_len) if causal else q_len * kv_len
    return int(4 * batch * num_heads * head_dim * pairs)


def flops_attention_varlen(num_heads: int, head_dim: int, q_lens, kv_lens, causal: bool = False) -> int:
    """Sum of :func:`flops_attention` over a ragged batch (``autotune.py:58-73``)."""
    if len(q_lens) != len(kv_lens):
        raise ValueError("q_lens and kv_lens must have the same length")
    return int(sum(flops_attention(num_heads, head_dim, int(q), int(k), causal=causal)
                   for q, k in zip(q_lens, kv_lens)))


def bytes_attention(mode: str, batch: int, q_len: int, kv_len: int, num_heads: int,
                    num_kv_heads: int, head_dim: int, elem_bytes: int = 2) -> int:
    """HBM bytes of the fused kernel: q + K + V + o (``autotune.py:76-106``)."""
    if mode == "decode":
        if q_len != 1:
            raise ValueError("decode accounting assumes q_len == 1")
        q_bytes = batch * num_heads * head_dim * elem_bytes
        kv_bytes = batch * kv_len * num_kv_heads * head_dim * 2 * elem_bytes
        return int(2 * q_bytes + kv_bytes)
    if mode == "prefill":
        q_bytes = batch * q_len * num_heads * head_dim * elem_bytes
        kv_bytes = batch * kv_len * num_kv_heads * head_dim * 2 * elem_bytes
        return int(2 * q_bytes + kv_bytes)
    raise ValueError(f"unknown mode {mode!r}")


def bytes_decode_paged(seq_lens, num_heads: int, num_kv_heads: int, head_dim: int,
                       q_elem_bytes: int = 2, kv_elem_bytes: int = 2, page_size: int | None = None,
                       quantized: bool = False) -> int:
    """Decode bytes for a ragged batch: q + o + sum_b ctx_b * (K + V).

    For a quantised cache the fp32 scales of every touched (page, KV head) are
    added (2 * 4 bytes each), the scale term of ``kv_bytes_per_token``
    (``quant.py:205-208``).  The page table is excluded, as in the reference.
    """
    lens = [int(x) for x in seq_lens]
    batch = len(lens)
    qo = 2 * batch * num_heads * head_dim * q_elem_bytes
    kv = sum(lens) * num_kv_heads * head_dim * 2 * kv_elem_bytes
    scales = 0
    if quantized:
        if page_size is None:
            raise ValueError("quantized accounting needs page_size")
        pages = sum(math.ceil(n / page_size) for n in lens)
        scales = pages * num_kv_heads * 2 * 4
    return int(qo + kv + scales)


def arithmetic_intensity(flops: float, nbytes: float) -> float:
    if nbytes <= 0:
        return float("inf")
    return float(flops) / float(nbytes)


def decode_split_k(batch: int, num_heads: int, num_kv_heads: int, max_pages: int,
                   num_cus: int = MI355X_CUS, min_pages_per_split: int = 8, max_split: int = 16) -> int:
    """Split-K partitions for a decode launch on MI355X.

    One workgroup handles one GQA group of up to 8 query heads for one
    partition, so a launch has ``batch * groups * split`` workgroups.  The
    rule asks for about one workgroup per CU, never fewer than
    ``min_pages_per_split`` pages per partition (shorter partitions spend more
    on the merge than they gain) and at most ``max_split`` partitions.  It was
    fitted on an MI355X sweep of B in {1, 8, 32, 128} x ctx in {128, 1024,
    4096, 16384} (32/8 heads, D128, page 16, fp16), where it picks the fastest
    measured split or one within 2 % of it.  It needs only host-known sizes,
    so it never synchronises with the device.
    """
    group = max(1, num_heads // max(1, num_kv_heads))
    heads_per_wg = 8 if group >= 8 else 4
    groups = num_kv_heads * math.ceil(group / heads_per_wg)
    base = max(1, batch * groups)
    split = math.ceil(num_cus / base)
    split = min(split, max_split, max(1, max_pages // min_pages_per_split))
    return int(max(1, split))


def decode_heads_per_workgroup(group: int, quantized: bool = False) -> int:
    """Query heads one decode workgroup serves: the MFMA decode (every int8 /
    fp8 cache, and fp16/bf16 caches with group >= 8) takes up to 32, the VALU
    decode (fp16/bf16, group < 8) 4."""
    if quantized or group >= 8:
        return 32
    return 4


def decode_partition(batch: int, num_heads: int, num_kv_heads: int, max_pages: int, total_pages: int,
                     num_cus: int = MI355X_CUS, min_pages_per_split: int = 8,
                     max_split: int = 16, quantized: bool = False, q_len: int = 1) -> tuple[int, int]:
    """``(split_k, pages_per_split)`` for a possibly ragged batch on MI355X.

    Every partition holds the same number of pages and split_k covers the
    longest sequence.  A uniform batch (``batch * max_pages`` below twice
    ``total_pages``) is spread over about one workgroup per CU with at most
    ``max_split`` partitions -- the same launch as :func:`decode_split_k`.  A
    skewed batch gets many small partitions (about 16 workgroups per CU, up to
    64 partitions), so the long sequences are streamed by many workgroups and
    the dispatcher balances the uneven rest.  Both regimes were measured on
    MI355X (32/8 heads, D128, page 16: the B x ctx sweep and 64 log-uniform
    lengths in [16, 65536]).
    """
    group = max(1, num_heads // max(1, num_kv_heads))
    rows = group * max(1, int(q_len))  # (query head, token) rows per KV head
    heads_per_wg = 32 if q_len > 1 else decode_heads_per_workgroup(group, quantized)
    groups = num_kv_heads * math.ceil(rows / heads_per_wg)
    max_pages = max(1, int(max_pages))
    total_pages = max(1, int(total_pages))
    skewed = batch * max_pages >= 2 * total_pages
    target_wgs = 16 * num_cus if skewed else num_cus
    cap = 64 if skewed else max_split
    chunk = max(min_pages_per_split, math.ceil(total_pages * groups / target_wgs))
    split = math.ceil(max_pages / chunk)
    if split > cap:
        split = cap
        chunk = math.ceil(max_pages / split)
    return int(max(1, split)), int(chunk)
