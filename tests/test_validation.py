"""Host-side input validation of the kernel wrappers.

The exception types and message fragments are the reference's contract,
matched by callers: decode ``flashattn_tile/kernels/decode.py:486-522,
578, 664-684``, prefill ``kernels/prefill.py:180-233, 270-274`` and the
oracle's per-sequence checks ``reference.py:113-119``.  Every case is
rejected before any device work, so the suite runs on the CPU: each one
builds a small valid problem, breaks one thing about it, and names the
fragment the error must carry.
"""

from __future__ import annotations

import pytest
import torch

from flashattntile_amd.kernels.decode import paged_decode_attention, paged_decode_attention_fp8
from flashattntile_amd.kernels.prefill import paged_prefill_attention, prefill_attention
from flashattntile_amd.paging import PagedKVCache

HEADS, KV_HEADS, DIM, PAGE = 6, 3, 32, 8
LENS = [3, 11, 6]


def _filled_cache(lens=LENS, page=PAGE, dtype=torch.float32, seed=5) -> PagedKVCache:
    """A cache whose pages are laid out back to front (last page first), so a
    test that reads them proves the table is followed."""
    g = torch.Generator().manual_seed(seed)
    per = [-(-n // page) for n in lens]
    pages = sum(per) + 1
    k = torch.randn(pages, page, KV_HEADS, DIM, generator=g).to(dtype)
    v = torch.randn(pages, page, KV_HEADS, DIM, generator=g).to(dtype)
    table = torch.zeros(len(lens), max(per), dtype=torch.int32)
    nxt = pages - 1
    for b, n in enumerate(per):
        for i in range(n):
            table[b, i] = nxt
            nxt -= 1
    return PagedKVCache(k, v, table, torch.tensor(lens, dtype=torch.int32), page)


def _query(batch=len(LENS), heads=HEADS, dim=DIM):
    return torch.randn(batch, heads, dim)


# (case id, call, exception, message fragment)
DECODE_CASES = [
    ("batch mismatch", lambda c: paged_decode_attention(_query(batch=4), c), ValueError, "q batch"),
    ("heads not a multiple of kv heads", lambda c: paged_decode_attention(_query(heads=7), c), ValueError,
     "divisible"),
    ("head_dim mismatch", lambda c: paged_decode_attention(_query(dim=16), c), ValueError, "head_dim"),
    ("2-D query", lambda c: paged_decode_attention(torch.randn(3, DIM), c), ValueError, r"\[batch, heads"),
    ("split_k zero", lambda c: paged_decode_attention(_query(), c, config={"split_k": 0}), ValueError,
     "split_k must be a positive"),
    ("split_k too large", lambda c: paged_decode_attention(_query(), c, config={"split_k": 100}), ValueError,
     "split_k must be <= 64"),
    ("foreign config key", lambda c: paged_decode_attention(_query(), c, config={"BLOCK_M": 32}), ValueError,
     "unknown decode config keys"),
    ("num_warps not a power of two", lambda c: paged_decode_attention(_query(), c, config={"num_warps": 3}),
     ValueError, "num_warps"),
    ("integer query", lambda c: paged_decode_attention(_query().to(torch.int32), c), ValueError,
     "floating point"),
    ("not a cache", lambda c: paged_decode_attention(_query(), (c.k_cache, c.v_cache)), TypeError,
     "PagedKVCache"),
]


@pytest.mark.parametrize("call,exc,fragment", [c[1:] for c in DECODE_CASES], ids=[c[0] for c in DECODE_CASES])
def test_decode_rejects(call, exc, fragment):
    with pytest.raises(exc, match=fragment):
        call(_filled_cache())


@pytest.mark.parametrize("empty", [0, 2])
def test_decode_rejects_a_sequence_without_tokens(empty):
    cache = _filled_cache()
    cache.seq_lens[empty] = 0
    with pytest.raises(ValueError, match="at least one cached token"):
        paged_decode_attention(_query(), cache)


@pytest.mark.parametrize("bad_id,fragment", [(-3, "negative page id"), (99, "references page 99")])
def test_decode_reports_bad_page_ids(bad_id, fragment):
    cache = _filled_cache()
    cache.page_table[1, 1] = bad_id  # sequence 1 (11 tokens) uses two pages
    with pytest.raises(AssertionError, match=fragment):
        paged_decode_attention(_query(), cache)


def test_quantised_decode_rejects_unquantised_caches_and_bad_scales():
    cache = _filled_cache()
    ones = torch.ones(cache.num_pages, KV_HEADS)
    with pytest.raises(ValueError, match="int8/float8"):
        paged_decode_attention_fp8(_query().half(), cache, {"k": ones, "v": ones})
    cache.k_cache = cache.k_cache.clamp(-4, 4).mul(30).to(torch.int8)
    cache.v_cache = cache.v_cache.clamp(-4, 4).mul(30).to(torch.int8)
    short = torch.ones(cache.num_pages - 1, KV_HEADS)
    with pytest.raises(ValueError, match="scales must have shape"):
        paged_decode_attention_fp8(_query().half(), cache, {"k": short, "v": short})


def _packed(q_lens, k_lens=None, heads=HEADS, kv_heads=KV_HEADS, dim=DIM, seed=9):
    k_lens = q_lens if k_lens is None else k_lens
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(sum(q_lens), heads, dim, generator=g)
    k = torch.randn(sum(k_lens), kv_heads, dim, generator=g)
    v = torch.randn(sum(k_lens), kv_heads, dim, generator=g)

    def offsets(lens):
        return torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)

    return q, k, v, offsets(q_lens), offsets(k_lens)


def _i32(values):
    return torch.tensor(values, dtype=torch.int32)


def _prefill(q, k, v, cq, ck, causal=True, **kw):
    mq = max(int(x) for x in (cq[1:] - cq[:-1]).tolist()) if cq.numel() > 1 else 1
    mk = max(int(x) for x in (ck[1:] - ck[:-1]).tolist()) if ck.numel() > 1 else 1
    return prefill_attention(q, k, v, cq, ck, kw.pop("mq", max(mq, 1)), kw.pop("mk", max(mk, 1)), causal=causal,
                             **kw)


PREFILL_CASES = [
    ("BLOCK_N not a power of two", lambda p: _prefill(*p, config={"BLOCK_N": 24}), "power of two"),
    ("foreign config key", lambda p: _prefill(*p, config={"split_k": 2}), "unknown prefill config keys"),
    ("num_stages zero", lambda p: _prefill(*p, config={"num_stages": 0}), "num_stages"),
    ("q offsets end early", lambda p: _prefill(p[0], p[1], p[2], _i32([0, 4, 12, 16]), p[4]),
     "cu_seqlens_q\\[-1\\] must equal q.shape"),
    ("k offsets end late", lambda p: _prefill(p[0], p[1], p[2], p[3], _i32([0, 4, 12, 25])),
     "cu_seqlens_k\\[-1\\] must equal k.shape"),
    ("offset counts differ", lambda p: _prefill(p[0], p[1], p[2], _i32([0, 17]), p[4]), "same batch dimension"),
    ("int64 offsets", lambda p: _prefill(p[0], p[1], p[2], p[3].long(), p[4].long()), "must be int32"),
    ("offsets not starting at 0", lambda p: _prefill(p[0], p[1], p[2], p[3] + 1, p[4] + 1),
     "must start at 0"),
    ("decreasing q offsets", lambda p: prefill_attention(p[0], p[1], p[2], _i32([0, 12, 5, 17]), p[4], 12, 8,
                                                         causal=False), "cu_seqlens_q must be non-decreasing"),
    ("k and v shapes differ", lambda p: _prefill(p[0], p[1], p[2][:-1], p[3], p[4]), "k shape"),
    ("mixed dtypes", lambda p: _prefill(p[0].half(), p[1], p[2], p[3], p[4]), "dtype mismatch"),
    ("4-D q", lambda p: _prefill(p[0].unsqueeze(0), p[1], p[2], p[3], p[4]), "must be 3-D"),
    ("max_seqlen_k zero", lambda p: _prefill(*p, mk=0), "max_seqlen_k must be positive"),
    ("max_seqlen_q below the longest", lambda p: _prefill(*p, mq=5), "smaller than the longest query"),
]


@pytest.mark.parametrize("call,fragment", [c[1:] for c in PREFILL_CASES], ids=[c[0] for c in PREFILL_CASES])
def test_prefill_rejects(call, fragment):
    with pytest.raises(ValueError, match=fragment):
        call(_packed([4, 8, 5]))


def test_prefill_rejects_decreasing_key_offsets():
    q, k, v, cq, _ = _packed([2, 2, 2])
    ck = torch.tensor([0, 4, 3, 6], dtype=torch.int32)
    with pytest.raises(ValueError, match="cu_seqlens_k must be non-decreasing"):
        prefill_attention(q, k, v, cq, ck, 2, 4, causal=False)


def test_causal_prefill_needs_at_least_as_many_keys_as_queries():
    q, k, v, cq, ck = _packed([6, 2], k_lens=[5, 3])
    with pytest.raises(ValueError, match="kv_len >= q_len"):
        prefill_attention(q, k, v, cq, ck, 6, 5, causal=True)
    prefill_attention_ok = _packed([6, 2], k_lens=[7, 3])
    with pytest.raises(RuntimeError, match="ROCm device"):  # valid: reaches the device check
        _prefill(*prefill_attention_ok)


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_rejects_queries_without_keys(causal):
    """A sequence with queries and no keys has nothing to attend: causal
    batches fail the bottom-right check first (the reference wrapper's own,
    kernels/prefill.py:227-229); non-causal ones get the oracle's message
    (reference.py:115-116) instead of zeros from the kernel."""
    q, k, v, cq, ck = _packed([3, 5, 2], k_lens=[4, 0, 6])
    fragment = "kv_len >= q_len" if causal else "sequence 1 has 5 queries but no keys"
    with pytest.raises(ValueError, match=fragment):
        prefill_attention(q, k, v, cq, ck, 5, 6, causal=causal)


def test_prefill_accepts_sequences_without_queries():
    """q_len = 0 with or without keys is a legal serving batch entry; it gets
    through validation to the device check."""
    q, k, v, cq, ck = _packed([3, 0, 2, 0], k_lens=[3, 0, 4, 7])
    with pytest.raises(RuntimeError, match="ROCm device"):
        prefill_attention(q, k, v, cq, ck, 3, 7, causal=True)


@pytest.mark.parametrize("causal", [True, False])
def test_paged_prefill_rejects_queries_without_keys(causal):
    cache = _filled_cache(lens=[9, 0, 4])
    q = torch.randn(9, HEADS, DIM)
    cq = torch.tensor([0, 3, 7, 9], dtype=torch.int32)  # sequence 1: 4 queries, no keys
    fragment = "kv_len >= q_len" if causal else "sequence 1 has 4 queries but no keys"
    with pytest.raises(ValueError, match=fragment):
        paged_prefill_attention(q, cache, cq, 4, causal=causal)
