"""GPU parity of multi-token (speculative) paged decode, ``q_len > 1``.

Token t of sequence b attends keys j <= seq_lens[b] - q_len + t of the paged
cache (bottom-right causal).  The oracle is ``ref_attention_paged_prefill``
with q_len-token chunks (gather through the table, then the fp32 varlen
restatement of flashattn_tile/reference.py); tolerance 2e-3 on the kernel's
result before its final rounding (tests/_parity.py).  Pools are permuted and
the slots past each sequence end are poisoned.  Quantised caches compare with
the oracle on the cache dequantised to q.dtype.
"""

from __future__ import annotations

import pytest
import torch

from _parity import assert_parity, force_decode_knobs, make_paged
from flashattntile_amd import PagedKVCache, paged_decode_attention, paged_decode_attention_fp8
from flashattntile_amd.kernels.decode import paged_decode_attention_multi
from flashattntile_amd.quant import quantize_cache
from oracle import quant_ref
from oracle.reference import ref_attention_paged_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(lens, T, h, hk, d, P, dtype, seed):
    k, v, pt, sl = make_paged(lens, hk, d, P, dtype, seed=seed, device=DEV)
    g = torch.Generator().manual_seed(seed + 50)
    q = torch.randn(len(lens), T, h, d, generator=g).to(dtype).to(DEV)
    return q, PagedKVCache(k, v, pt, sl, P)


def _ref32(q, k, v, cache, scale=None):
    B, T, H, D = q.shape
    cu = [i * T for i in range(B + 1)]
    out = ref_attention_paged_prefill(q.reshape(B * T, H, D).cpu(), k.cpu(), v.cpu(), cache.page_table.cpu(),
                                      cache.seq_lens.cpu(), cu, causal=True, softmax_scale=scale, return_fp32=True)
    return out.reshape(B, T, H, D)


LENS = [40, 17, 255, 1000]


@pytest.fixture(params=[4, 8], autouse=True)
def mfma_waves(request, monkeypatch):
    """Every multi-token case on the MFMA decode with 4 and 8 waves."""
    force_decode_knobs(monkeypatch, num_warps=request.param)
    return request.param


@pytest.mark.parametrize("split_k", [1, 4, None])
@pytest.mark.parametrize("T", [2, 3, 4, 8, 16])
@pytest.mark.parametrize("h,hk", [(8, 8), (8, 2), (32, 8), (32, 1)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_multi_token_decode_matches_oracle(dtype, h, hk, T, split_k):
    label = f"multi decode {dtype} H{h}/{hk} T{T} split={split_k}"
    print(label, flush=True)
    q, cache = _case(LENS, T, h, hk, 128, 16, dtype, seed=h + hk + T)
    cfg = None if split_k is None else {"split_k": split_k}
    out = paged_decode_attention_multi(q, cache, config=cfg)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == dtype
    assert_parity(out, _ref32(q, cache.k_cache, cache.v_cache, cache), label=label)


@pytest.mark.parametrize("P", [16, 32, 64])
@pytest.mark.parametrize("T", [2, 5, 32])
def test_multi_token_decode_d64_and_page_sizes(P, T):
    label = f"multi decode D64 P{P} T{T}"
    print(label, flush=True)
    q, cache = _case([33, 64, 300], T, 16, 4, 64, P, torch.float16, seed=P + T)
    out = paged_decode_attention_multi(q, cache, softmax_scale=0.11, config={"split_k": 3})
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache.k_cache, cache.v_cache, cache, scale=0.11), label=label)


@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
@pytest.mark.parametrize("T", [2, 4])
def test_multi_token_decode_quantised(mode, T):
    label = f"multi decode {mode} T{T}"
    print(label, flush=True)
    q, cache = _case(LENS, T, 32, 8, 128, 16, torch.float16, seed=T)
    qc, scales = quantize_cache(cache, mode=mode)
    out = paged_decode_attention_multi(q, qc, scales=scales, config={"split_k": 2})
    torch.cuda.synchronize()
    k = quant_ref.dequantize_pages(qc.k_cache, scales.k, torch.float16)
    v = quant_ref.dequantize_pages(qc.v_cache, scales.v, torch.float16)
    assert_parity(out, _ref32(q, k, v, cache), label=label)


def test_one_token_equals_single_query_decode():
    """q_len = 1 through the multi-token entry is the single-query decode."""
    q, cache = _case(LENS, 1, 32, 8, 128, 16, torch.bfloat16, seed=3)
    a = paged_decode_attention_multi(q, cache, config={"split_k": 2})
    b = paged_decode_attention(q[:, 0].contiguous(), cache, config={"split_k": 2})
    torch.cuda.synchronize()
    assert torch.equal(a[:, 0], b)
    qc, scales = quantize_cache(cache, mode="int8")
    a8 = paged_decode_attention_multi(q, qc, scales=scales)
    b8 = paged_decode_attention_fp8(q[:, 0].contiguous(), qc, scales)
    torch.cuda.synchronize()
    assert torch.equal(a8[:, 0], b8)


def test_multi_token_rows_with_no_visible_key_in_a_block():
    """Short last partitions: with split 8 on 40 keys and T = 16, the last
    block of some partitions holds keys no early token may see; those rows
    must stay finite and exact."""
    q, cache = _case([40, 16, 47], 16, 8, 2, 128, 16, torch.float16, seed=11)
    out = paged_decode_attention_multi(q, cache, config={"split_k": 8, "pages_per_split": 1})
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert_parity(out, _ref32(q, cache.k_cache, cache.v_cache, cache), label="multi decode masked blocks")


def test_multi_token_validation():
    q, cache = _case([3, 40], 4, 8, 2, 128, 16, torch.float16, seed=1)
    with pytest.raises(ValueError, match="new tokens"):
        paged_decode_attention_multi(q, cache)
    q2, cache2 = _case([8, 40], 4, 8, 2, 128, 16, torch.float16, seed=1)
    with pytest.raises(ValueError, match="scales"):
        paged_decode_attention_multi(q2, cache2, scales={"k": None, "v": None})
    with pytest.raises(ValueError, match="batch, q_len"):
        paged_decode_attention_multi(q2[:, 0], cache2)


def test_multi_token_op_compile_and_backend_route():
    """flashattn_tile::paged_decode_multi (eager, inside torch.compile, and
    with an int8 cache) and the backend's 4-D decode route give exactly the
    function's result."""
    from flashattntile_amd.backend import AttentionMetadata, FlashAttnTileBackend

    print("multi decode op / compile / backend", flush=True)
    q, cache = _case(LENS, 3, 32, 8, 128, 16, torch.float16, seed=77)
    want = paged_decode_attention_multi(q, cache, softmax_scale=0.09, config={"split_k": 2})
    args = (cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, 16, 0.09, 2)
    got = torch.ops.flashattn_tile.paged_decode_multi(q, *args)

    def fn(x):
        return torch.ops.flashattn_tile.paged_decode_multi(x, *args)

    got_c = torch.compile(fn, fullgraph=True, backend="eager")(q)
    backend = FlashAttnTileBackend(num_heads=32, num_kv_heads=8, head_dim=128, page_size=16)
    got_b = backend.forward(q, cache, AttentionMetadata(softmax_scale=0.09))
    want_b = paged_decode_attention_multi(q, cache, softmax_scale=0.09)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(got_c, want) and torch.equal(got_b, want_b)
    qc, sc = quantize_cache(cache, "int8")
    want_q = paged_decode_attention_multi(q, qc, softmax_scale=0.09, config={"split_k": 2}, scales=sc)
    got_q = torch.ops.flashattn_tile.paged_decode_multi(q, qc.k_cache, qc.v_cache, qc.page_table, qc.seq_lens, 16,
                                                        0.09, 2, sc.k, sc.v)
    torch.cuda.synchronize()
    assert torch.equal(got_q, want_q)
