"""GPU parity of ``FlashAttnTileBackend.forward`` on every route.

The reference checks that its backend routes decode (3-D, and
``[batch, 1, heads, head_dim]`` squeezed) and packed prefill to exactly the
oracle's result (tests/test_ops.py:111-142, backend.py:132-175).  Here each
route runs the HIP kernels on the device and is compared with the fp32
oracle within 2e-3 (tests/_parity.py):

* decode, 3-D and ``[B, 1, H, D]`` (bit-identical to each other), with the
  metadata's page table and lengths replacing the cache's;
* decode of an int8 / fp8 cache through ``kv_scales`` (oracle on the cache
  dequantised to q.dtype, the reference's dequantise-then-attend);
* packed causal prefill with ``max_seqlen_*`` given or left to the backend;
* paged prefill of a chunk whose K/V are already appended;
* multi-token decode of a ``[B, T, H, D]`` query.
"""

from __future__ import annotations

import pytest
import torch

from _parity import assert_parity, make_paged, make_query, make_varlen
from flashattntile_amd import PagedKVCache
from flashattntile_amd.backend import AttentionMetadata, FlashAttnTileBackend
from oracle import quant_ref
from oracle.reference import ref_attention_paged, ref_attention_paged_prefill, ref_attention_varlen

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, HKV, D, P = 32, 8, 128, 16


@pytest.fixture
def backend():
    return FlashAttnTileBackend(num_heads=H, num_kv_heads=HKV, head_dim=D, page_size=P)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_route_3d_and_squeezed(backend, dtype):
    print(f"backend decode {dtype}", flush=True)
    k, v, pt, sl = make_paged([700, 33, 4096], HKV, D, P, dtype, seed=1, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, P)
    q = make_query(3, H, D, dtype, seed=2, device=DEV)
    meta = AttentionMetadata(page_table=pt, seq_lens=sl, is_prefill=False, softmax_scale=0.09)
    out3 = backend.forward(q, cache, meta)
    out4 = backend.forward(q.unsqueeze(1), cache, meta)
    torch.cuda.synchronize()
    ref = ref_attention_paged(q.cpu(), k.cpu(), v.cpu(), pt.cpu(), sl.cpu(), softmax_scale=0.09, return_fp32=True)
    assert out3.shape == q.shape and out3.dtype == dtype
    assert torch.equal(out3, out4)
    assert_parity(out3, ref, label=f"backend decode {dtype}")


def test_decode_route_uses_metadata_table_and_lengths(backend):
    """``_resolve_cache`` semantics (backend.py:119-130): the metadata's page
    table / seq_lens replace the cache's own."""
    print("backend decode metadata override", flush=True)
    k, v, pt, sl = make_paged([500, 120], HKV, D, P, torch.float16, seed=3, device=DEV)
    stale = PagedKVCache(k, v, torch.zeros_like(pt), torch.ones_like(sl), P)
    q = make_query(2, H, D, torch.float16, seed=4, device=DEV)
    shorter = torch.tensor([333, 7], dtype=torch.int32, device=DEV)
    out = backend.forward(q, stale, AttentionMetadata(page_table=pt, seq_lens=shorter))
    torch.cuda.synchronize()
    ref = ref_attention_paged(q.cpu(), k.cpu(), v.cpu(), pt.cpu(), shorter.cpu(), return_fp32=True)
    assert_parity(out, ref, label="backend decode metadata override")


@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
def test_decode_route_quantised_cache(backend, mode, qdtype):
    print(f"backend quant decode {mode} {qdtype}", flush=True)
    k, v, pt, sl = make_paged([900, 64, 17], HKV, D, P, torch.float32, seed=5, device="cpu")
    qk, sk = quant_ref.quantize_pages(k, mode)
    qv, sv = quant_ref.quantize_pages(v, mode)
    cache = PagedKVCache(qk.to(DEV), qv.to(DEV), pt.to(DEV), sl.to(DEV), P)
    q = make_query(3, H, D, qdtype, seed=6, device=DEV)
    meta = AttentionMetadata(is_prefill=False, kv_scales={"k": sk.to(DEV), "v": sv.to(DEV)})
    out = backend.forward(q.unsqueeze(1), cache, meta)
    torch.cuda.synchronize()
    ref = ref_attention_paged(q.cpu(), quant_ref.dequantize_pages(qk, sk, qdtype),
                              quant_ref.dequantize_pages(qv, sv, qdtype), pt, sl, return_fp32=True)
    assert_parity(out, ref, label=f"backend quant decode {mode} {qdtype}")


@pytest.mark.parametrize("given_max", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_route_packed(backend, dtype, given_max):
    print(f"backend prefill {dtype} max given={given_max}", flush=True)
    lens = [3, 700, 129]
    q, k, v, cu = make_varlen(lens, H, HKV, D, dtype, seed=7, device=DEV)
    cache = backend.allocate_kv_cache(batch=3, max_seq_len=16, dtype=dtype, device=DEV)
    meta = AttentionMetadata(cu_seqlens_q=cu, cu_seqlens_k=cu, is_prefill=True, k=k, v=v, softmax_scale=0.1,
                             max_seqlen_q=max(lens) if given_max else None,
                             max_seqlen_k=max(lens) if given_max else None)
    out = backend.forward(q, cache, meta)
    torch.cuda.synchronize()
    ref = ref_attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), causal=True, softmax_scale=0.1,
                               return_fp32=True)
    assert out.shape == q.shape
    assert_parity(out, ref, label=f"backend prefill {dtype}")


def test_prefill_route_paged_chunk(backend):
    """A 40-token chunk after a 300-token prefix, its K/V already in the
    cache: the paged prefill route against the paged-prefill oracle."""
    print("backend paged prefill", flush=True)
    lens_k, lens_q = [340, 41], [40, 41]
    k, v, pt, sl = make_paged(lens_k, HKV, D, P, torch.float16, seed=8, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, P)
    q = torch.randn(sum(lens_q), H, D, generator=torch.Generator().manual_seed(9)).half().to(DEV)
    cu = torch.tensor([0, 40, 81], dtype=torch.int32, device=DEV)
    out = backend.forward(q, cache, AttentionMetadata(cu_seqlens_q=cu, is_prefill=True, paged_prefill=True))
    torch.cuda.synchronize()
    ref = ref_attention_paged_prefill(q.cpu(), k.cpu(), v.cpu(), pt.cpu(), sl.cpu(), cu.cpu(), causal=True,
                                      return_fp32=True)
    assert_parity(out, ref, label="backend paged prefill")


def test_multi_token_decode_route(backend):
    print("backend multi-token decode", flush=True)
    k, v, pt, sl = make_paged([300, 45], HKV, D, P, torch.bfloat16, seed=10, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, P)
    q = torch.randn(2, 3, H, D, generator=torch.Generator().manual_seed(11)).bfloat16().to(DEV)
    out = backend.forward(q, cache, AttentionMetadata())
    torch.cuda.synchronize()
    cu = torch.tensor([0, 3, 6], dtype=torch.int32)
    ref = ref_attention_paged_prefill(q.reshape(6, H, D).cpu(), k.cpu(), v.cpu(), pt.cpu(), sl.cpu(), cu,
                                      causal=True, return_fp32=True).reshape(2, 3, H, D)
    assert_parity(out, ref, label="backend multi-token decode")


def test_route_names_and_errors(backend):
    print("backend routes and errors", flush=True)
    k, v, pt, sl = make_paged([20, 30], HKV, D, P, torch.float16, seed=12, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, P)
    q = make_query(2, H, D, torch.float16, seed=13, device=DEV)
    assert backend.route(q, AttentionMetadata()) == "decode"
    assert backend.route(q, AttentionMetadata(kv_scales={})) == "decode_quant"
    assert backend.route(q.unsqueeze(1).expand(2, 2, H, D), AttentionMetadata()) == "decode_multi"
    assert backend.route(q, AttentionMetadata(is_prefill=True)) == "prefill"
    assert backend.route(q, AttentionMetadata(is_prefill=True, paged_prefill=True)) == "prefill_paged"
    with pytest.raises(ValueError, match="heads, backend expects"):
        backend.forward(q[:, :16].contiguous(), cache, AttentionMetadata())
    with pytest.raises(ValueError, match="query must be 3-D"):
        backend.forward(q[0], cache, AttentionMetadata())
    with pytest.raises(ValueError, match="requires attn_metadata.k"):
        cu = torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV)
        backend.forward(q, cache, AttentionMetadata(is_prefill=True, cu_seqlens_q=cu, cu_seqlens_k=cu))
    with pytest.raises(TypeError, match="PagedKVCache"):
        backend.forward(q, (k, v), AttentionMetadata())
