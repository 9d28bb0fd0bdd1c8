"""Operator boundary: registration, schemas, fake kernels, torch.compile,
backend surface, and the absence of any CPU fallback."""

from __future__ import annotations

import pytest
import torch

import flashattntile_amd as fat
from flashattntile_amd.backend import AttentionMetadata, FlashAttnTileBackend
from flashattntile_amd.ops import PAGED_DECODE_OP, PAGED_DECODE_QUANT_OP, PREFILL_OP, ops_available
from flashattntile_amd.paging import allocate, append_tokens

SCHEMAS = {
    "paged_decode": "flashattn_tile::paged_decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor page_table, "
                    "Tensor seq_lens, SymInt page_size, float softmax_scale, SymInt split_k) -> Tensor",
    "prefill_varlen": "flashattn_tile::prefill_varlen(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, "
                      "Tensor cu_seqlens_k, SymInt max_seqlen_q, SymInt max_seqlen_k, bool causal, "
                      "float softmax_scale) -> Tensor",
}


def _cache(batch=2, length=12, page_size=16, kv_heads=2, head_dim=8, dtype=torch.float32, device="cpu"):
    cache = allocate(batch, length, kv_heads, head_dim, page_size, dtype=dtype, device=device)
    for _ in range(length):
        append_tokens(cache, torch.randn(batch, kv_heads, head_dim).to(dtype).to(device),
                      torch.randn(batch, kv_heads, head_dim).to(dtype).to(device))
    return cache


def test_custom_ops_registered_with_reference_schemas():
    assert ops_available()
    for name, schema in SCHEMAS.items():
        assert str(getattr(torch.ops.flashattn_tile, name).default._schema) == schema
    assert PAGED_DECODE_OP in str(torch.ops.flashattn_tile.paged_decode._schemas)
    assert PREFILL_OP in str(torch.ops.flashattn_tile.prefill_varlen._schemas)
    assert PAGED_DECODE_QUANT_OP in str(torch.ops.flashattn_tile.paged_decode_quant._schemas)


def test_fake_paged_decode_shapes():
    with torch._subclasses.fake_tensor.FakeTensorMode():
        q = torch.empty(3, 4, 8, device="meta")
        k = torch.empty(12, 16, 2, 8, device="meta")
        pt = torch.empty(3, 3, dtype=torch.int32, device="meta")
        sl = torch.full((3,), 5, dtype=torch.int32, device="meta")
        out = torch.ops.flashattn_tile.paged_decode(q, k, k, pt, sl, 16, 0.35, 1)
        sc = torch.empty(12, 2, device="meta")
        outq = torch.ops.flashattn_tile.paged_decode_quant(q, k.to(torch.int8), k.to(torch.int8), sc, sc, pt, sl,
                                                            16, 0.35, 2)
    assert out.shape == (3, 4, 8) and out.dtype == torch.float32 and out.device.type == "meta"
    assert outq.shape == (3, 4, 8)


def test_fake_prefill_varlen_shapes():
    with torch._subclasses.fake_tensor.FakeTensorMode():
        q = torch.empty(11, 4, 8, device="meta")
        k = torch.empty(11, 2, 8, device="meta")
        cu = torch.full((3,), 0, dtype=torch.int32, device="meta")
        out = torch.ops.flashattn_tile.prefill_varlen(q, k, k, cu, cu, 7, 7, True, 0.35)
    assert out.shape == (11, 4, 8) and out.device.type == "meta"


def test_fake_prefill_paged_shapes():
    with torch._subclasses.fake_tensor.FakeTensorMode():
        q = torch.empty(11, 4, 8, device="meta")
        k = torch.empty(12, 16, 2, 8, device="meta")
        pt = torch.empty(2, 3, dtype=torch.int32, device="meta")
        sl = torch.full((2,), 9, dtype=torch.int32, device="meta")
        cu = torch.full((3,), 0, dtype=torch.int32, device="meta")
        out = torch.ops.flashattn_tile.prefill_paged(q, k, k, pt, sl, cu, 7, 16, True, 0.35)
    assert out.shape == (11, 4, 8) and out.device.type == "meta"


def test_fake_paged_decode_multi_shapes():
    with torch._subclasses.fake_tensor.FakeTensorMode():
        q = torch.empty(3, 4, 8, 16, device="meta")
        k = torch.empty(12, 16, 2, 16, device="meta")
        pt = torch.empty(3, 3, dtype=torch.int32, device="meta")
        sl = torch.full((3,), 9, dtype=torch.int32, device="meta")
        out = torch.ops.flashattn_tile.paged_decode_multi(q, k, k, pt, sl, 16, 0.25, 0)
        sc = torch.empty(12, 2, device="meta")
        outq = torch.ops.flashattn_tile.paged_decode_multi(q, k.to(torch.int8), k.to(torch.int8), pt, sl, 16, 0.25,
                                                            2, sc, sc)
    assert out.shape == (3, 4, 8, 16) and out.device.type == "meta" and outq.shape == (3, 4, 8, 16)
    assert str(torch.ops.flashattn_tile.paged_decode_multi.default._schema) == (
        "flashattn_tile::paged_decode_multi(Tensor q, Tensor k_cache, Tensor v_cache, Tensor page_table, "
        "Tensor seq_lens, SymInt page_size, float softmax_scale, SymInt split_k, Tensor? k_scale=None, "
        "Tensor? v_scale=None) -> Tensor")


def test_compile_fullgraph_has_zero_graph_breaks():
    """Traced on meta tensors so no kernel runs on this CPU-only host; the GPU
    suite compiles and runs the same function on the device."""
    q = torch.empty(2, 4, 8, device="meta", dtype=torch.float16)
    k = torch.empty(4, 16, 2, 8, device="meta", dtype=torch.float16)
    pt = torch.zeros(2, 2, dtype=torch.int32, device="meta")
    sl = torch.zeros(2, dtype=torch.int32, device="meta")
    cu = torch.zeros(3, dtype=torch.int32, device="meta")
    kv = torch.empty(9, 2, 8, device="meta", dtype=torch.float16)

    def dec(x):
        return torch.ops.flashattn_tile.paged_decode(x, k, k, pt, sl, 16, 0.35, 1) * 2

    def pre(x):
        return torch.ops.flashattn_tile.prefill_varlen(x, kv, kv, cu, cu, 6, 6, True, 0.35) + 1

    def pre_paged(x):
        return torch.ops.flashattn_tile.prefill_paged(x, k, k, pt, sl, cu, 6, 16, True, 0.35) - 1

    def dec_multi(x):
        return torch.ops.flashattn_tile.paged_decode_multi(x, k, k, pt, sl, 16, 0.35, 0) * 3

    pre_arg = torch.empty(9, 4, 8, device="meta", dtype=torch.float16)
    multi_arg = torch.empty(2, 3, 4, 8, device="meta", dtype=torch.float16)
    for fn, arg in ((dec, q), (pre, pre_arg), (pre_paged, pre_arg), (dec_multi, multi_arg)):
        explanation = torch._dynamo.explain(fn)(arg)
        assert explanation.graph_break_count == 0, explanation.break_reasons
        assert explanation.graph_count == 1
        out = torch.compile(fn, fullgraph=True, backend="eager")(arg)
        assert out.shape == arg.shape


def test_cpu_tensors_raise_instead_of_falling_back():
    cache = _cache(dtype=torch.float16)
    q = torch.randn(2, 4, 8).half()
    with pytest.raises(RuntimeError, match="ROCm device"):
        fat.paged_decode_attention(q, cache)
    with pytest.raises(RuntimeError, match="ROCm device"):
        torch.ops.flashattn_tile.paged_decode(q, cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens,
                                              16, 0.35, 1)
    lens = [3, 6]
    qp = torch.randn(9, 4, 8).half()
    kp = torch.randn(9, 2, 8).half()
    cu = torch.tensor([0, 3, 9], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fat.prefill_attention(qp, kp, kp, cu, cu, max(lens), max(lens))
    cache2 = _cache(batch=2, length=6, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fat.paged_prefill_attention(qp, cache2, cu, 6)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fat.DecodeLaunch(q, cache)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fat.AppendLaunch(cache)


def test_backend_kv_cache_shape_matches_allocate():
    backend = FlashAttnTileBackend(num_heads=8, num_kv_heads=2, head_dim=16, page_size=16)
    cache = backend.allocate_kv_cache(batch=2, max_seq_len=160, dtype=torch.float32, device="cpu")
    shape = backend.get_kv_cache_shape(num_blocks=cache.num_pages, block_size=16, num_kv_heads=2, head_dim=16)
    assert shape == (2, cache.num_pages, 16, 2, 16)
    assert shape[1:] == cache.k_cache.shape
    assert backend.get_kv_cache_shape_per_tensor(cache.num_pages, 16, 2, 16) == cache.k_cache.shape
    assert backend.get_name() == "flashattn_tile"


def test_backend_validation_and_routing_errors():
    backend = FlashAttnTileBackend(num_heads=4, num_kv_heads=2, head_dim=8, page_size=16)
    cache = _cache()
    with pytest.raises(ValueError, match="cu_seqlens"):
        backend.forward(torch.randn(2, 4, 8), cache, AttentionMetadata(is_prefill=True))
    with pytest.raises(ValueError, match="divisible"):
        FlashAttnTileBackend(num_heads=5, num_kv_heads=2, head_dim=8, page_size=16)
    with pytest.raises(TypeError, match="PagedKVCache"):
        backend.forward(torch.randn(2, 4, 8), object(), AttentionMetadata())
    with pytest.raises(ValueError, match="heads"):
        backend.forward(torch.randn(2, 3, 8), cache, AttentionMetadata())
    cu = torch.tensor([0, 3], dtype=torch.int32)
    with pytest.raises(ValueError, match="attn_metadata.k"):
        backend.forward(torch.randn(3, 4, 8), cache, AttentionMetadata(is_prefill=True, cu_seqlens_q=cu,
                                                                       cu_seqlens_k=cu))
    # Paged prefill routing (extension field) needs only cu_seqlens_q and
    # reaches the kernel wrapper, which refuses CPU tensors.
    with pytest.raises(ValueError, match="cu_seqlens_q"):
        backend.forward(torch.randn(3, 4, 8), cache, AttentionMetadata(is_prefill=True, paged_prefill=True))
    with pytest.raises(RuntimeError, match="ROCm device"):
        backend.forward(torch.randn(2, 4, 8), cache, AttentionMetadata(is_prefill=True, paged_prefill=True,
                                                                       cu_seqlens_q=torch.tensor(
                                                                           [0, 1, 2], dtype=torch.int32)))
    # Decode routing reaches the kernel wrapper, which refuses CPU tensors.
    with pytest.raises(RuntimeError, match="ROCm device"):
        backend.forward(torch.randn(2, 1, 4, 8), cache, AttentionMetadata(softmax_scale=0.35))
    # A [batch, q_len > 1, heads, dim] decode query routes to multi-token decode.
    with pytest.raises(RuntimeError, match="ROCm device"):
        backend.forward(torch.randn(2, 3, 4, 8), cache, AttentionMetadata(softmax_scale=0.35))
    with pytest.raises(ValueError, match="heads"):
        backend.forward(torch.randn(2, 3, 5, 8), cache, AttentionMetadata())


def test_native_availability_is_graceful():
    from flashattntile_amd import native

    if torch.cuda.is_available():
        assert native.is_available() or native.unavailable_reason()
    else:
        assert not native.is_available()
        assert native.unavailable_reason()
        with pytest.raises(RuntimeError, match="unavailable"):
            native.paged_decode_attention(torch.zeros(1, 1, 8), None, None, None, None, 16)
