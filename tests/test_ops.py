"""Operator boundary: registration, schemas, fake kernels, torch.compile,
backend surface, and the absence of any CPU fallback."""

from __future__ import annotations

import pytest
import torch

import flashattntile_amd as fat
from flashattntile_amd.backend import AttentionMetadata, FlashAttnTileBackend
from flashattntile_amd.ops import PAGED_DECODE_OP, PAGED_DECODE_QUANT_OP, PREFILL_OP, ops_available
from flashattntile_amd.paging import PagedKVCache

SCHEMAS = {
    "paged_decode": "flashattn_tile::paged_decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor page_table, "
                    "Tensor seq_lens, SymInt page_size, float softmax_scale, SymInt split_k) -> Tensor",
    "prefill_varlen": "flashattn_tile::prefill_varlen(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, "
                      "Tensor cu_seqlens_k, SymInt max_seqlen_q, SymInt max_seqlen_k, bool causal, "
                      "float softmax_scale) -> Tensor",
}


def _cache(lens=(12, 12), page_size=16, kv_heads=2, head_dim=8, dtype=torch.float32, seed=3) -> PagedKVCache:
    """Host cache with identity page order, filled with seeded N(0,1) rows."""
    g = torch.Generator().manual_seed(seed)
    per = [-(-n // page_size) for n in lens]
    shape = (sum(per), page_size, kv_heads, head_dim)
    table = torch.zeros(len(lens), max(per), dtype=torch.int32)
    at = 0
    for b, n in enumerate(per):
        table[b, :n] = torch.arange(at, at + n, dtype=torch.int32)
        at += n
    return PagedKVCache(torch.randn(shape, generator=g).to(dtype), torch.randn(shape, generator=g).to(dtype), table,
                        torch.tensor(lens, dtype=torch.int32), page_size)


def test_custom_ops_registered_with_reference_schemas():
    assert ops_available()
    for name, schema in SCHEMAS.items():
        assert str(getattr(torch.ops.flashattn_tile, name).default._schema) == schema
    assert PAGED_DECODE_OP in str(torch.ops.flashattn_tile.paged_decode._schemas)
    assert PREFILL_OP in str(torch.ops.flashattn_tile.prefill_varlen._schemas)
    assert PAGED_DECODE_QUANT_OP in str(torch.ops.flashattn_tile.paged_decode_quant._schemas)


# (batch, q heads, kv heads, head_dim, pages, page_size, dtype) of the meta
# problems the fake kernels are traced on.
FAKE_DECODE_SHAPES = [
    (1, 2, 1, 64, 5, 8, torch.float16),
    (5, 12, 4, 32, 40, 32, torch.bfloat16),
    (2, 16, 16, 128, 9, 1, torch.float32),
]


@pytest.mark.parametrize("b,h,hk,d,pages,ps,dtype", FAKE_DECODE_SHAPES)
def test_fake_decode_ops_give_the_query_shape_and_dtype(b, h, hk, d, pages, ps, dtype):
    """Under FakeTensorMode no kernel runs: both decode ops report an output
    of the query's shape, dtype and device (kernels/decode.py's register_fake
    contract, flashattn_tile/ops.py:56-73)."""
    with torch._subclasses.fake_tensor.FakeTensorMode():
        q = torch.empty(b, h, d, dtype=dtype, device="meta")
        kv = torch.empty(pages, ps, hk, d, dtype=dtype, device="meta")
        table = torch.empty(b, pages, dtype=torch.int32, device="meta")
        lens = torch.empty(b, dtype=torch.int32, device="meta")
        scales = torch.empty(pages, hk, device="meta")
        outs = [torch.ops.flashattn_tile.paged_decode(q, kv, kv, table, lens, ps, 0.125, 2)]
        if dtype != torch.float32:
            codes = kv.to(torch.float8_e4m3fn)
            outs.append(torch.ops.flashattn_tile.paged_decode_quant(q, codes, codes, scales, scales, table, lens, ps,
                                                                     0.125, 1))
    for out in outs:
        assert (tuple(out.shape), out.dtype, out.device.type) == ((b, h, d), dtype, "meta")


@pytest.mark.parametrize("tokens,h,hk,d,dtype", [(1, 4, 4, 64, torch.float16), (37, 24, 8, 128, torch.bfloat16)])
def test_fake_prefill_op_gives_the_query_shape_and_dtype(tokens, h, hk, d, dtype):
    with torch._subclasses.fake_tensor.FakeTensorMode():
        q = torch.empty(tokens, h, d, dtype=dtype, device="meta")
        kv = torch.empty(tokens + 3, hk, d, dtype=dtype, device="meta")
        cq = torch.empty(4, dtype=torch.int32, device="meta")
        out = torch.ops.flashattn_tile.prefill_varlen(q, kv, kv, cq, cq, tokens, tokens + 3, False, 0.25)
    assert (tuple(out.shape), out.dtype, out.device.type) == ((tokens, h, d), dtype, "meta")


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
    cache2 = _cache(lens=(6, 6), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fat.paged_prefill_attention(qp, cache2, cu, 6)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fat.DecodeLaunch(q, cache)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fat.AppendLaunch(cache)


@pytest.mark.parametrize("hk,d,ps,batch,max_len", [(1, 64, 32, 3, 70), (4, 128, 8, 1, 8), (8, 32, 1, 2, 5)])
def test_backend_cache_shape_agrees_with_its_allocation(hk, d, ps, batch, max_len):
    """The vLLM-style 5-D shape is (K and V, blocks, block_size, kv heads,
    head_dim), and the cache the backend allocates is exactly one of its two
    halves (flashattn_tile/backend.py:57-60, paging.py:30-60)."""
    backend = FlashAttnTileBackend(num_heads=2 * hk, num_kv_heads=hk, head_dim=d, page_size=ps)
    cache = backend.allocate_kv_cache(batch=batch, max_seq_len=max_len, dtype=torch.bfloat16, device="cpu")
    assert cache.num_pages >= batch * -(-max_len // ps)
    five = backend.get_kv_cache_shape(cache.num_pages, ps, hk, d)
    assert five[0] == 2 and five[1:] == tuple(cache.v_cache.shape) == tuple(cache.k_cache.shape)
    assert backend.get_kv_cache_shape_per_tensor(cache.num_pages, ps, hk, d) == five[1:]
    assert FlashAttnTileBackend.get_kv_cache_shape(7, 4, 3, 2) == (2, 7, 4, 3, 2)


def test_backend_reports_its_name():
    assert FlashAttnTileBackend(num_heads=1, num_kv_heads=1, head_dim=32, page_size=4).get_name() == "flashattn_tile"


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


def test_native_probe_never_raises_and_explains_itself():
    """is_available() / unavailable_reason() are total (flashattn_tile/
    native.py:54-84): the reason is empty exactly when the path is usable."""
    from flashattntile_amd import native

    usable = native.is_available()
    reason = native.unavailable_reason()
    assert isinstance(usable, bool) and isinstance(reason, str)
    assert usable == (reason == "")


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the host without a ROCm device")
def test_native_decode_without_a_device_raises_with_the_reason():
    from flashattntile_amd import native

    assert not native.is_available()
    cache = _cache(lens=(3,), head_dim=64)
    with pytest.raises(RuntimeError, match="unavailable") as info:
        native.paged_decode_attention(torch.zeros(1, 4, 64), cache.k_cache, cache.v_cache, cache.page_table,
                                      cache.seq_lens, 16)
    assert native.unavailable_reason() in str(info.value)
