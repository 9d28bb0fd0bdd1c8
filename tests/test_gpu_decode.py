"""GPU parity of the HIP paged decode against the fp32 oracle.

Inputs are unscaled N(0,1) (harsher than the reference tests' 0.2 factor),
pages are scattered by a seeded permutation and the slots past each
sequence's end are poisoned (K = 30, V = 500) so any masking error shows.
Tolerance: 2e-3 on the kernel's result before its final rounding (see
tests/_parity.py); quantised caches are compared with the oracle run on the
cache dequantised to q.dtype (the reference's own dequantise-then-attend).
"""

from __future__ import annotations

import math

import pytest
import torch

from _parity import assert_parity, force_decode_knobs, make_paged, make_query, ulp
from flashattntile_amd import PagedKVCache, paged_decode_attention, paged_decode_attention_fp8
from flashattntile_amd.kernels.decode import paged_decode_launch
from oracle import quant_ref
from oracle.reference import ref_attention_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODD_LENS = [1, 17, 255, 1000]
GQA = [(8, 8), (8, 2), (8, 1), (32, 8), (32, 1)]


@pytest.fixture(params=["auto", "valu", "mfma", "mfma8", "generic"])
def decode_kernel(request, monkeypatch):
    """Run with the library's choice and with each decode kernel forced: the
    VALU decode, the MFMA decode with 4 and with 8 waves per workgroup (the
    library picks 8 only for long partitions in small grids), and the generic
    LDS-tiled decode (the library's choice only for shapes the other two do
    not take)."""
    knobs = {"valu": {"kernel": "valu"}, "mfma": {"kernel": "mfma", "num_warps": 4},
             "mfma8": {"kernel": "mfma", "num_warps": 8}, "generic": {"kernel": "generic"}}.get(request.param)
    if knobs:
        force_decode_knobs(monkeypatch, **knobs)
    return request.param


def _case(lens, h, hk, d, P, dtype, seed=0):
    k, v, pt, sl = make_paged(lens, hk, d, P, dtype, seed=seed, device=DEV)
    q = make_query(len(lens), h, d, dtype, seed=seed + 1, device=DEV)
    return q, PagedKVCache(k, v, pt, sl, P)


def _ref32(q, cache, scale=None):
    return ref_attention_paged(q.cpu(), cache.k_cache.cpu(), cache.v_cache.cpu(), cache.page_table.cpu(),
                               cache.seq_lens.cpu(), softmax_scale=scale, return_fp32=True)


@pytest.mark.parametrize("split_k", [1, 4])
@pytest.mark.parametrize("page_size", [16, 32])
@pytest.mark.parametrize("h,hk", GQA)
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_matches_oracle(dtype, d, h, hk, page_size, split_k, decode_kernel):
    label = f"decode {decode_kernel} {dtype} D{d} H{h}/{hk} P{page_size} sk{split_k}"
    print(label, flush=True)
    q, cache = _case(ODD_LENS, h, hk, d, page_size, dtype, seed=d + h + hk)
    out = paged_decode_attention(q, cache, config={"split_k": split_k})
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == dtype
    assert_parity(out, _ref32(q, cache), label=label)


@pytest.mark.parametrize("page_size", [4, 8, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_page_sizes(dtype, page_size, decode_kernel):
    label = f"decode {decode_kernel} pages {dtype} P{page_size}"
    print(label, flush=True)
    d = 128 if page_size >= 8 else 128
    lens = [3, 64, 65, 300]
    q, cache = _case(lens, 32, 8, d, page_size, dtype, seed=page_size)
    for split_k in (1, 3):
        out = paged_decode_attention(q, cache, config={"split_k": split_k})
        torch.cuda.synchronize()
        assert_parity(out, _ref32(q, cache), label=f"{label} sk{split_k}")


def test_decode_more_splits_than_pages():
    """Empty partitions must contribute nothing (reference test_decode.py:132-139)."""
    print("decode split 16 > pages", flush=True)
    q, cache = _case([8, 20], 4, 2, 64, 16, torch.float16, seed=24)
    out = paged_decode_attention(q, cache, config={"split_k": 16})
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache), label="split16")


@pytest.mark.parametrize("hk", [8, 1])
def test_split_k_agreement_and_softmax_scale(hk, decode_kernel):
    print(f"decode split agreement {decode_kernel} H32/{hk}", flush=True)
    lens = [1, 17, 255, 1000, 4096, 333]
    q, cache = _case(lens, 32, hk, 128, 16, torch.float16, seed=22)
    ref = _ref32(q, cache, scale=0.05)
    outs = {}
    for s in (1, 2, 5, 8, 16, 64):
        outs[s] = paged_decode_attention(q, cache, softmax_scale=0.05, config={"split_k": s})
    torch.cuda.synchronize()
    for s, o in outs.items():
        assert_parity(o, ref, label=f"scale0.05 sk{s}")
        assert (o.float() - outs[1].float()).abs().max().item() <= 2e-3
    neg = paged_decode_attention(q, cache, softmax_scale=-0.05, config={"split_k": 3})
    torch.cuda.synchronize()
    assert_parity(neg, _ref32(q, cache, scale=-0.05), label="negative scale")


def _quant_case(lens, h, hk, d, P, qdtype, mode, seed):
    k, v, pt, sl = make_paged(lens, hk, d, P, torch.float32, seed=seed, device="cpu")
    qk, sk = quant_ref.quantize_pages(k, mode)
    qv, sv = quant_ref.quantize_pages(v, mode)
    q = make_query(len(lens), h, d, qdtype, seed=seed + 1, device=DEV)
    cache = PagedKVCache(qk.to(DEV), qv.to(DEV), pt.to(DEV), sl.to(DEV), P)
    deq_k = quant_ref.dequantize_pages(qk, sk, qdtype)
    deq_v = quant_ref.dequantize_pages(qv, sv, qdtype)
    ref = ref_attention_paged(q.cpu(), deq_k, deq_v, pt, sl, return_fp32=True)
    return q, cache, {"k": sk.to(DEV), "v": sv.to(DEV)}, ref


@pytest.mark.parametrize("split_k", [1, 4])
@pytest.mark.parametrize("h,hk", [(8, 2), (32, 8), (8, 8), (32, 1)])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
def test_quant_decode_matches_dequantized_oracle(mode, qdtype, d, h, hk, split_k, decode_kernel):
    label = f"quant {decode_kernel} {mode} {qdtype} D{d} H{h}/{hk} sk{split_k}"
    print(label, flush=True)
    q, cache, scales, ref = _quant_case(ODD_LENS, h, hk, d, 16, qdtype, mode, seed=13 + d)
    if decode_kernel == "valu" and h // hk >= 8:
        # the VALU decode takes 8-bit caches only for groups below 8 (its
        # 8-head form spills); the library says so instead of launching
        with pytest.raises(RuntimeError, match="VALU decode takes int8/fp8 caches"):
            paged_decode_attention_fp8(q, cache, scales, config={"split_k": split_k})
        return
    out = paged_decode_attention_fp8(q, cache, scales, config={"split_k": split_k})
    torch.cuda.synchronize()
    assert out.dtype == qdtype
    assert_parity(out, ref, label=label)


@pytest.mark.parametrize("d,P", [(128, 8), (128, 32), (128, 64), (64, 16), (64, 128)])
@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
def test_quant_decode_page_sizes(mode, qdtype, d, P, decode_kernel):
    """8-bit caches at page sizes from the floor (the rows of one 16-byte
    load, 8 at D128 and 16 at D64) up: k_scale and v_scale are applied per
    load, whose rows must lie in one page."""
    label = f"quant {decode_kernel} {mode} {qdtype} D{d} P{P}"
    print(label, flush=True)
    q, cache, scales, ref = _quant_case(ODD_LENS, 32, 8, d, P, qdtype, mode, seed=17 + P)
    for split_k in (1, 3):
        out = paged_decode_attention_fp8(q, cache, scales, config={"split_k": split_k})
        torch.cuda.synchronize()
        assert_parity(out, ref, label=f"{label} sk{split_k}")


@pytest.mark.parametrize("order", ["random", "growing"])
@pytest.mark.parametrize("split_k", [1, 4])
@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
def test_quant_decode_extreme_page_scales(mode, split_k, order, decode_kernel):
    """Per-page V magnitudes from 1e-6 to 4e4 (K from 1e-2 to 10, logits
    with a standard deviation near 10), so the (page, KV head) scales span
    ten decades and neighbouring pages (which may share a 32-key block)
    differ by up to that much; "growing" orders each sequence's pages by
    increasing V magnitude.  With fp16 queries the kernels apply k_scale to
    the fp32 scores, as the reference's quantised kernel does
    (kernels/decode.py:419-429), so the oracle here dequantises to fp32, as
    the reference's own numerics test does (tests/test_numerics.py:152):
    at these logits the fp16 rounding of a dequantised K alone moves the
    softmax by 0.5 %.  2e-3 relative to each output row's magnitude beyond
    the final fp16 rounding."""
    label = f"quant {decode_kernel} {mode} extreme page scales {order} sk{split_k}"
    print(label, flush=True)
    lens = [700, 4096, 129, 33]
    k, v, pt, sl = make_paged(lens, 8, 128, 16, torch.float32, seed=41, device="cpu", poison=False)
    g = torch.Generator().manual_seed(42)
    n = k.shape[0]
    v_exp = torch.rand(n, generator=g) * 10.0 - 6.0  # log10 of the page's V magnitude, 1e-6 .. 1e4
    k_exp = torch.rand(n, generator=g) * 3.0 - 2.0
    if order == "growing":  # page j of each sequence gets a larger V magnitude than page j - 1
        for b, ln in enumerate(lens):
            pages = pt[b, : -(-ln // 16)].long()
            v_exp[pages] = torch.linspace(-6.0, 4.0, len(pages))
    v = v * torch.pow(10.0, v_exp).view(n, 1, 1, 1) * 4.0 / 4.5  # |v| stays below fp16 max after dequant
    k = k * torch.pow(10.0, k_exp).view(n, 1, 1, 1)
    qk, sk = quant_ref.quantize_pages(k, mode)
    qv, sv = quant_ref.quantize_pages(v, mode)
    q = make_query(len(lens), 32, 128, torch.float16, seed=43, device=DEV)
    cache = PagedKVCache(qk.to(DEV), qv.to(DEV), pt.to(DEV), sl.to(DEV), 16)
    ref = ref_attention_paged(q.cpu().float(), quant_ref.dequantize_pages(qk, sk, torch.float32),
                              quant_ref.dequantize_pages(qv, sv, torch.float32), pt, sl, return_fp32=True)
    out = paged_decode_attention_fp8(q, cache, {"k": sk.to(DEV), "v": sv.to(DEV)}, config={"split_k": split_k})
    torch.cuda.synchronize()
    o32, r32 = out.float().cpu(), ref.float()
    scale = r32.abs().amax(dim=-1, keepdim=True).clamp_min(1.0)
    rounding = 0.5 * ulp(torch.maximum(o32.abs(), r32.abs()), torch.float16)
    excess = ((o32 - r32).abs() - rounding) / scale
    print(f"{label}: max relative error beyond rounding {excess.max().item():.3e}", flush=True)
    assert torch.isfinite(o32).all() and excess.max().item() <= 2e-3, label


def test_permuted_pool_is_bit_identical():
    """Relocating pages (and remapping the table) must not change one bit."""
    print("decode permutation invariance", flush=True)
    q, cache = _case([700, 1, 4096, 129], 32, 8, 128, 16, torch.bfloat16, seed=31)
    out = paged_decode_attention(q, cache, config={"split_k": 4})
    g = torch.Generator().manual_seed(5)
    perm = torch.randperm(cache.num_pages, generator=g).to(DEV)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(cache.num_pages, device=DEV)
    moved = PagedKVCache(cache.k_cache[perm].contiguous(), cache.v_cache[perm].contiguous(),
                         inv[cache.page_table.long()].to(torch.int32), cache.seq_lens, cache.page_size)
    out2 = paged_decode_attention(q, moved, config={"split_k": 4})
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_baseline_config_b32_ctx4096():
    """fp16, B32, ctx 4096, 32/8 heads, D128, page 16."""
    print("decode B32 ctx4096", flush=True)
    q, cache = _case([4096] * 32, 32, 8, 128, 16, torch.float16, seed=1)
    for split_k in (1, 4, 8):
        out = paged_decode_attention(q, cache, config={"split_k": split_k})
        torch.cuda.synchronize()
        assert_parity(out, _ref32(q, cache), label=f"B32 ctx4096 sk{split_k}")


def test_long_context_and_skewed_batch():
    """B1 ctx 131072 (split 16) and 64 log-uniform lengths."""
    print("decode ctx131072", flush=True)
    q, cache = _case([131072], 32, 8, 128, 16, torch.float16, seed=2)
    out = paged_decode_attention(q, cache, config={"split_k": 16})
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache), label="ctx131072 sk16")
    print("decode skewed batch", flush=True)
    g = torch.Generator().manual_seed(64)
    lens = [int(math.exp(x)) for x in (torch.rand(64, generator=g) * (math.log(65536) - math.log(16))
                                        + math.log(16)).tolist()]
    q, cache = _case(lens, 32, 8, 128, 16, torch.float16, seed=3)
    out = paged_decode_attention(q, cache)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache), label="skewed64")


@pytest.mark.parametrize("h,hk,d,P", [(32, 1, 128, 16), (32, 8, 64, 16), (32, 8, 128, 32), (32, 8, 128, 64),
                                      (64, 1, 128, 16), (16, 1, 64, 32), (48, 3, 128, 16)])
def test_stress_variants(h, hk, d, P):
    label = f"stress H{h}/{hk} D{d} P{P}"
    print(label, flush=True)
    q, cache = _case([16, 1000, 8191, 3000], h, hk, d, P, torch.float16, seed=h + hk + d + P)
    out = paged_decode_attention(q, cache)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache), label=label)


def test_launch_reuses_buffers():
    """paged_decode_launch with caller-owned out/workspace (no allocation)."""
    print("decode launch reuse", flush=True)
    from flashattntile_amd import _hip
    q, cache = _case([100, 2000], 32, 8, 128, 16, torch.float16, seed=40)
    out = torch.empty_like(q)
    ws = torch.empty(_hip.decode_workspace_bytes(2, 32, 128, 8), dtype=torch.uint8, device=DEV)
    r = paged_decode_launch(q, cache, 128 ** -0.5, 8, out=out, workspace=ws)
    torch.cuda.synchronize()
    assert r.data_ptr() == out.data_ptr()
    assert_parity(out, _ref32(q, cache), label="launch reuse")


def test_native_library_is_the_path():
    import flashattntile_amd._hip as hip
    assert hip.is_loaded(), hip.load_error()
    with open("/proc/self/maps") as fh:
        assert "libfat_hip.so" in fh.read()


@pytest.mark.parametrize("kern", ["valu", "mfma"])
@pytest.mark.parametrize("split_k,pps", [(4, 16), (2, 8), (8, 3), (1, 5), (3, 200)])
def test_fixed_pages_per_split(split_k, pps, kern):
    """Fixed-size partitions (pages_per_split > 0): equal to the oracle whether
    split_k * pages_per_split covers the longest sequence or falls short (then
    the last partition takes the remaining pages).  Every partition of a fixed
    size reads its first page ids before seq_len is known; sequences of 5, 16
    and 37 tokens end inside a wave's first unit, and partitions past a
    sequence's end read nothing."""
    label = f"decode fixed partitions {kern} sk{split_k} pps{pps}"
    print(label, flush=True)
    lens = [5, 1000, 37, 4096, 16, 2500]
    q, cache = _case(lens, 32, 8, 128, 16, torch.float16, seed=50 + pps)
    out = paged_decode_attention(q, cache, config={"split_k": split_k, "pages_per_split": pps, "kernel": kern})
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache), label=label)


def test_auto_partition_skewed_batch():
    """config=None on a skewed batch picks fixed-size partitions."""
    from flashattntile_amd.kernels.decode import _resolve_config
    print("decode auto partition skewed", flush=True)
    g = torch.Generator().manual_seed(77)
    lens = [int(math.exp(x)) for x in (torch.rand(48, generator=g) * (math.log(30000) - math.log(16))
                                        + math.log(16)).tolist()]
    q, cache = _case(lens, 32, 8, 128, 16, torch.bfloat16, seed=7)
    total = sum(-(-n // 16) for n in lens)
    cfg = _resolve_config(None, q, cache, max(lens), total)
    assert cfg["pages_per_split"] > 0
    out = paged_decode_attention(q, cache)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache), label="auto partition skewed")


@pytest.mark.parametrize("layout", ["transposed", "every_other_column"])
def test_decode_strided_page_table_and_seq_lens(layout):
    """A page table whose columns are not unit-strided (a transposed layout,
    or every second column of a wider table) and a strided seq_lens give the
    contiguous launch's exact bits: the wrapper makes them dense before the
    kernel reads them (the reference honours any strides, kernels/decode.py:89).
    DecodeLaunch, which keeps raw pointers across runs, refuses them."""
    from flashattntile_amd.kernels.decode import DecodeLaunch

    q, cache = _case([700, 33, 1, 400], 8, 2, 128, 16, torch.float16, seed=41)
    pt, sl = cache.page_table, cache.seq_lens
    if layout == "transposed":
        pt_s = pt.t().contiguous().t()
    else:
        wide = torch.full((pt.shape[0], 2 * pt.shape[1]), -7, dtype=torch.int32, device=DEV)
        wide[:, ::2] = pt
        pt_s = wide[:, ::2]
    sl_s = torch.stack([sl, torch.full_like(sl, 99999)], dim=1)[:, 0]
    assert pt_s.stride(-1) != 1 and not sl_s.is_contiguous() and torch.equal(pt_s, pt) and torch.equal(sl_s, sl)
    strided = PagedKVCache(cache.k_cache, cache.v_cache, pt_s, sl_s, cache.page_size)
    for split in (1, 3):
        want = paged_decode_attention(q, cache, config={"split_k": split})
        got = paged_decode_attention(q, strided, config={"split_k": split})
        torch.cuda.synchronize()
        assert torch.equal(got, want), (layout, split)
    assert_parity(got, _ref32(q, cache), label=f"decode strided table {layout}")
    with pytest.raises(ValueError, match="contiguous"):
        DecodeLaunch(q, strided)
