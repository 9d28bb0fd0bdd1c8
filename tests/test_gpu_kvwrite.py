"""GPU parity of the KV write path: ``fat_quantize_pages`` and ``fat_append_kv``.

Both are byte/integer work, so the bar is bit-exact:
* quantisation codes and fp32 scales equal the oracle's
  (``oracle/quant_ref.quantize_pages``, the restatement of
  ``flashattn_tile/quant.py:84-142`` run by torch on the CPU) -- on random
  pages of every source dtype and, with the scale pinned to exactly 1, on
  every finite fp16 value and on fp32 values at and beside every fp8 rounding
  boundary, which checks the gfx950 conversion against torch's;
* appended pages and lengths equal a per-element restatement of
  ``flashattn_tile/paging.py:172-210``; an int8/fp8 copy maintained by the
  append equals the oracle's quantisation of the whole updated cache.
"""

from __future__ import annotations

import math

import pytest
import torch

from flashattntile_amd import _hip
from flashattntile_amd.paging import PagedKVCache, append_tokens
from flashattntile_amd.quant import quantize_cache, quantize_kv_pages
from oracle import quant_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
FP8 = getattr(torch, "float8_e4m3fn", None)
MODES = ["int8", "float8_e4m3fn"]
QMAX = {"int8": 127.0, "float8_e4m3fn": 448.0}


def _bytes(t: torch.Tensor) -> torch.Tensor:
    return t.detach().cpu().contiguous().view(torch.uint8)


def _assert_codes_equal(got: torch.Tensor, want: torch.Tensor, what: str) -> None:
    g, w = _bytes(got), _bytes(want)
    bad = (g != w).nonzero()
    assert bad.numel() == 0, f"{what}: {bad.shape[0]} codes differ, first at {bad[0].tolist()}: " \
                             f"{int(g[tuple(bad[0])])} vs {int(w[tuple(bad[0])])}"


def _quantize_hip(x: torch.Tensor, mode: str):
    dtype = torch.int8 if mode == "int8" else FP8
    codes = torch.empty(x.shape, dtype=dtype, device=x.device)
    scale = torch.empty(x.shape[0], x.shape[2], dtype=torch.float32, device=x.device)
    _hip.quantize_pages(x, codes, scale)
    torch.cuda.synchronize()
    return codes, scale


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("src_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(37, 16, 8, 128), (9, 32, 2, 64), (5, 1, 3, 256), (6, 7, 2, 36), (3, 64, 2, 128)])
@pytest.mark.parametrize("magnitude", [1.0, 1e-3, 300.0])
def test_quantize_pages_matches_oracle(mode, src_dtype, shape, magnitude):
    print(f"quantize {mode} {src_dtype} {shape} x{magnitude}", flush=True)
    g = torch.Generator().manual_seed(sum(shape) + int(magnitude * 7))
    x = (torch.randn(shape, generator=g) * magnitude).to(src_dtype)
    x[0] = 0  # an all-zero page: scale floors at 1e-8
    codes, scale = _quantize_hip(x.to(DEV), mode)
    want_codes, want_scale = quant_ref.quantize_pages(x, mode)
    assert scale.dtype == torch.float32 and tuple(scale.shape) == (shape[0], shape[2])
    assert torch.equal(scale.cpu(), want_scale), (scale.cpu() - want_scale).abs().max()
    _assert_codes_equal(codes, want_codes, f"{mode} {src_dtype} {shape}")
    assert torch.all(scale[0] == torch.tensor(1e-8, dtype=torch.float32).to(DEV))


@pytest.mark.parametrize("mode", MODES)
def test_quantize_strided_and_misaligned_views(mode):
    """Views whose strides are not the packed ones: a head slice (16-byte
    chunks still aligned) and a head_dim window starting one element in
    (misaligned: the one-element-per-lane kernels)."""
    g = torch.Generator().manual_seed(11)
    big = torch.randn(7, 16, 4, 72, generator=g).half()
    for view in (big[:, :, 1:3, :64], big[:, :, :, 1:65], big[:, ::2, :, 8:72]):
        print(f"quantize view strides {view.stride()}", flush=True)
        # The same view of a device copy.
        dview = big.to(DEV).as_strided(view.shape, view.stride(), view.storage_offset())
        codes, scale = _quantize_hip(dview, mode)
        want_codes, want_scale = quant_ref.quantize_pages(view, mode)
        assert torch.equal(scale.cpu(), want_scale)
        _assert_codes_equal(codes, want_codes, f"view {view.stride()}")
    # A strided destination: codes land in a [.., 64] window of 72-wide rows.
    x = torch.randn(3, 16, 2, 64, generator=g).bfloat16()
    dst_full = torch.zeros(3, 16, 2, 72, dtype=torch.int8 if mode == "int8" else FP8, device=DEV)
    dst = dst_full[..., :64]
    scale = torch.empty(3, 2, dtype=torch.float32, device=DEV)
    _hip.quantize_pages(x.to(DEV), dst, scale)
    torch.cuda.synchronize()
    want_codes, want_scale = quant_ref.quantize_pages(x, mode)
    _assert_codes_equal(dst, want_codes, "strided dst")
    assert torch.all(_bytes(dst_full[..., 64:]) == 0), "wrote outside the destination window"


def _unit_pages(values: torch.Tensor, qmax: float, dtype: torch.dtype, P: int = 16, D: int = 64):
    """Pack ``values`` into [pages, P, 1, D] units whose absmax is exactly
    ``qmax`` (element 0 of every unit), so the scale is exactly 1."""
    per = P * D - 1
    n = values.numel()
    pages = (n + per - 1) // per
    flat = torch.zeros(pages, P * D, dtype=torch.float32)
    flat[:, 0] = qmax
    body = torch.zeros(pages * per, dtype=torch.float32)
    body[:n] = values.float()
    flat[:, 1:] = body.view(pages, per)
    x = flat.view(pages, P, 1, D).to(dtype)
    assert torch.equal(x.float().view(pages, -1)[:, 1:].reshape(-1)[:n], values.float())
    return x


@pytest.mark.parametrize("mode", MODES)
def test_every_fp16_value_quantises_like_torch(mode):
    """All finite fp16 values within range, at scale 1: int8 round-half-even
    and the fp16 -> e4m3fn conversion, code for code."""
    qmax = QMAX[mode]
    allv = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
    vals = allv[torch.isfinite(allv) & (allv.float().abs() <= qmax)]
    x = _unit_pages(vals, qmax, torch.float16)
    print(f"fp16 sweep {mode}: {vals.numel()} values in {x.shape[0]} pages", flush=True)
    codes, scale = _quantize_hip(x.to(DEV), mode)
    assert torch.all(scale.cpu() == 1.0)
    want_codes, _ = quant_ref.quantize_pages(x, mode)
    _assert_codes_equal(codes, want_codes, f"fp16 sweep {mode}")


def test_fp8_rounding_boundaries_match_torch():
    """fp32 values at, between and one ulp either side of the midpoint of
    every pair of adjacent e4m3fn values (incl. subnormals and +-0), plus
    random ones, at scale 1."""
    table = quant_ref.fp8_table()
    pos = table[:0x7F].double()  # 0 .. 448, finite, increasing
    mids = ((pos[1:] + pos[:-1]) / 2).float()
    below = torch.nextafter(mids, torch.full_like(mids, -math.inf))
    above = torch.nextafter(mids, torch.full_like(mids, math.inf))
    g = torch.Generator().manual_seed(5)
    rand = torch.cat([(torch.rand(200000, generator=g) * 2 - 1) * 448,
                      (torch.rand(100000, generator=g) * 2 - 1) * 2.0 ** -5])
    one = torch.cat([pos.float(), mids, below, above])
    vals = torch.cat([one, -one, rand, torch.tensor([-0.0, 0.0, 2.0 ** -10, -(2.0 ** -10), 2.0 ** -11])])
    x = _unit_pages(vals, 448.0, torch.float32)
    codes, scale = _quantize_hip(x.to(DEV), "float8_e4m3fn")
    assert torch.all(scale.cpu() == 1.0)
    want_codes, _ = quant_ref.quantize_pages(x, "float8_e4m3fn")
    _assert_codes_equal(codes, want_codes, "fp8 boundaries")


def test_int8_ties_round_half_even():
    ks = torch.arange(-127, 127, dtype=torch.float32)
    ties = ks + 0.5
    vals = torch.cat([ties, torch.nextafter(ties, ties - 1), torch.nextafter(ties, ties + 1), ks,
                      torch.tensor([-0.0, 126.99999, -127.0])])
    x = _unit_pages(vals, 127.0, torch.float32)
    codes, _ = _quantize_hip(x.to(DEV), "int8")
    want_codes, _ = quant_ref.quantize_pages(x, "int8")
    _assert_codes_equal(codes, want_codes, "int8 ties")
    # Spot-check the closed form: 0.5 -> 0, 1.5 -> 2, -2.5 -> -2.
    flat = codes.cpu().view(x.shape[0], -1)[:, 1:].reshape(-1)
    lut = {float(v): int(c) for v, c in zip(vals.tolist(), flat[:vals.numel()].tolist())}
    assert lut[0.5] == 0 and lut[1.5] == 2 and lut[-2.5] == -2 and lut[126.5] == 126


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_quantize_kv_pages_routes_to_hip(mode, dtype):
    g = torch.Generator().manual_seed(2)
    k = torch.randn(12, 16, 4, 128, generator=g).to(dtype)
    v = torch.randn(12, 16, 4, 128, generator=g).to(dtype)
    qk, qv, sk, sv, info = quantize_kv_pages(k.to(DEV), v.to(DEV), mode=mode)
    assert qk.is_cuda and info["mode"] == mode
    for got, gs, src in ((qk, sk, k), (qv, sv, v)):
        want, ws = quant_ref.quantize_pages(src, mode)
        _assert_codes_equal(got, want, "quantize_kv_pages")
        assert torch.equal(gs.cpu(), ws)
    assert info["scale_min"] == float(sk.min()) and info["scale_max"] == float(sk.max())


# ---------------------------------------------------------------------------
# Append
# ---------------------------------------------------------------------------
def _cache(lens, hkv, d, P, dtype, extra_pages=3, seed=0):
    """A cache with room for 4 more tokens per sequence, pages permuted."""
    g = torch.Generator().manual_seed(seed)
    maxp = max((n + 4 + P - 1) // P for n in lens)
    pages = len(lens) * maxp + extra_pages
    k = torch.randn(pages, P, hkv, d, generator=g).to(dtype)
    v = torch.randn(pages, P, hkv, d, generator=g).to(dtype)
    perm = torch.randperm(pages, generator=g).to(torch.int32)
    pt = perm[: len(lens) * maxp].view(len(lens), maxp).clone()
    sl = torch.tensor(lens, dtype=torch.int32)
    return PagedKVCache(k, v, pt, sl, P)


def _append_restated(k, v, pt, sl, P, nk, nv):
    """paging.py:172-210, element by element on CPU copies."""
    k, v, sl = k.clone(), v.clone(), sl.clone()
    for b in range(sl.numel()):
        pos = int(sl[b])
        page = int(pt[b, pos // P])
        k[page, pos % P] = nk[b]
        v[page, pos % P] = nv[b]
        sl[b] += 1
    return k, v, sl


def _to(cache, dev):
    return PagedKVCache(cache.k_cache.to(dev), cache.v_cache.to(dev), cache.page_table.to(dev),
                        cache.seq_lens.to(dev), cache.page_size)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hkv,d,P", [(2, 128, 16), (8, 64, 32), (1, 256, 1), (3, 36, 8)])
def test_append_matches_reference(dtype, hkv, d, P):
    lens = [0, P - 1, P, 2 * P + 3, 77]
    host = _cache(lens, hkv, d, P, dtype, seed=hkv * d + P)
    cache = _to(host, DEV)
    g = torch.Generator().manual_seed(1)
    k, v, sl = host.k_cache, host.v_cache, host.seq_lens
    for step in range(3):
        print(f"append {dtype} Hkv{hkv} D{d} P{P} step {step}", flush=True)
        nk = torch.randn(len(lens), hkv, d, generator=g).to(dtype)
        nv = torch.randn(len(lens), hkv, d, generator=g).to(dtype)
        append_tokens(cache, nk.to(DEV), nv.to(DEV))
        k, v, sl = _append_restated(k, v, host.page_table, sl, P, nk, nv)
        torch.cuda.synchronize()
        assert torch.equal(cache.seq_lens.cpu(), sl)
        assert torch.equal(_bytes(cache.k_cache), _bytes(k))
        assert torch.equal(_bytes(cache.v_cache), _bytes(v))


def test_append_non_contiguous_new_rows():
    host = _cache([3, 9], 2, 64, 16, torch.float16, seed=4)
    cache = _to(host, DEV)
    g = torch.Generator().manual_seed(8)
    wide_k = torch.randn(2, 2, 128, generator=g).half()
    wide_v = torch.randn(2, 2, 128, generator=g).half()
    nk, nv = wide_k[..., 32:96], wide_v[..., ::2]
    append_tokens(cache, wide_k.to(DEV)[..., 32:96], wide_v.to(DEV)[..., ::2])
    k, v, sl = _append_restated(host.k_cache, host.v_cache, host.page_table, host.seq_lens, 16, nk, nv)
    torch.cuda.synchronize()
    assert torch.equal(_bytes(cache.k_cache), _bytes(k)) and torch.equal(_bytes(cache.v_cache), _bytes(v))
    assert torch.equal(cache.seq_lens.cpu(), sl)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hkv,d,P", [(2, 128, 16), (4, 64, 32), (2, 36, 8)])
def test_append_keeps_quantised_copy_equal_to_full_requantisation(mode, dtype, hkv, d, P):
    lens = [0, P - 1, 2 * P, 45]
    host = _cache(lens, hkv, d, P, dtype, seed=7 + d)
    cache = _to(host, DEV)
    qcache, scales = quantize_cache(cache, mode=mode)
    g = torch.Generator().manual_seed(9)
    for step in range(4):
        print(f"append+requant {mode} {dtype} Hkv{hkv} D{d} P{P} step {step}", flush=True)
        # Large new rows so the appended token usually sets its page's absmax.
        nk = (torch.randn(len(lens), hkv, d, generator=g) * (1 + 3 * (step % 2))).to(dtype)
        nv = (torch.randn(len(lens), hkv, d, generator=g) * (1 + 3 * (step % 2))).to(dtype)
        append_tokens(cache, nk.to(DEV), nv.to(DEV), quantized=(qcache, scales))
        torch.cuda.synchronize()
        assert qcache.seq_lens is cache.seq_lens
        wk, wsk = quant_ref.quantize_pages(cache.k_cache.cpu(), mode)
        wv, wsv = quant_ref.quantize_pages(cache.v_cache.cpu(), mode)
        assert torch.equal(scales.k.cpu(), wsk) and torch.equal(scales.v.cpu(), wsv)
        _assert_codes_equal(qcache.k_cache, wk, "K copy")
        _assert_codes_equal(qcache.v_cache, wv, "V copy")


@pytest.mark.parametrize("mode", MODES)
def test_append_sequences_sharing_a_page(mode):
    """Two sequences whose next tokens land in different slots of one
    physical page: both rows are written and the page's requantisation sees
    both (it runs after every row of the call is in place)."""
    P, hkv, d = 16, 2, 64
    g = torch.Generator().manual_seed(21)
    k = torch.randn(4, P, hkv, d, generator=g).half()
    v = torch.randn(4, P, hkv, d, generator=g).half()
    pt = torch.tensor([[2, 0], [2, 1]], dtype=torch.int32)  # logical block 0 of both -> page 2
    sl = torch.tensor([3, 9], dtype=torch.int32)
    cache = PagedKVCache(k.to(DEV), v.to(DEV), pt.to(DEV), sl.to(DEV), P)
    qcache, scales = quantize_cache(cache, mode=mode)
    nk = torch.randn(2, hkv, d, generator=g).half() * 50
    nv = torch.randn(2, hkv, d, generator=g).half() * 50
    append_tokens(cache, nk.to(DEV), nv.to(DEV), quantized=(qcache, scales))
    torch.cuda.synchronize()
    wk, wv, wsl = _append_restated(k, v, pt, sl, P, nk, nv)
    assert torch.equal(_bytes(cache.k_cache), _bytes(wk)) and torch.equal(cache.seq_lens.cpu(), wsl)
    qk_want, sk_want = quant_ref.quantize_pages(wk, mode)
    assert torch.equal(scales.k.cpu(), sk_want)
    _assert_codes_equal(qcache.k_cache, qk_want, "shared page")


def test_append_bounds():
    """validate=True raises before any launch; validate=False skips the
    out-of-range entry on the device and leaves its length."""
    P = 16
    host = _cache([5, 30], 2, 64, P, torch.float16, seed=3)
    host.seq_lens[1] = host.capacity  # full
    cache = _to(host, DEV)
    nk = torch.randn(2, 2, 64).half()
    nv = torch.randn(2, 2, 64).half()
    with pytest.raises(AssertionError, match="capacity"):
        append_tokens(cache, nk.to(DEV), nv.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(cache.seq_lens.cpu(), host.seq_lens) and torch.equal(cache.k_cache.cpu(), host.k_cache)
    append_tokens(cache, nk.to(DEV), nv.to(DEV), validate=False)
    torch.cuda.synchronize()
    assert cache.seq_lens.cpu().tolist() == [6, host.capacity]
    want_k = host.k_cache.clone()
    want_k[int(host.page_table[0, 0]), 5] = nk[0]
    assert torch.equal(cache.k_cache.cpu(), want_k)
    # A page id outside the pool is reported with validation on ...
    bad = _to(_cache([5, 7], 2, 64, P, torch.float16, seed=3), DEV)
    bad.page_table[1, 0] = bad.num_pages
    with pytest.raises(AssertionError, match="outside"):
        append_tokens(bad, nk.to(DEV), nv.to(DEV))
    # ... and skipped on the device without it.
    before = bad.k_cache.clone()
    append_tokens(bad, nk.to(DEV), nv.to(DEV), validate=False)
    torch.cuda.synchronize()
    assert bad.seq_lens.cpu().tolist() == [6, 7]
    assert torch.equal(bad.k_cache[int(bad.page_table[0, 0]), 5].cpu(), nk[0])
    changed = (bad.k_cache != before).flatten(1).any(dim=1).nonzero().flatten().tolist()
    assert changed == [int(bad.page_table[0, 0])]
