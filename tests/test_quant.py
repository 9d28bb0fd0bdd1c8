"""Quantisation format: product helpers vs the oracle restatement and KATs."""

from __future__ import annotations

import math

import pytest
import torch

from flashattntile_amd import quant
from flashattntile_amd.paging import allocate, append_tokens
from oracle import quant_ref

FP8 = getattr(torch, "float8_e4m3fn", None)


def test_fp8_table_matches_torch_exhaustively():
    """All 256 OCP e4m3fn codes: bit-field decoding == torch's conversion."""
    table = quant_ref.fp8_table()
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(FP8).float()
    same = (table == codes) | (torch.isnan(table) & torch.isnan(codes))
    assert bool(same.all())
    assert table[0x7E].item() == 448.0 and table[0x08].item() == 2.0 ** -6 and table[0x01].item() == 2.0 ** -9
    assert math.isnan(table[0x7F].item()) and math.isnan(table[0xFF].item())


def test_int8_kats():
    # One page, one head: absmax 2.54 -> scale 0.02; values map to integers.
    x = torch.tensor([2.54, -1.27, 0.01, 0.03, -0.05, 0.0, 0.5, -2.54]).view(1, 8, 1, 1)
    q, s = quant_ref.quantize_pages(x, "int8")
    assert s.shape == (1, 1)
    assert abs(s.item() - 2.54 / 127) < 1e-9
    # 0.01/0.02 = 0.5 -> 0 (half to even), 0.03/0.02 = 1.5 -> 2, -0.05/0.02 = -2.5 -> -2
    assert q.view(-1).tolist() == [127, -64, 0, 2, -2, 0, 25, -127]
    # All-zero page: scale floors at 1e-8 and everything quantises to 0.
    qz, sz = quant_ref.quantize_pages(torch.zeros(2, 4, 3, 2), "int8")
    assert torch.all(sz == 1e-8) and torch.all(qz == 0)


def test_fp8_kats():
    x = torch.tensor([448.0, -448.0, 1.0, 0.0]).view(1, 4, 1, 1) * 0.5
    q, s = quant_ref.quantize_pages(x, "float8_e4m3fn")
    assert abs(s.item() - 224.0 / 448.0) < 1e-12
    assert q.view(torch.uint8).view(-1).tolist() == [0x7E, 0xFE, 0x38, 0x00]  # 448, -448, 1.0, 0


@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_product_quantise_equals_oracle(mode, out_dtype):
    g = torch.Generator().manual_seed(3)
    k = torch.randn(6, 16, 2, 64, generator=g).to(torch.float16)
    v = torch.randn(6, 16, 2, 64, generator=g).to(torch.float16)
    qk, qv, sk, sv, info = quant.quantize_kv_pages(k, v, mode=mode)
    ok, osk = quant_ref.quantize_pages(k, mode)
    ov, osv = quant_ref.quantize_pages(v, mode)
    assert info["mode"] == mode and sk.shape == (6, 2)
    assert torch.equal(qk.view(torch.uint8), ok.view(torch.uint8))
    assert torch.equal(qv.view(torch.uint8), ov.view(torch.uint8))
    assert torch.equal(sk, osk) and torch.equal(sv, osv)
    dk, dv = quant.dequantize_kv_pages(qk, qv, sk, sv, out_dtype=out_dtype)
    assert torch.equal(dk, quant_ref.dequantize_pages(ok, osk, out_dtype))
    assert torch.equal(dv, quant_ref.dequantize_pages(ov, osv, out_dtype))
    # Error bound of the format: |x - deq| <= scale/2 (int8) or half an fp8 ulp
    # (<= 16 * scale at the top binade), plus the output dtype's rounding.
    err = (dk.float() - k.float()).abs()
    rel = {torch.float16: 1e-3, torch.bfloat16: 4e-3, torch.float32: 1e-6}[out_dtype]
    bound = sk[:, None, :, None] * (0.5 if mode == "int8" else 16.0) + rel * k.float().abs()
    assert torch.all(err <= bound)


def test_quantize_cache_roundtrip_shapes():
    cache = allocate(2, 20, 2, 16, 16, dtype=torch.float32)
    for _ in range(20):
        append_tokens(cache, torch.randn(2, 2, 16), torch.randn(2, 2, 16))
    qc, scales = quant.quantize_cache(cache, mode="int8")
    assert qc.k_cache.dtype == torch.int8 and scales.k.shape == (cache.num_pages, 2)
    assert scales.as_dict()["granularity"] == "per_page_per_head"
    deq = quant.dequantize_cache(qc, scales, out_dtype=torch.float32)
    assert deq.k_cache.shape == cache.k_cache.shape
    assert (deq.k_cache - cache.k_cache).abs().max() <= scales.k.max() / 2 + 1e-6


def test_bytes_per_token_kats():
    """results/numerics.json:43-47 of the reference: 4100 vs 2052 bytes."""
    assert quant.kv_bytes_per_token(8, 128, "fp16", 16) == 4100.0
    assert quant.kv_bytes_per_token(8, 128, "int8", 16) == 2052.0
    assert quant.kv_bytes_per_token(8, 128, "fp8", 16) == 2052.0
    assert quant.kv_bytes_per_token(8, 128, "int8", 16) < quant.kv_bytes_per_token(8, 128, "fp16", 16) / 1.9


def test_modes_and_errors():
    assert "int8" in quant.available_quant_modes()
    assert quant.default_quant_mode() in ("int8", "float8_e4m3fn")
    with pytest.raises(ValueError, match="unknown quantisation mode"):
        quant.quantize_kv_pages(torch.zeros(1, 2, 1, 2), torch.zeros(1, 2, 1, 2), mode="int4")
    with pytest.raises(ValueError, match="float cache"):
        quant.quantize_kv_pages(torch.zeros(1, 2, 1, 2, dtype=torch.int8), torch.zeros(1, 2, 1, 2, dtype=torch.int8))
    with pytest.raises(ValueError, match="scale_k shape"):
        quant.dequantize_kv_pages(torch.zeros(2, 2, 1, 2, dtype=torch.int8), torch.zeros(2, 2, 1, 2, dtype=torch.int8),
                                  torch.ones(3, 1), torch.ones(3, 1))


def _nearest_even_fp8(y: float, table: torch.Tensor) -> int:
    """Brute force: among the finite e4m3fn codes with the sign of y (rounding
    keeps the sign, also for results of zero), the one nearest to y; a tie
    goes to the even code (round to nearest even)."""
    sign = 0x80 if math.copysign(1.0, y) < 0 else 0x00
    same = [c for c in range(256) if (c & 0x80) == sign and not math.isnan(table[c].item())]
    best = min(abs(table[c].item() - y) for c in same)
    cands = [c for c in same if abs(table[c].item() - y) == best]
    assert len(cands) <= 2
    return min(cands, key=lambda c: c & 1)


def test_oracle_fp8_cast_is_round_to_nearest_even():
    """The oracle's fp8 codes (torch's cast) against a brute-force
    nearest-even search over the 256-code table, at and beside every rounding
    midpoint.  The GPU tests then hold the gfx950 conversion to the oracle."""
    table = quant_ref.fp8_table()
    pos = table[:0x7F].double()
    mids = ((pos[1:] + pos[:-1]) / 2).float()
    vals = torch.cat([pos.float(), mids, torch.nextafter(mids, mids - 1), torch.nextafter(mids, mids + 1),
                      torch.tensor([2.0 ** -10, 2.0 ** -11, 3 * 2.0 ** -11])])
    vals = torch.cat([vals, -vals])
    x = torch.zeros(vals.numel() + 1)
    x[0] = 448.0  # absmax 448: scale exactly 1
    x[1:] = vals
    q, s = quant_ref.quantize_pages(x.view(1, -1, 1, 1), "float8_e4m3fn")
    assert s.item() == 1.0
    codes = q.view(torch.uint8).view(-1)[1:].tolist()
    for y, c in zip(vals.tolist(), codes):
        assert c == _nearest_even_fp8(y, table), (y, hex(c))


@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
def test_append_with_quantised_copy_cpu(mode):
    """append_tokens(..., quantized=(qcache, scales)) keeps the copy equal to
    quantize_cache of the updated cache (CPU tensors: the torch path)."""
    g = torch.Generator().manual_seed(4)
    cache = allocate(3, 40, 2, 32, 8, dtype=torch.float16)
    for _ in range(5):
        append_tokens(cache, torch.randn(3, 2, 32, generator=g).half(), torch.randn(3, 2, 32, generator=g).half())
    qc, scales = quant.quantize_cache(cache, mode=mode)
    for step in range(10):
        nk = (torch.randn(3, 2, 32, generator=g) * (1 + 4 * (step % 2))).half()
        nv = torch.randn(3, 2, 32, generator=g).half()
        append_tokens(cache, nk, nv, quantized=(qc, scales))
        full, fs = quant.quantize_cache(cache, mode=mode)
        assert torch.equal(qc.k_cache.view(torch.uint8), full.k_cache.view(torch.uint8))
        assert torch.equal(qc.v_cache.view(torch.uint8), full.v_cache.view(torch.uint8))
        assert torch.equal(scales.k, fs.k) and torch.equal(scales.v, fs.v)
    assert qc.seq_lens is cache.seq_lens and cache.seq_lens.tolist() == [15, 15, 15]
    with pytest.raises(AssertionError, match="quantised pages"):
        append_tokens(cache, nk, nv, quantized=(cache, scales))
