"""GPU tests of the per-launch kernel choice (ABI field ``kernel``) and of
the gfx950 tuned-config store routing ``config=None`` launches.

A launch forced through the config reaches the library as the ``kernel``
field (the library reads no environment); the library's own choice must be
bit-identical to the forced kernel it picks, and a launch taken from the
store must be bit-identical to the same config passed explicitly.  Parity against the fp32 oracle (2e-3,
tests/_parity.py) is checked once per kernel.
"""

from __future__ import annotations

import json

import pytest
import torch

from _parity import assert_parity, make_paged, make_query, make_varlen
from flashattntile_amd import (PagedKVCache, paged_decode_attention, paged_decode_attention_multi,
                               paged_prefill_attention, prefill_attention)
from flashattntile_amd import autotune as at
from oracle.reference import ref_attention_paged, ref_attention_paged_prefill, ref_attention_varlen

pytestmark = pytest.mark.gpu
DEV = "cuda"
LENS = [1, 17, 255, 1000, 4096]


def _decode_case(lens, h, hk, dtype, seed):
    k, v, pt, sl = make_paged(lens, hk, 128, 16, dtype, seed=seed, device=DEV)
    return make_query(len(lens), h, 128, dtype, seed=seed + 1, device=DEV), PagedKVCache(k, v, pt, sl, 16)


@pytest.mark.parametrize("h,hk", [(32, 8), (8, 2), (32, 1)])
def test_decode_kernel_field_selects_the_kernel(h, hk):
    """Each forced kernel passes parity, and the library's own choice is
    bit-identical to one of them (VALU for groups below 8, MFMA from 8)."""
    label = f"decode kernel field H{h}/{hk}"
    print(label, flush=True)
    q, cache = _decode_case(LENS, h, hk, torch.bfloat16, seed=h + hk)
    ref = ref_attention_paged(q.cpu(), cache.k_cache.cpu(), cache.v_cache.cpu(), cache.page_table.cpu(),
                              cache.seq_lens.cpu(), return_fp32=True)
    outs = {kern: paged_decode_attention(q, cache, config={"split_k": 4, "kernel": kern})
            for kern in ("valu", "mfma", "generic")}
    auto = paged_decode_attention(q, cache, config={"split_k": 4})
    torch.cuda.synchronize()
    for kern, out in outs.items():
        assert_parity(out, ref, label=f"{label} {kern}")
    assert torch.equal(auto, outs["valu" if h // hk < 8 else "mfma"]), label


def test_multi_token_decode_kernel_choice():
    print("multi-token decode kernel choice", flush=True)
    k, v, pt, sl = make_paged([40, 300], 8, 128, 16, torch.float16, seed=3, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, 16)
    q = torch.randn(2, 3, 32, 128, generator=torch.Generator().manual_seed(4)).half().to(DEV)
    a = paged_decode_attention_multi(q, cache, config={"split_k": 2, "kernel": "mfma"})
    b = paged_decode_attention_multi(q, cache, config={"split_k": 2})
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="one query per sequence"):
        paged_decode_attention_multi(q, cache, config={"split_k": 2, "kernel": "valu"})


@pytest.mark.parametrize("kern", ["pingpong", "wide", "4wave", "4wave_split"])
def test_prefill_kernel_field_selects_the_kernel(kern):
    """A forced prefill kernel passes parity, packed and paged (the wide
    kernel through staged copies of the paged K/V), and the library's own
    choice for this shape (ping-pong: 384 blocks of 256 rows) is
    bit-identical to forcing it."""
    label = f"prefill kernel={kern}"
    print(label, flush=True)
    lens = [1, 255, 1000]
    q, k, v, cu = make_varlen(lens, 32, 8, 128, torch.float16, seed=11, device=DEV)
    out_cfg = prefill_attention(q, k, v, cu, cu, max(lens), max(lens), causal=True, config={"kernel": kern})
    auto = prefill_attention(q, k, v, cu, cu, max(lens), max(lens), causal=True, config={})
    torch.cuda.synchronize()
    if kern == "pingpong":
        assert torch.equal(out_cfg, auto), label
    ref = ref_attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), causal=True, return_fp32=True)
    assert_parity(out_cfg, ref, label=label)
    kc, vc, pt, sl = make_paged(lens, 8, 128, 16, torch.float16, seed=12, device=DEV)
    cache = PagedKVCache(kc, vc, pt, sl, 16)
    # wide: the paged launch runs on packed copies of the used K/V rows, in the
    # staging workspace the wrapper allocates (without it the library refuses,
    # tests/test_abi.py)
    p_cfg = paged_prefill_attention(q, cache, cu, max(lens), config={"kernel": kern})
    torch.cuda.synchronize()
    ref_p = ref_attention_paged_prefill(q.cpu(), kc.cpu(), vc.cpu(), pt.cpu(), sl.cpu(), cu.cpu(), causal=True,
                                        return_fp32=True)
    assert_parity(p_cfg, ref_p, label=f"paged {label}")


def test_store_routes_config_none_launches(tmp_path, monkeypatch):
    print("tuned store routes config=None launches", flush=True)
    path = tmp_path / "store.json"
    monkeypatch.setenv("FAT_TUNED_CONFIGS", str(path))
    q, cache = _decode_case(LENS, 32, 8, torch.float16, seed=21)
    total = sum(-(-n // 16) for n in LENS)
    sig = at.decode_signature(len(LENS), 32, 8, 128, 16, max(LENS), total, torch.float16)
    for cfg in ({"split_k": 3, "pages_per_split": 0, "num_warps": 8, "kernel": "mfma"},
                {"split_k": 5, "pages_per_split": 16, "num_warps": 4, "kernel": "valu"}):
        at.save_best("decode", sig, cfg)
        got = paged_decode_attention(q, cache)
        want = paged_decode_attention(q, cache, config=dict(cfg))
        torch.cuda.synchronize()
        assert torch.equal(got, want), cfg
    lens = [1, 255, 1000]
    qp, k, v, cu = make_varlen(lens, 32, 8, 128, torch.bfloat16, seed=22, device=DEV)
    psig = at.prefill_signature(3, 32, 8, 128, 1000, 1000, True)
    for kern in ("pingpong", "wide", "4wave", "4wave_split"):
        at.save_best("prefill", psig, {"kernel": kern})
        got = prefill_attention(qp, k, v, cu, cu, 1000, 1000, causal=True)
        want = prefill_attention(qp, k, v, cu, cu, 1000, 1000, causal=True, config={"kernel": kern})
        torch.cuda.synchronize()
        assert torch.equal(got, want), kern


def test_committed_store_entry_runs(monkeypatch):
    """A committed decode entry (B8 ctx1024 fp16, from a tuning run on
    MI355X) routes config=None to its stored launch, which passes parity."""
    data = json.loads(at.TUNED_CONFIGS_PATH.read_text())
    sig = "B8_H32_Hkv8_D128_P16_L1024_fp16"
    entry = data["configs"].get(f"decode:{sig}")
    if entry is None:
        pytest.skip("no tuned entry for B8 ctx1024 in the committed store")
    print(f"committed store entry {sig} {entry['config']}", flush=True)
    monkeypatch.setenv("FAT_TUNED_CONFIGS", str(at.TUNED_CONFIGS_PATH))
    q, cache = _decode_case([1024] * 8, 32, 8, torch.float16, seed=31)
    got = paged_decode_attention(q, cache)
    want = paged_decode_attention(q, cache, config=dict(entry["config"]))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    ref = ref_attention_paged(q.cpu(), cache.k_cache.cpu(), cache.v_cache.cpu(), cache.page_table.cpu(),
                              cache.seq_lens.cpu(), return_fp32=True)
    assert_parity(got, ref, label=f"store {sig}")
