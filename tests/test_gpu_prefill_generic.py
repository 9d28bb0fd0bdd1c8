"""GPU parity of the generic (fp32 VALU) prefill kernel, prefill_generic.hip.

It takes what the MFMA prefill kernels do not: fp32 inputs (the reference
sends them to its fp32 torch path, flashattn_tile/kernels/prefill.py:286-290)
and head_dim 16 or 512, packed and paged; forced with ``kernel="generic"``
it also runs the fp16/bf16 shapes the MFMA kernels take.

Oracle: the fp32 restatement of the reference (oracle/reference.py).  fp32
outputs must be within 1e-5 of it relative to max(1, |ref|): only the order
of the fp32 sums and the exp2 of the scores differ, while rounding K, V or
P to fp16 or bf16 anywhere on the path would move N(0,1) data by up to
5e-4.  fp16/bf16 outputs use the north star's 2e-3 (tests/_parity.py).
"""

from __future__ import annotations

import pytest
import torch

from _parity import assert_parity, force_prefill_knobs, make_paged, make_varlen
from flashattntile_amd import PagedKVCache, prefill_attention
from flashattntile_amd.kernels.prefill import paged_prefill_attention
from oracle.reference import ref_attention_paged_prefill, ref_attention_varlen

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODD_LENS = [1, 17, 255, 1000]
FP32_RTOL = 1e-5


def _check(out, ref, label, rtol=FP32_RTOL):
    if out.dtype != torch.float32:
        assert_parity(out, ref, label=label)
        return
    o = out.float().cpu()
    err = (o - ref).abs()
    rel = (err / ref.abs().clamp_min(1.0)).max().item()
    print(f"{label} max_abs={err.max().item():.3e} max_rel={rel:.3e}", flush=True)
    assert torch.isfinite(o).all(), f"{label}: non-finite output"
    assert rel <= rtol, f"{label}: {rel:.3e} > {rtol} relative to max(1, |ref|)"


def _ref_varlen(q, k, v, cu_q, cu_k, causal, scale=None):
    return ref_attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=causal,
                                softmax_scale=scale, return_fp32=True)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("h,hk", [(8, 8), (8, 2)])
@pytest.mark.parametrize("d", [16, 32, 64, 128, 256, 512])
def test_fp32_prefill_matches_oracle(d, h, hk, causal):
    label = f"generic prefill fp32 D{d} H{h}/{hk} causal={causal}"
    print(label, flush=True)
    q, k, v, cu = make_varlen(ODD_LENS, h, hk, d, torch.float32, seed=d + h + hk, device=DEV)
    out = prefill_attention(q, k, v, cu, cu, max(ODD_LENS), max(ODD_LENS), causal=causal)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == torch.float32
    _check(out, _ref_varlen(q, k, v, cu, cu, causal), label)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [16, 512])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_head_dim_16_and_512_match_oracle(dtype, d, causal):
    """head_dim 16 and 512 have no MFMA prefill kernel: the automatic choice
    runs the generic one."""
    label = f"generic prefill {dtype} D{d} H32/8 causal={causal}"
    print(label, flush=True)
    q, k, v, cu = make_varlen(ODD_LENS, 32, 8, d, dtype, seed=d + 5, device=DEV)
    out = prefill_attention(q, k, v, cu, cu, max(ODD_LENS), max(ODD_LENS), causal=causal)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    _check(out, _ref_varlen(q, k, v, cu, cu, causal), label)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_forced_generic_on_mfma_shapes(dtype, d, causal, monkeypatch):
    force_prefill_knobs(monkeypatch, kernel="generic")
    label = f"generic prefill forced {dtype} D{d} H8/1 causal={causal}"
    print(label, flush=True)
    q, k, v, cu = make_varlen(ODD_LENS, 8, 1, d, dtype, seed=d + 9, device=DEV)
    out = prefill_attention(q, k, v, cu, cu, max(ODD_LENS), max(ODD_LENS), causal=causal)
    torch.cuda.synchronize()
    _check(out, _ref_varlen(q, k, v, cu, cu, causal), label)


def test_fp32_queries_shorter_than_keys_and_custom_scale():
    """Bottom-right causal alignment with q_len < kv_len (a chunk after a
    prefix) and a non-default softmax scale; separate K and V sequences.
    Scale 0.3 makes the logits 3.4x those of the default 128^-0.5, and the
    fp32 rounding of a logit (kernel and oracle alike) grows with it, so the
    fp32 bound grows by the same factor."""
    print("generic prefill fp32 q_len < kv_len, scale 0.3", flush=True)
    lq, lk = [5, 64, 200, 1], [40, 64, 777, 300]
    g = torch.Generator().manual_seed(21)
    q = torch.randn(sum(lq), 16, 128, generator=g).to(DEV)
    k = torch.randn(sum(lk), 4, 128, generator=g).to(DEV)
    v = torch.randn(sum(lk), 4, 128, generator=g).to(DEV)
    cq = torch.tensor([0] + torch.cumsum(torch.tensor(lq), 0).tolist(), dtype=torch.int32, device=DEV)
    ck = torch.tensor([0] + torch.cumsum(torch.tensor(lk), 0).tolist(), dtype=torch.int32, device=DEV)
    for causal in (True, False):
        out = prefill_attention(q, k, v, cq, ck, max(lq), max(lk), causal=causal, softmax_scale=0.3)
        torch.cuda.synchronize()
        _check(out, _ref_varlen(q, k, v, cq, ck, causal, scale=0.3), f"fp32 lq<lk causal={causal}",
               rtol=FP32_RTOL * 0.3 * 128 ** 0.5)


# (kv_len, q_len): sequences with no queries, with and without keys.
EMPTY_Q = [(0, 0), (40, 0), (17, 17), (0, 0), (300, 300), (129, 0), (64, 1), (700, 513), (9, 0)]


@pytest.mark.parametrize("causal", [True, False])
def test_fp32_sequences_without_queries(causal):
    print(f"generic prefill fp32 empty-query entries causal={causal}", flush=True)
    g = torch.Generator().manual_seed(3)
    lk = [p[0] for p in EMPTY_Q]
    lq = [p[1] for p in EMPTY_Q]
    q = torch.randn(sum(lq), 8, 64, generator=g).to(DEV)
    k = torch.randn(sum(lk), 2, 64, generator=g).to(DEV)
    v = torch.randn(sum(lk), 2, 64, generator=g).to(DEV)
    cq = torch.tensor([0] + torch.cumsum(torch.tensor(lq), 0).tolist(), dtype=torch.int32, device=DEV)
    ck = torch.tensor([0] + torch.cumsum(torch.tensor(lk), 0).tolist(), dtype=torch.int32, device=DEV)
    out = prefill_attention(q, k, v, cq, ck, max(lq), max(lk), causal=causal)
    torch.cuda.synchronize()
    _check(out, _ref_varlen(q, k, v, cq, ck, causal), f"fp32 empty-q causal={causal}")


def test_fp32_refuses_the_mfma_kernels(monkeypatch):
    force_prefill_knobs(monkeypatch, kernel="pingpong")
    q, k, v, cu = make_varlen([64], 8, 8, 64, torch.float32, device=DEV)
    with pytest.raises(RuntimeError, match="fp32 runs on the generic prefill kernel only"):
        prefill_attention(q, k, v, cu, cu, 64, 64)


CHUNKS = [(1000, 1000), (300, 77), (129, 1), (64, 64), (517, 200), (5, 3), (40, 0)]


def _paged_case(h, hk, d, P, dtype, seed):
    lens_k = [c[0] for c in CHUNKS]
    lens_q = [c[1] for c in CHUNKS]
    k, v, pt, sl = make_paged(lens_k, hk, d, P, dtype, seed=seed, device=DEV)
    g = torch.Generator().manual_seed(seed + 100)
    q = torch.randn(sum(lens_q), h, d, generator=g).to(dtype).to(DEV)
    cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens_q), 0).tolist(), dtype=torch.int32, device=DEV)
    return q, PagedKVCache(k, v, pt, sl, P), cu, max(lens_q)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("P", [1, 16])
@pytest.mark.parametrize("dtype,d", [(torch.float32, 128), (torch.float32, 16), (torch.float16, 512),
                                     (torch.bfloat16, 16)])
def test_paged_generic_matches_oracle(dtype, d, P, causal):
    """Paged (chunked) prefill on the generic kernel: pages scattered by a
    seeded permutation, slots past each sequence end poisoned."""
    label = f"generic paged prefill {dtype} D{d} P{P} causal={causal}"
    print(label, flush=True)
    q, cache, cu, mq = _paged_case(8, 2, d, P, dtype, seed=d + P)
    out = paged_prefill_attention(q, cache, cu, mq, causal=causal)
    torch.cuda.synchronize()
    ref = ref_attention_paged_prefill(q.cpu(), cache.k_cache.cpu(), cache.v_cache.cpu(), cache.page_table.cpu(),
                                      cache.seq_lens.cpu(), cu.cpu(), causal=causal, return_fp32=True)
    _check(out, ref, label)
