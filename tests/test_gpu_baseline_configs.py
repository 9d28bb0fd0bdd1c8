"""Parity at BASELINE.json's full sizes, through the launches the product
actually makes.

Every test here runs with ``FAT_TUNED_CONFIGS`` pointing at the committed
gfx950 store (``flashattntile_amd/tuned_configs_gfx950.json``), so a
``config=None`` call takes the stored launch for its shape and the
heuristic otherwise -- exactly what a serving process and ``bench.py`` do.

* every decode and prefill entry of the committed store is run at its own
  shape (the configs[1] B x ctx sweep, configs[3] int8/fp8 B128 ctx16384,
  configs[4] B1 ctx131072, MQA, D64, bf16, 4-token decode, configs[2]
  prefill lengths and paged prefill); a few sequences (decode) or a head
  subset (prefill) are checked against the fp32 oracle -- the reference's
  own sampling of big shapes, tests/test_kernel_correctness.py:186-196;
* configs[0], the reference's CPU workload (B4, ctx ~ U[64, 512], a
  256-page pool, seeded permutation), is checked whole;
* configs[4]'s 64-sequence log-uniform batch and its MQA / D64 / page 32 and
  64 variants run with ``config=None``.

Pools are generated on the device (seeded) and only the pages of the checked
sequences are copied to the host for the oracle.  int8/fp8 pools are
quantised by the product's ``quantize_kv_pages`` (bit-exact against the
oracle's quantiser in test_gpu_kvwrite.py) and the oracle attends over the
codes dequantised to q.dtype by ``oracle.quant_ref``.  Tolerance: 2e-3 on the
kernel's result before its final rounding (tests/_parity.py).
"""

from __future__ import annotations

import math
import re

import pytest
import torch

from _parity import assert_parity
from flashattntile_amd import (PagedKVCache, paged_decode_attention, paged_decode_attention_fp8,
                               paged_decode_attention_multi, paged_prefill_attention, prefill_attention)
from flashattntile_amd import autotune as at
from flashattntile_amd.quant import quantize_kv_pages
from oracle import quant_ref
from oracle.reference import ref_attention_paged, ref_attention_paged_prefill, ref_attention_varlen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _store_entries(kind: str) -> list[str]:
    import json

    data = json.loads(at.TUNED_CONFIGS_PATH.read_text())
    return sorted(e["signature"] for e in data["configs"].values() if e["kind"] == kind)


@pytest.fixture(autouse=True)
def committed_store(monkeypatch):
    monkeypatch.setenv("FAT_TUNED_CONFIGS", str(at.TUNED_CONFIGS_PATH))
    yield
    torch.cuda.empty_cache()


_DECODE_SIG = re.compile(r"B(\d+)_H(\d+)_Hkv(\d+)_D(\d+)_P(\d+)_L(\d+)_(fp16|bf16|int8|fp8)(?:_T(\d+))?(_ragged)?$")


def _table(lens, page, seed):
    """Seeded permutation of a pool holding exactly the batch's pages."""
    g = torch.Generator().manual_seed(seed)
    pages_per = [max(1, -(-n // page)) for n in lens]
    perm = torch.randperm(sum(pages_per), generator=g).to(torch.int32)
    table = torch.zeros(len(lens), max(pages_per), dtype=torch.int32)
    at_ = 0
    for b, n in enumerate(pages_per):
        table[b, :n] = perm[at_:at_ + n]
        at_ += n
    return table, sum(pages_per)


def _pool(num_pages, page, hkv, d, dtype, seed):
    """K, V pools ~ N(0, 1) generated on the device in fp32 chunks."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    out = []
    for _ in range(2):
        t = torch.empty(num_pages, page, hkv, d, dtype=dtype, device=DEV)
        step = max(1, (1 << 27) // (page * hkv * d))
        for s in range(0, num_pages, step):
            e = min(num_pages, s + step)
            t[s:e] = torch.randn(e - s, page, hkv, d, generator=gen, device=DEV).to(dtype)
        out.append(t)
    return out


def _quant_pool(num_pages, page, hkv, d, mode, seed):
    """int8 / fp8 pools and their scales, quantised chunk by chunk."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    qdt = torch.int8 if mode == "int8" else torch.float8_e4m3fn
    codes = [torch.empty(num_pages, page, hkv, d, dtype=qdt, device=DEV) for _ in range(2)]
    scales = [torch.empty(num_pages, hkv, dtype=torch.float32, device=DEV) for _ in range(2)]
    step = max(1, (1 << 26) // (page * hkv * d))
    for s in range(0, num_pages, step):
        e = min(num_pages, s + step)
        kf = torch.randn(e - s, page, hkv, d, generator=gen, device=DEV)
        vf = torch.randn(e - s, page, hkv, d, generator=gen, device=DEV)
        qk, qv, sk, sv, _ = quantize_kv_pages(kf, vf, mode)
        codes[0][s:e], codes[1][s:e], scales[0][s:e], scales[1][s:e] = qk, qv, sk, sv
    return codes, scales


def _sequence_ref(q_rows, cache, b, qdtype, scales=None, q_len=1, scale=None):
    """fp32 oracle of sequence b alone: its pages gathered to the host under a
    compact table.  ``q_rows``: its query ([H, D], or [T, H, D])."""
    n = int(cache.seq_lens[b])
    pages = cache.page_table[b, : -(-n // cache.page_size)].long()
    k = cache.k_cache[pages].cpu()
    v = cache.v_cache[pages].cpu()
    if scales is not None:
        k = quant_ref.dequantize_pages(k, scales[0][pages].cpu(), qdtype)
        v = quant_ref.dequantize_pages(v, scales[1][pages].cpu(), qdtype)
    table = torch.arange(len(pages), dtype=torch.int32).unsqueeze(0)
    lens = torch.tensor([n], dtype=torch.int32)
    if q_len == 1:
        return ref_attention_paged(q_rows.unsqueeze(0).cpu(), k, v, table, lens, softmax_scale=scale,
                                   return_fp32=True)[0]
    cu = torch.tensor([0, q_len], dtype=torch.int32)
    return ref_attention_paged_prefill(q_rows.cpu(), k, v, table, lens, cu, causal=True, softmax_scale=scale,
                                       return_fp32=True)


def _check_rows(out, q, cache, rows, label, scales=None, q_len=1):
    for b in rows:
        ref = _sequence_ref(q[b], cache, b, q.dtype, scales=scales, q_len=q_len)
        assert_parity(out[b], ref, label=f"{label} seq{b}")


def _rows(batch):
    return sorted({0, batch // 2, batch - 1})


@pytest.mark.parametrize("sig", _store_entries("decode"))
def test_committed_decode_entry_at_full_size(sig):
    """A decode entry of the committed store at its own shape, launched with
    ``config=None`` (the stored launch), checked on 2-3 sequences."""
    m = _DECODE_SIG.match(sig)
    assert m, sig
    B, H, HKV, D, P, L = (int(m.group(i)) for i in range(1, 7))
    tag, T = m.group(7), int(m.group(8) or 1)
    seq = [L] * B
    if m.group(9):  # ragged: the tuner's only ragged shape is the skewed benchmark batch
        from flashattntile_amd.tune import skewed_lens
        seq = skewed_lens()
        assert (B, L) == (len(seq), max(seq)), f"{sig}: not the tuner's skewed batch"
    label = f"store decode {sig}"
    print(label, flush=True)
    stored = at.best_config("decode", sig)
    table, num_pages = _table(seq, P, seed=B + L)
    lens = torch.tensor(seq, dtype=torch.int32)
    qdtype = torch.bfloat16 if tag == "bf16" else torch.float16
    g = torch.Generator().manual_seed(L + H)
    shape = (B, T, H, D) if T > 1 else (B, H, D)
    q = torch.randn(shape, generator=g).to(qdtype).to(DEV)
    scales = None
    if tag in ("int8", "fp8"):
        (k, v), scales = _quant_pool(num_pages, P, HKV, D, tag if tag == "int8" else "float8_e4m3fn", seed=B * L)
    else:
        k, v = _pool(num_pages, P, HKV, D, qdtype, seed=B * L)
    cache = PagedKVCache(k, v, table.to(DEV), lens.to(DEV), P)
    if T > 1:
        out = paged_decode_attention_multi(q, cache)
        want = paged_decode_attention_multi(q, cache, config=dict(stored))
    elif scales is not None:
        sc = {"k": scales[0], "v": scales[1]}
        out = paged_decode_attention_fp8(q, cache, sc)
        want = paged_decode_attention_fp8(q, cache, sc, config=dict(stored))
    else:
        out = paged_decode_attention(q, cache)
        want = paged_decode_attention(q, cache, config=dict(stored))
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"{label}: config=None did not take the stored launch {stored}"
    _check_rows(out, q, cache, _rows(B), label, scales=scales, q_len=T)


@pytest.mark.parametrize("sig", _store_entries("prefill") + _store_entries("prefill_paged"))
def test_committed_prefill_entry_at_full_size(sig):
    """A prefill entry of the committed store (one causal sequence of its
    length, 32/8 heads, D128; paged: page 16) with ``config=None``, fp16 and
    bf16, checked against the oracle on two query-head groups (8 heads,
    the KV heads 0-1 and 6-7)."""
    m = re.match(r"B1_H32_Hkv8_D128_(?:P(\d+)_)?Lq(\d+)(?:_Lk\d+)?_c1$", sig)
    assert m, sig
    paged_p, L = m.group(1), int(m.group(2))
    for dtype in (torch.float16, torch.bfloat16):
        label = f"store prefill {sig} {dtype}"
        print(label, flush=True)
        g = torch.Generator().manual_seed(L)
        q = torch.randn(L, 32, 128, generator=g).to(dtype).to(DEV)
        k = torch.randn(L, 8, 128, generator=g).to(dtype).to(DEV)
        v = torch.randn(L, 8, 128, generator=g).to(dtype).to(DEV)
        cu = torch.tensor([0, L], dtype=torch.int32, device=DEV)
        if paged_p is None:
            out = prefill_attention(q, k, v, cu, cu, L, L, causal=True)
        else:
            P = int(paged_p)
            table, num_pages = _table([L], P, seed=L + 1)
            perm = table[0].long()
            kc = torch.empty(num_pages, P, 8, 128, dtype=dtype, device=DEV)
            vc = torch.empty_like(kc)
            kc[perm.to(DEV)] = k.view(-1, P, 8, 128)
            vc[perm.to(DEV)] = v.view(-1, P, 8, 128)
            cache = PagedKVCache(kc, vc, table.to(DEV), torch.tensor([L], dtype=torch.int32, device=DEV), P)
            out = paged_prefill_attention(q, cache, cu, L, causal=True)
        torch.cuda.synchronize()
        cu_c = torch.tensor([0, L], dtype=torch.int32)
        for h0, kv0 in ((0, 0), (24, 6)):
            ref = ref_attention_varlen(q[:, h0:h0 + 8].cpu(), k[:, kv0:kv0 + 2].cpu(), v[:, kv0:kv0 + 2].cpu(),
                                       cu_c, cu_c, causal=True, return_fp32=True)
            assert_parity(out[:, h0:h0 + 8], ref, label=f"{label} heads {h0}-{h0 + 7}")
        del q, k, v, out


def test_configs0_cpu_reference_workload():
    """B4, 32/8 heads, D128, page 16, ctx ~ U{64..512} (seeded),
    a 256-page pool and a seeded randperm(256) table sliced to [4, 32]; fp16
    pages; the whole batch against the oracle."""
    print("configs[0] B4 ctx U[64,512] pool 256", flush=True)
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(64, 513, (4,), generator=g).to(torch.int32)
    table = torch.randperm(256, generator=g)[:128].to(torch.int32).view(4, 32)
    k = torch.randn(256, 16, 8, 128, generator=g).half()
    v = torch.randn(256, 16, 8, 128, generator=g).half()
    q = torch.randn(4, 32, 128, generator=g).half()
    cache = PagedKVCache(k.to(DEV), v.to(DEV), table.to(DEV), lens.to(DEV), 16)
    out = paged_decode_attention(q.to(DEV), cache)
    torch.cuda.synchronize()
    ref = ref_attention_paged(q, k, v, table, lens, return_fp32=True)
    assert_parity(out, ref, label=f"configs[0] lens {lens.tolist()}")


@pytest.mark.parametrize("h,hk,d,P", [(32, 8, 128, 16), (32, 1, 128, 16), (32, 8, 64, 16), (32, 8, 128, 32),
                                      (32, 8, 128, 64)])
def test_configs4_log_uniform_batch(h, hk, d, P):
    """64 sequences with log-uniform lengths in [16, 65536]
    (seeded), with the MQA / D64 / page 32 and 64 variants, ``config=None``."""
    label = f"configs[4] 64 log-uniform H{h}/{hk} D{d} P{P}"
    print(label, flush=True)
    g = torch.Generator().manual_seed(64)
    lo, hi = math.log(16), math.log(65536)
    lens = [int(math.exp(x)) for x in (torch.rand(64, generator=g) * (hi - lo) + lo).tolist()]
    table, num_pages = _table(lens, P, seed=65)
    k, v = _pool(num_pages, P, hk, d, torch.float16, seed=66)
    q = torch.randn(64, h, d, generator=g).half().to(DEV)
    cache = PagedKVCache(k, v, table.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV), P)
    out = paged_decode_attention(q, cache)
    torch.cuda.synchronize()
    longest = max(range(64), key=lambda b: lens[b])
    shortest = min(range(64), key=lambda b: lens[b])
    _check_rows(out, q, cache, sorted({0, 31, 63, longest, shortest}), label)
