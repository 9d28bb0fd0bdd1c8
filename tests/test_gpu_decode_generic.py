"""GPU parity of the decode shapes only the generic (LDS-tiled) decode kernel
takes, and of the native decode entry that reaches them.

* fp32 queries and caches (the reference's native decode accepts fp32,
  csrc/paged_decode.cu:317, and its Python wrapper falls back to its fp32
  oracle for them, kernels/decode.py:569-576);
* page sizes 1-3 and other sizes that are not a power of two or lie below
  the VALU/MFMA kernels' floor (4-16 rows);
* head_dim 32 and 256;
* int8/fp8 caches with pages below the floor;
* ``native.paged_decode_attention`` with the binding's contract: fp16 / bf16
  / fp32, page_size 1..32 (also smaller than the cache's page dimension),
  head_dim 64/128, and zeros for sequences of length <= 0
  (csrc/paged_decode.cu:135-143), plus its argument errors.

Oracle: the fp32 restatement of the reference (oracle/reference.py);
tolerance 2e-3 on the kernel's result before its final rounding
(tests/_parity.py), and for fp32 outputs 1e-5 relative to max(1, |ref|).
"""

from __future__ import annotations

import pytest
import torch

from _parity import assert_parity, make_paged, make_query
from flashattntile_amd import PagedKVCache, native, paged_decode_attention, paged_decode_attention_fp8
from oracle import quant_ref
from oracle.reference import ref_attention_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"
LENS = [1, 17, 255, 1000]


def _case(lens, h, hk, d, P, dtype, seed):
    k, v, pt, sl = make_paged(lens, hk, d, P, dtype, seed=seed, device=DEV)
    return make_query(len(lens), h, d, dtype, seed=seed + 1, device=DEV), PagedKVCache(k, v, pt, sl, P)


def _ref32(q, cache, scale=None):
    return ref_attention_paged(q.cpu().float(), cache.k_cache.cpu().float(), cache.v_cache.cpu().float(),
                               cache.page_table.cpu(), cache.seq_lens.cpu(), softmax_scale=scale,
                               return_fp32=True)


# fp32 against the fp32 oracle: only the order of the fp32 sums and the
# exp2 of the scores differ, a few ulps of the output per element.  1e-5
# relative would catch K, V or P rounded to fp16 or bf16 anywhere on the
# path (fp16 rounding moves N(0,1) data by up to 5e-4).
FP32_RTOL = 1e-5


def _fp32_parity(out, ref, label):
    o = out.float().cpu()
    err = (o - ref).abs()
    rel = (err / ref.abs().clamp_min(1.0)).max().item()
    print(f"{label} max_abs={err.max().item():.3e} max_rel={rel:.3e}", flush=True)
    assert out.dtype == torch.float32 and torch.isfinite(out).all(), label
    assert rel <= FP32_RTOL, f"{label}: {rel:.3e} > {FP32_RTOL} relative to max(1, |ref|)"


@pytest.mark.parametrize("split_k", [1, 3])
@pytest.mark.parametrize("P", [1, 3, 16])
@pytest.mark.parametrize("h,hk", [(8, 8), (32, 8), (32, 1)])
@pytest.mark.parametrize("d", [64, 128])
def test_fp32_decode(d, h, hk, P, split_k):
    label = f"fp32 decode D{d} H{h}/{hk} P{P} sk{split_k}"
    print(label, flush=True)
    q, cache = _case(LENS, h, hk, d, P, torch.float32, seed=d + h + P)
    out = paged_decode_attention(q, cache, config={"split_k": split_k})
    torch.cuda.synchronize()
    _fp32_parity(out, _ref32(q, cache), label)


@pytest.mark.parametrize("P", [1, 2, 3, 5, 6, 12, 24])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_small_and_odd_pages(dtype, P):
    """Pages below the fast kernels' floor or not a power of two run on the
    generic kernel under the library's own choice."""
    label = f"generic pages {dtype} P{P}"
    print(label, flush=True)
    q, cache = _case(LENS, 32, 8, 128, P, dtype, seed=P)
    for split_k in (1, 4):
        out = paged_decode_attention(q, cache, config={"split_k": split_k})
        torch.cuda.synchronize()
        assert_parity(out, _ref32(q, cache), label=f"{label} sk{split_k}")


@pytest.mark.parametrize("d", [16, 32, 256, 512])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_head_dims_16_to_512(dtype, d):
    """Head dims the fast kernels do not take (16, 32, 256, 512) run on the
    generic kernel; at 16, 8 heads x 16 dims leave half its output threads
    idle, at 512 its K/V tiles fill 128 KB of LDS."""
    label = f"generic D{d} {dtype}"
    print(label, flush=True)
    q, cache = _case(LENS + [4096], 16, 4, d, 16, dtype, seed=d)
    for split_k in (1, 5):
        out = paged_decode_attention(q, cache, config={"split_k": split_k})
        torch.cuda.synchronize()
        if dtype == torch.float32:
            _fp32_parity(out, _ref32(q, cache), f"{label} sk{split_k}")
        else:
            assert_parity(out, _ref32(q, cache), label=f"{label} sk{split_k}")


@pytest.mark.parametrize("P", [1, 4, 7])
@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
def test_quant_small_pages(mode, qdtype, P):
    """int8/fp8 pages below the 8-row floor: the generic kernel dequantises
    as the other decode kernels do (K with fp16 queries exact in fp32 and
    k_scale on the scores, as the reference's quantised kernel,
    kernels/decode.py:419-429; V, and K with bf16 queries, rounded to
    q.dtype); the oracle dequantises to q.dtype first (the reference's
    dequantise-then-attend path, kernels/decode.py:674-682)."""
    label = f"generic quant {mode} {qdtype} P{P}"
    print(label, flush=True)
    k, v, pt, sl = make_paged(LENS, 8, 128, P, torch.float32, seed=P + 7, device="cpu")
    qk, sk = quant_ref.quantize_pages(k, mode)
    qv, sv = quant_ref.quantize_pages(v, mode)
    q = make_query(len(LENS), 32, 128, qdtype, seed=P + 8, device=DEV)
    cache = PagedKVCache(qk.to(DEV), qv.to(DEV), pt.to(DEV), sl.to(DEV), P)
    ref = ref_attention_paged(q.cpu(), quant_ref.dequantize_pages(qk, sk, qdtype),
                              quant_ref.dequantize_pages(qv, sv, qdtype), pt, sl, return_fp32=True)
    for split_k in (1, 3):
        out = paged_decode_attention_fp8(q, cache, {"k": sk.to(DEV), "v": sv.to(DEV)}, config={"split_k": split_k})
        torch.cuda.synchronize()
        assert_parity(out, ref, label=f"{label} sk{split_k}")


@pytest.mark.parametrize("d", [16, 512])
@pytest.mark.parametrize("mode", ["int8", "float8_e4m3fn"])
def test_quant_head_dims_16_and_512(mode, d):
    label = f"generic quant {mode} D{d}"
    print(label, flush=True)
    k, v, pt, sl = make_paged(LENS, 4, d, 16, torch.float32, seed=d + 3, device="cpu")
    qk, sk = quant_ref.quantize_pages(k, mode)
    qv, sv = quant_ref.quantize_pages(v, mode)
    q = make_query(len(LENS), 16, d, torch.float16, seed=d + 4, device=DEV)
    cache = PagedKVCache(qk.to(DEV), qv.to(DEV), pt.to(DEV), sl.to(DEV), 16)
    ref = ref_attention_paged(q.cpu(), quant_ref.dequantize_pages(qk, sk, torch.float16),
                              quant_ref.dequantize_pages(qv, sv, torch.float16), pt, sl, return_fp32=True)
    for split_k in (1, 3):
        out = paged_decode_attention_fp8(q, cache, {"k": sk.to(DEV), "v": sv.to(DEV)}, config={"split_k": split_k})
        torch.cuda.synchronize()
        assert_parity(out, ref, label=f"{label} sk{split_k}")


def test_generic_equals_fast_kernels_on_their_shapes():
    """Forced onto a shape the fast kernels take, the generic kernel agrees
    with them within the tolerance (same maths, different reduction order)."""
    print("generic vs fast kernels", flush=True)
    q, cache = _case([700, 4096, 33, 129], 32, 8, 128, 16, torch.float16, seed=5)
    ref = _ref32(q, cache)
    for split_k in (1, 4):
        gen = paged_decode_attention(q, cache, config={"split_k": split_k, "kernel": "generic"})
        fast = paged_decode_attention(q, cache, config={"split_k": split_k})
        torch.cuda.synchronize()
        assert_parity(gen, ref, label=f"generic forced sk{split_k}")
        assert (gen.float() - fast.float()).abs().max().item() <= 4e-3


# ---------------------------------------------------------------------------
# native.paged_decode_attention: the reference binding's contract
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("P", [1, 2, 3, 7, 8, 16, 24, 32])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_native_decode(dtype, P):
    label = f"native {dtype} P{P}"
    print(label, flush=True)
    for d, (h, hk) in ((128, (32, 8)), (64, (8, 2))):
        q, cache = _case(LENS, h, hk, d, P, dtype, seed=P + d)
        out = native.paged_decode_attention(q, cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, P)
        torch.cuda.synchronize()
        ref = _ref32(q, cache)
        if dtype == torch.float32:
            _fp32_parity(out, ref, f"{label} D{d}")
        else:
            assert_parity(out, ref, label=f"{label} D{d}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_native_zero_and_negative_lengths_give_zeros(dtype):
    """``paged_decode.cu:135-143``: a sequence with seq_len <= 0 writes zeros;
    the other sequences of the batch are unaffected."""
    print(f"native zero lengths {dtype}", flush=True)
    q, cache = _case([300, 5, 64, 17], 32, 8, 128, 16, dtype, seed=3)
    lens = torch.tensor([300, 0, 64, -4], dtype=torch.int32, device=DEV)
    out = native.paged_decode_attention(q, cache.k_cache, cache.v_cache, cache.page_table, lens, 16, 0.07)
    torch.cuda.synchronize()
    assert torch.all(out[1] == 0) and torch.all(out[3] == 0)
    live = [0, 2]
    ref = ref_attention_paged(q[live].cpu().float(), cache.k_cache.cpu().float(), cache.v_cache.cpu().float(),
                              cache.page_table[live].cpu(), lens[live].cpu(), softmax_scale=0.07, return_fp32=True)
    if dtype == torch.float32:
        _fp32_parity(out[live], ref, "native live rows")
    else:
        assert_parity(out[live], ref, label="native live rows")


def test_native_page_size_below_the_cache_page_dimension():
    """page_size smaller than the pages' slot count: only the first
    page_size slots of each page are tokens (the binding indexes slots with
    page_size and the cache's strides)."""
    print("native page_size < page dim", flush=True)
    q, cache = _case([40, 300], 16, 4, 128, 16, torch.float16, seed=9)
    P = 5
    lens = cache.seq_lens.cpu()
    # re-pack: token t at slot t % 5 of logical page t // 5, pages of 16 slots
    k_full, v_full, table = cache.k_cache.cpu(), cache.v_cache.cpu(), cache.page_table.cpu()
    need = [-(-int(n) // P) for n in lens]
    pool_k = torch.full((sum(need) + 1, 16, 4, 128), 7.0, dtype=torch.float16)
    pool_v = torch.full_like(pool_k, -3.0)
    new_table = torch.zeros(2, max(need), dtype=torch.int32)
    at_ = 1
    for b, n in enumerate(lens.tolist()):
        for lp in range(need[b]):
            new_table[b, lp] = at_ + lp
            for s in range(P):
                t = lp * P + s
                if t < n:
                    src_page = int(table[b, t // 16])
                    pool_k[at_ + lp, s] = k_full[src_page, t % 16]
                    pool_v[at_ + lp, s] = v_full[src_page, t % 16]
        at_ += need[b]
    out = native.paged_decode_attention(q, pool_k.to(DEV), pool_v.to(DEV), new_table.to(DEV), cache.seq_lens, P)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache), label="native page_size 5 of 16")


def test_native_argument_errors():
    """The binding's checks (paged_decode.cu:306-323) raise RuntimeError
    before anything is enqueued."""
    print("native argument errors", flush=True)
    q, cache = _case([30, 40], 8, 2, 128, 16, torch.float16, seed=1)
    k, v, pt, sl = cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens
    cases = [
        ((q.cpu(), k, v, pt, sl, 16), "q must be a CUDA tensor"),
        ((q, k.cpu(), v, pt, sl, 16), "KV cache must be CUDA tensors"),
        ((q, k, v, pt.cpu(), sl, 16), "metadata must be CUDA tensors"),
        ((q[0], k, v, pt, sl, 16), r"q must be \[batch, heads, head_dim\]"),
        ((q.transpose(0, 1).contiguous().transpose(0, 1), k, v, pt, sl, 16), "q must be contiguous"),
        ((q, k, v, pt.long(), sl, 16), "page_table must be int32"),
        ((q, k, v, pt, sl.long(), 16), "seq_lens must be int32"),
        ((q.float(), k, v, pt, sl, 16), "q and cache dtypes must match"),
        ((q, k, v[:-1], pt, sl, 16), "k/v cache shapes must match"),
        ((q, k, v, pt, sl, 0), r"page_size must be in \[1, 32\]"),
        ((q, k, v, pt, sl, 33), r"page_size must be in \[1, 32\]"),
        ((q, k, v, pt[:1], sl, 16), "page_table batch must match q"),
        ((q, k, v, pt, sl[:1], 16), "seq_lens batch must match q"),
        ((q[:, :7].contiguous(), k, v, pt, sl, 16), "heads must be divisible by KV heads"),
        ((q.to(torch.int16), k.to(torch.int16), v.to(torch.int16), pt, sl, 16), "supports fp16, bf16 and fp32"),
    ]
    for args, msg in cases:
        with pytest.raises(RuntimeError, match=msg):
            native.paged_decode_attention(*args)
