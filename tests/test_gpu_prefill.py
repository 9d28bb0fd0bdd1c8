"""GPU parity of the HIP varlen prefill against the fp32 oracle.

Unscaled N(0,1) inputs; tolerance 2e-3 on the kernel's result before the
final rounding to the output dtype (tests/_parity.py).  Covers the
reference's GPU test matrix (tests/test_kernel_correctness.py:71-127,
tests/test_prefill.py:54-89) plus BASELINE configs[2]: single sequences of
512..8192 tokens and a mixed pack of 8 sequences with lengths in [1, 4096].
"""

from __future__ import annotations

import pytest
import torch

from _parity import assert_parity, force_prefill_knobs, make_paged, make_varlen, ulp
from flashattntile_amd import PagedKVCache, prefill_attention
from flashattntile_amd.kernels.prefill import paged_prefill_attention, prefill_launch
from oracle.reference import ref_attention_paged_prefill, ref_attention_varlen

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODD_LENS = [1, 17, 255, 1000]


@pytest.fixture(params=["auto", "pingpong", "wide", "4wave", "4wave_split"])
def kernel(request, monkeypatch):
    """Run the test with the library's automatic choice and with each prefill
    kernel forced (8-wave ping-pong with 32 or 64 rows per wave, 4-wave,
    4-wave key split), whatever the shape.  The wide kernel takes head_dim
    128 only; tests with other head dims check that it refuses them."""
    if request.param != "auto":
        force_prefill_knobs(monkeypatch, kernel=request.param)
    return request.param


def _ref32(q, k, v, cu_q, cu_k, causal, scale=None):
    return ref_attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=causal,
                                softmax_scale=scale, return_fp32=True)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("h,hk", [(8, 8), (8, 2), (8, 1), (32, 8)])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_matches_oracle(dtype, d, h, hk, causal, kernel):
    label = f"prefill {kernel} {dtype} D{d} H{h}/{hk} causal={causal}"
    print(label, flush=True)
    q, k, v, cu = make_varlen(ODD_LENS, h, hk, d, dtype, seed=d + h + hk, device=DEV)
    if kernel == "wide" and d != 128:
        with pytest.raises(RuntimeError, match="wide prefill kernel takes packed head_dim-128"):
            prefill_attention(q, k, v, cu, cu, max(ODD_LENS), max(ODD_LENS), causal=causal)
        return
    out = prefill_attention(q, k, v, cu, cu, max(ODD_LENS), max(ODD_LENS), causal=causal)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == dtype
    assert_parity(out, _ref32(q, k, v, cu, cu, causal), label=label)


# (kv_len, q_len) per sequence: entries with no queries, with and without
# keys, at both ends and between sequences that have work (a serving batch
# where some sequences have no new tokens this step).
EMPTY_Q = [(0, 0), (40, 0), (17, 17), (0, 0), (300, 300), (129, 0), (64, 1), (700, 513), (9, 0)]


def _varlen_kq(pairs, h, hk, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    lk = [p[0] for p in pairs]
    lq = [p[1] for p in pairs]

    def offsets(lens):
        return torch.tensor([0] + torch.cumsum(torch.tensor(lens), 0).tolist(), dtype=torch.int32, device=DEV)

    q = torch.randn(sum(lq), h, d, generator=g).to(dtype).to(DEV)
    k = torch.randn(sum(lk), hk, d, generator=g).to(dtype).to(DEV)
    v = torch.randn(sum(lk), hk, d, generator=g).to(dtype).to(DEV)
    return q, k, v, offsets(lq), offsets(lk), max(lq), max(lk)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_batch_with_sequences_without_queries(dtype, causal, kernel):
    """q_len = 0 sequences take the kernels' early return and leave the
    other sequences' results unchanged: parity for the whole batch, and
    bit-identity, on a forced kernel, with the same batch without them."""
    label = f"prefill {kernel} {dtype} empty-query entries causal={causal}"
    print(label, flush=True)
    q, k, v, cq, ck, mq, mk = _varlen_kq(EMPTY_Q, 16, 4, 128, dtype, seed=41)
    out = prefill_attention(q, k, v, cq, ck, mq, mk, causal=causal)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, k, v, cq, ck, causal), label=label)
    if kernel == "auto":  # the smaller batch may get another kernel
        return
    # The same work without the empty entries on the same kernel: identical bits.
    keep = [i for i, (_, n) in enumerate(EMPTY_Q) if n > 0]
    kst, qst = ck.tolist(), cq.tolist()
    k2 = torch.cat([k[kst[i]:kst[i + 1]] for i in keep])
    v2 = torch.cat([v[kst[i]:kst[i + 1]] for i in keep])
    lens_k = [EMPTY_Q[i][0] for i in keep]
    lens_q = [EMPTY_Q[i][1] for i in keep]
    ck2 = torch.tensor([0] + torch.cumsum(torch.tensor(lens_k), 0).tolist(), dtype=torch.int32, device=DEV)
    cq2 = torch.tensor([0] + torch.cumsum(torch.tensor(lens_q), 0).tolist(), dtype=torch.int32, device=DEV)
    out2 = prefill_attention(q, k2, v2, cq2, ck2, mq, max(lens_k), causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), label


# head_dim 32 runs on every prefill kernel; head_dim 256 on the 4-wave kernel
# only (O and Q take 192 registers per lane), which the others refuse.
HEAD_DIM_KERNELS = {32: [None, "pingpong", "4wave", "4wave_split"], 256: [None, "4wave"]}


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [32, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_head_dims_32_and_256(dtype, d, causal):
    """The reference's prefill is generic over a power-of-two head_dim
    (flashattn_tile/kernels/prefill.py:59-89); 32 and 256 against the oracle
    on ragged lengths, GQA 8/2, every kernel that takes them."""
    q, k, v, cu = make_varlen(ODD_LENS, 8, 2, d, dtype, seed=d + 3, device=DEV)
    ref = _ref32(q, k, v, cu, cu, causal)
    for kern in HEAD_DIM_KERNELS[d]:
        label = f"prefill {kern or 'auto'} {dtype} D{d} causal={causal}"
        print(label, flush=True)
        out = prefill_attention(q, k, v, cu, cu, max(ODD_LENS), max(ODD_LENS), causal=causal,
                                config={"kernel": kern})
        torch.cuda.synchronize()
        assert_parity(out, ref, label=label)


def test_prefill_head_dim_256_refuses_the_8_wave_kernels():
    q, k, v, cu = make_varlen([70], 4, 2, 256, torch.float16, seed=4, device=DEV)
    for kern in ("pingpong", "4wave_split"):
        with pytest.raises(RuntimeError, match="head_dim 256 runs on the 4-wave"):
            prefill_attention(q, k, v, cu, cu, 70, 70, causal=True, config={"kernel": kern})


@pytest.mark.parametrize("seqlen", [1, 2, 63, 64, 65, 127, 128, 129, 1000])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_single_odd_length(seqlen, dtype, kernel):
    q, k, v, cu = make_varlen([seqlen], 8, 2, 128, dtype, seed=8, device=DEV)
    for causal in (True, False):
        label = f"prefill {kernel} single L{seqlen} {dtype} causal={causal}"
        print(label, flush=True)
        out = prefill_attention(q, k, v, cu, cu, seqlen, seqlen, causal=causal)
        torch.cuda.synchronize()
        assert_parity(out, _ref32(q, k, v, cu, cu, causal), label=label)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_kv_longer_than_q(dtype, causal, kernel):
    """Bottom-right causal alignment with kv_len > q_len (chunked-prefill shape)."""
    label = f"prefill {kernel} q<kv {dtype} causal={causal}"
    print(label, flush=True)
    g = torch.Generator().manual_seed(3)
    lq, lk = [3, 50, 129, 1], [10, 300, 129, 77]
    q = torch.randn(sum(lq), 8, 128, generator=g).to(dtype).to(DEV)
    k = torch.randn(sum(lk), 2, 128, generator=g).to(dtype).to(DEV)
    v = torch.randn(sum(lk), 2, 128, generator=g).to(dtype).to(DEV)
    cq = torch.tensor([0, 3, 53, 182, 183], dtype=torch.int32, device=DEV)
    ck = torch.tensor([0, 10, 310, 439, 516], dtype=torch.int32, device=DEV)
    out = prefill_attention(q, k, v, cq, ck, max(lq), max(lk), causal=causal, softmax_scale=0.07)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, k, v, cq, ck, causal, scale=0.07), label=label)


@pytest.mark.parametrize("scale", [-0.08, 0.0])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_non_positive_scales(dtype, causal, scale, kernel):
    """The MFMA kernels take a positive scale: a negative one runs as its
    magnitude with Q's signs flipped as Q is loaded, a zero one with Q zeroed
    (every logit 0, so each query averages its visible V rows).  Packed and
    paged (the wide kernel through staged K/V) against the oracle."""
    label = f"prefill {kernel} {dtype} scale={scale} causal={causal}"
    print(label, flush=True)
    lens = [1, 17, 255, 1000, 640]
    q, k, v, cu = make_varlen(lens, 32, 8, 128, dtype, seed=71, device=DEV)
    out = prefill_attention(q, k, v, cu, cu, max(lens), max(lens), causal=causal, softmax_scale=scale)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, k, v, cu, cu, causal, scale=scale), label=label)
    kc, vc, pt, sl = make_paged(lens, 8, 128, 16, dtype, seed=72, device=DEV)
    cache = PagedKVCache(kc, vc, pt, sl, 16)
    out_p = paged_prefill_attention(q, cache, cu, max(lens), causal=causal, softmax_scale=scale)
    torch.cuda.synchronize()
    ref_p = ref_attention_paged_prefill(q.cpu(), kc.cpu(), vc.cpu(), pt.cpu(), sl.cpu(), cu.cpu(), causal=causal,
                                        softmax_scale=scale, return_fp32=True)
    assert_parity(out_p, ref_p, label=f"paged {label}")


def _wide_pack(n, seed):
    """n (kv_len, q_len) pairs: queries of 1-1300 tokens, some after a prefix
    of up to 700 keys, a few without queries."""
    g = torch.Generator().manual_seed(seed)
    pairs = []
    for i in range(n):
        lq = int(torch.randint(1, 1301, (1,), generator=g))
        pre = int(torch.randint(0, 701, (1,), generator=g)) if i % 3 == 1 else 0
        if i % 7 == 5:
            lq = 0
        pairs.append((lq + pre, lq))
    return pairs


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("n", [2, 16, 17, 40])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_wide_kernel_pack_orders(dtype, n, causal):
    """The wide kernel runs packs of 2-16 sequences in an order it ranks on
    the device (longest causal chain first) and larger packs in block order;
    either way every (query block, sequence) item is computed once.  Ragged
    packs on both sides of that limit, with prefixes and sequences without
    queries, against the oracle."""
    label = f"prefill wide pack of {n} {dtype} causal={causal}"
    print(label, flush=True)
    q, k, v, cq, ck, mq, mk = _varlen_kq(_wide_pack(n, seed=n), 8, 2, 128, dtype, seed=n + 1)
    out = prefill_attention(q, k, v, cq, ck, mq, mk, causal=causal, config={"kernel": "wide"})
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, k, v, cq, ck, causal), label=label)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_mixed_pack_baseline(dtype, kernel):
    """BASELINE configs[2] mixed pack: 8 sequences, lengths uniform in [1, 4096]."""
    g = torch.Generator().manual_seed(2024)
    lens = torch.randint(1, 4097, (8,), generator=g).tolist()
    lens[0] |= 1  # at least one odd length
    label = f"prefill {kernel} mixed {lens} {dtype}"
    print(label, flush=True)
    q, k, v, cu = make_varlen(lens, 32, 8, 128, dtype, seed=5, device=DEV)
    out = prefill_attention(q, k, v, cu, cu, max(lens), max(lens), causal=True)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, k, v, cu, cu, True), label=label)


@pytest.mark.parametrize("seqlen", [512, 2048, 8192])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_long_sequence_head_subsets(seqlen, dtype, kernel):
    """BASELINE configs[2] single sequences (32/8 heads, D128, causal): all
    heads are computed by the kernel; the oracle checks the query heads of
    KV heads 0 and 7 (the oracle's [H, L, L] fp32 scores are kept small)."""
    q, k, v, cu = make_varlen([seqlen], 32, 8, 128, dtype, seed=seqlen, device=DEV)
    label = f"prefill {kernel} L{seqlen} {dtype}"
    print(label, flush=True)
    out = prefill_attention(q, k, v, cu, cu, seqlen, seqlen, causal=True)
    torch.cuda.synchronize()
    for kvh in (0, 7):
        hs = slice(4 * kvh, 4 * kvh + 4)
        ref = _ref32(q[:, hs].contiguous(), k[:, kvh:kvh + 1].contiguous(), v[:, kvh:kvh + 1].contiguous(),
                     cu, cu, True, scale=128 ** -0.5)
        assert_parity(out[:, hs], ref, label=f"{label} kv{kvh}")


def _first_and_last_rows_ref(q, k, v, L, n, kvh):
    """fp32 oracle for query rows [0, n) and [L - n, L) of one causal
    L-token sequence (the query heads of KV head kvh): the first n rows see
    only the first n tokens, and under bottom-right alignment the last n rows
    are exactly an n-query prefill over all L keys."""
    hs = slice(4 * kvh, 4 * kvh + 4)
    kk, vv = k[:, kvh:kvh + 1].cpu().contiguous(), v[:, kvh:kvh + 1].cpu().contiguous()
    cu_n = torch.tensor([0, n], dtype=torch.int32)
    cu_l = torch.tensor([0, L], dtype=torch.int32)
    first = ref_attention_varlen(q[:n, hs].cpu().contiguous(), kk[:n].contiguous(), vv[:n].contiguous(), cu_n, cu_n,
                                 causal=True, return_fp32=True)
    last = ref_attention_varlen(q[L - n:, hs].cpu().contiguous(), kk, vv, cu_n, cu_l, causal=True, return_fp32=True)
    return hs, first, last


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_32k_sequence_first_and_last_rows(dtype):
    """One causal sequence of 32768 tokens (32/8 heads, D128), four times
    BASELINE's longest prefill: the kernels address K/V with 32-bit offsets
    per sequence and run 128 query blocks per head.  The first and last 256
    rows of KV heads 0 and 7 against the fp32 oracle."""
    L, n = 32768, 256
    label = f"prefill 32k {dtype}"
    print(label, flush=True)
    q, k, v, cu = make_varlen([L], 32, 8, 128, dtype, seed=32, device=DEV)
    out = prefill_attention(q, k, v, cu, cu, L, L, causal=True)
    torch.cuda.synchronize()
    for kvh in (0, 7):
        hs, first, last = _first_and_last_rows_ref(q, k, v, L, n, kvh)
        assert_parity(out[:n, hs], first, label=f"{label} kv{kvh} first rows")
        assert_parity(out[L - n:, hs], last, label=f"{label} kv{kvh} last rows")


def test_prefill_launch_into_strided_output():
    """prefill_launch writes into a caller-provided (head-strided) buffer."""
    print("prefill strided out", flush=True)
    q, k, v, cu = make_varlen([40, 70], 8, 2, 64, torch.float16, seed=1, device=DEV)
    big = torch.zeros(110, 8, 128, dtype=torch.float16, device=DEV)
    out = big[:, :, :64]
    prefill_launch(q, k, v, cu, cu, 70, 70, True, 64 ** -0.5, out=out)
    torch.cuda.synchronize()
    assert torch.all(big[:, :, 64:] == 0)
    assert_parity(out, _ref32(q, k, v, cu, cu, True), label="strided out")


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_output_rows_only_8_byte_aligned(dtype, d, kernel):
    """Output rows that start 8 bytes past a 16-byte boundary (base offset 4
    elements, head stride d + 4): the kernels store each row in 8-byte pieces
    there, and the 4-element gaps between heads stay untouched."""
    print(f"prefill 8-byte-aligned out {dtype} D{d} {kernel}", flush=True)
    q, k, v, cu = make_varlen([300, 77, 129], 8, 2, d, dtype, seed=5, device=DEV)
    big = torch.zeros(q.shape[0], 8, d + 4, dtype=dtype, device=DEV)
    out = big[:, :, 4:]
    assert out.data_ptr() % 16 == 8 and (out.stride(1) * out.element_size()) % 16 == 8
    if kernel == "wide" and d != 128:
        with pytest.raises(RuntimeError, match="wide prefill kernel"):
            prefill_launch(q, k, v, cu, cu, 300, 300, True, d ** -0.5, out=out, kernel=kernel)
        return
    prefill_launch(q, k, v, cu, cu, 300, 300, True, d ** -0.5, out=out, kernel=None if kernel == "auto" else kernel)
    torch.cuda.synchronize()
    assert torch.all(big[:, :, :4] == 0)
    assert_parity(out, _ref32(q, k, v, cu, cu, True), label=f"8-byte-aligned out D{d} {kernel}")


def test_ops_compile_on_device():
    """The custom ops inside a torch.compile(fullgraph=True) graph on the GPU."""
    print("prefill compile", flush=True)
    q, k, v, cu = make_varlen([3, 6], 4, 2, 64, torch.float16, seed=2, device=DEV)

    def fn(x):
        return torch.ops.flashattn_tile.prefill_varlen(x, k, v, cu, cu, 6, 6, True, 0.35)

    out = torch.compile(fn, fullgraph=True, backend="eager")(q)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, k, v, cu, cu, True, scale=0.35), label="compiled prefill op")


@pytest.mark.parametrize("huge", [7.0e4, 1.0e6, 3.0e8])
def test_prefill_bf16_v_beyond_fp16_range(huge, kernel):
    """bf16 V rows of magnitude >= 2^15: V is staged as fp16 scaled by 2^-s
    (per staging wave in the 4-wave kernels and in the ping-pong kernel
    without a workspace; per KV head from the pre-pass when the ping-pong
    kernel has one, as prefill_attention gives it, and the sequence has the
    2048 queries that enable it) and O is tracked as acc * 2^e.
    Key 300 (tile 4) holds huge/8 and the last two keys +-huge, so the scale
    grows twice along the sequence; queries before key 300 never see a huge
    row but read rows staged by the same wave (tile 4), which must keep the
    2e-3 absolute bound; the others are checked relative to their magnitude."""
    label = f"prefill {kernel} bf16 |v| up to {huge:g}"
    print(label, flush=True)
    L = 2112  # >= 2048 queries: the ping-pong kernel takes the V pre-pass
    q, k, v, cu = make_varlen([L], 8, 2, 128, torch.bfloat16, seed=21)
    g = torch.Generator().manual_seed(22)
    for j, f in ((300, huge / 8), (L - 2, -huge), (L - 1, huge)):
        v[j] = (torch.sign(torch.randn(2, 128, generator=g)) * f).to(torch.bfloat16)
    q, k, v, cu = q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV)
    out = prefill_attention(q, k, v, cu, cu, L, L, causal=True)
    torch.cuda.synchronize()
    ref = _ref32(q, k, v, cu, cu, True)
    assert_parity(out[:300], ref[:300], label=f"{label} (queries that see no huge row)")
    # 2e-3 relative to each output row's magnitude, beyond the final rounding
    o32, r32 = out[300:].float().cpu(), ref[300:].float()
    scale = r32.abs().amax(dim=-1, keepdim=True).clamp_min(1.0)
    rounding = 0.5 * ulp(torch.maximum(o32.abs(), r32.abs()), torch.bfloat16)
    excess = ((o32 - r32).abs() - rounding) / scale
    print(f"{label}: max relative error beyond rounding {excess.max().item():.3e}", flush=True)
    assert torch.isfinite(o32).all() and excess.max().item() <= 2e-3, label


def test_prefill_bf16_with_and_without_workspace():
    """bf16 on the ping-pong kernel with the workspace (V converted to fp16
    by the pre-pass, one scale per sequence and KV head) and without it (V converted tile
    by tile in the kernel): bit-identical while every |v| < 2^15 (both scales
    are 1), and both within the tolerance when a row reaches 1e6.  The
    sequence has the 2048 queries from which the library runs the pre-pass."""
    from flashattntile_amd import _hip

    print("prefill bf16 workspace / no workspace", flush=True)
    L = 2304
    q, k, v, cu = make_varlen([L], 32, 8, 128, torch.bfloat16, seed=31, device=DEV)
    outs = []
    for big in (False, True):
        if big:
            v[700, 3] = 1.0e6
        with_ws = prefill_launch(q, k, v, cu, cu, L, L, True, 128 ** -0.5, kernel="pingpong")
        no_ws = torch.empty_like(q)
        _hip.prefill_varlen(q, k, v, cu, cu, no_ws, L, L, True, 128 ** -0.5, workspace=None,
                            kernel=_hip.KERNEL_PREFILL_PINGPONG)
        torch.cuda.synchronize()
        outs.append((with_ws, no_ws))
    assert torch.equal(outs[0][0], outs[0][1])
    for kvh in (0, 3):
        hs = slice(4 * kvh, 4 * kvh + 4)
        ref = _ref32(q[:, hs].contiguous(), k[:, kvh:kvh + 1].contiguous(), v[:, kvh:kvh + 1].contiguous(), cu, cu,
                     True)
        for name, out in zip(("workspace", "no workspace"), outs[1]):
            o32, r32 = out[:, hs].float().cpu(), ref.float()
            scale = r32.abs().amax(dim=-1, keepdim=True).clamp_min(1.0)
            rounding = 0.5 * ulp(torch.maximum(o32.abs(), r32.abs()), torch.bfloat16)
            excess = ((o32 - r32).abs() - rounding) / scale
            print(f"kv{kvh} {name}: max relative error beyond rounding {excess.max().item():.3e}", flush=True)
            assert torch.isfinite(o32).all() and excess.max().item() <= 2e-3, (kvh, name)


def test_prefill_bf16_prepass_keeps_sequences_independent():
    """The bf16 V pre-pass scales V per (sequence, KV head): a V row of 1e12
    in one sequence and inf in another leave the other sequences of the same
    packed launch at parity with the oracle and bit-identical to the launch
    without a workspace (in-kernel conversion, scale 1 on clean tiles), and
    the inf still reaches the queries of its own sequence that see it."""
    from flashattntile_amd import _hip

    lens = [2304, 2560, 2432, 2048]  # a mean of >= 2048 queries: the pre-pass runs
    H, HKV, D = 32, 8, 128
    q, k, v, cu = make_varlen(lens, H, HKV, D, torch.bfloat16, seed=37, device=DEV)
    starts = cu.tolist()
    huge_row, inf_row = starts[1] + 900, starts[2] + 1500
    v[huge_row, 2, 5] = 1.0e12
    v[inf_row, 2, 7] = float("inf")
    v[inf_row, 5, 0] = float("-inf")
    L = max(lens)
    out = torch.empty_like(q)
    a = _hip.prefill_args(q, k, v, cu, cu, out, L, L, True, D ** -0.5, kernel=_hip.KERNEL_PREFILL_PINGPONG)
    need = _hip.prefill_varlen_workspace_bytes(a)
    print(f"prefill bf16 pre-pass isolation: workspace {need} B", flush=True)
    assert 0 < need <= _hip.prefill_workspace_bytes(k.shape[0], HKV, D)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    a.workspace = ws.data_ptr()
    _hip.prefill_varlen_with_args(a, _hip.current_stream_handle(q.device))
    no_ws = torch.empty_like(q)
    _hip.prefill_varlen(q, k, v, cu, cu, no_ws, L, L, True, D ** -0.5, workspace=None,
                        kernel=_hip.KERNEL_PREFILL_PINGPONG)
    torch.cuda.synchronize()
    for b in (0, 3):
        rows = slice(starts[b], starts[b + 1])
        assert torch.equal(out[rows], no_ws[rows]), f"clean sequence {b}: pre-pass and in-kernel differ"
        cu1 = torch.tensor([0, lens[b]], dtype=torch.int32)
        for kvh in (2, 5, 0):
            hs = slice(kvh * (H // HKV), (kvh + 1) * (H // HKV))
            qs = q[rows, hs].contiguous().cpu()
            ref = _ref32(qs, k[rows, kvh:kvh + 1].contiguous(), v[rows, kvh:kvh + 1].contiguous(), cu1, cu1, True)
            assert_parity(out[rows, hs], ref, label=f"pre-pass isolation: clean sequence {b}, KV head {kvh}")
    # Sequence 2's queries that see its inf key (causal: query i sees key j
    # iff j <= i) have a non-finite output in the inf's column, in every head
    # of that KV head, as the oracle's have.
    seen = slice(inf_row, starts[3])
    for kvh, col in ((2, 7), (5, 0)):
        hs = slice(kvh * (H // HKV), (kvh + 1) * (H // HKV))
        assert not torch.isfinite(out[seen, hs, col].float()).any(), kvh
