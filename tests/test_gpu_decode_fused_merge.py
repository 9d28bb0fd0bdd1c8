"""Split-K decode with the merge inside the decode launch (merge_counters).

With counters, the last partition of each (sequence, head group) to finish
merges the partitions with the merge kernel's own arithmetic, so its output
must equal the two-launch merge bit for bit; every launch must leave the
counters zero for the next one (in-order launches share them, graph replays
reuse them).  The two-launch path itself is checked against the fp32 oracle
in test_gpu_decode.py; here one case per kernel is also checked against it.
"""

from __future__ import annotations

import pytest
import torch

from _parity import assert_parity, make_paged, make_query
from flashattntile_amd import PagedKVCache, _hip
from flashattntile_amd.kernels.decode import DecodeLaunch, merge_counters, paged_decode_attention, paged_decode_launch
from oracle import quant_ref
from oracle.reference import ref_attention_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"
LENS = [1, 17, 255, 1000, 4096, 300]


def _cache(lens, h, hk, d, P, dtype, seed):
    k, v, pt, sl = make_paged(lens, hk, d, P, dtype, seed=seed, device=DEV)
    return make_query(len(lens), h, d, dtype, seed=seed + 1, device=DEV), PagedKVCache(k, v, pt, sl, P)


def _quant_cache(lens, h, hk, d, P, qdtype, mode, seed):
    k, v, pt, sl = make_paged(lens, hk, d, P, torch.float32, seed=seed, device="cpu")
    qk, sk = quant_ref.quantize_pages(k, mode)
    qv, sv = quant_ref.quantize_pages(v, mode)
    q = make_query(len(lens), h, d, qdtype, seed=seed + 1, device=DEV)
    return q, PagedKVCache(qk.to(DEV), qv.to(DEV), pt.to(DEV), sl.to(DEV), P), {"k": sk.to(DEV), "v": sv.to(DEV)}


def _zeros(q):
    rows = q.shape[0] * (q.shape[1] if q.dim() == 4 else 1)
    return torch.zeros(_hip.decode_counters_bytes(rows, q.shape[-2]) // 4, dtype=torch.int32, device=DEV)


def _both(q, cache, split, kernel, scales=None, waves=None):
    """(two-launch merge, in-launch merge, counters after it)."""
    two = paged_decode_launch(q, cache, q.shape[-1] ** -0.5, split, scales=scales, kernel=kernel,
                              waves_per_group=waves)
    cnt = _zeros(q)
    one = paged_decode_launch(q, cache, q.shape[-1] ** -0.5, split, scales=scales, kernel=kernel,
                              waves_per_group=waves, counters=cnt)
    torch.cuda.synchronize()
    return two, one, cnt


@pytest.mark.parametrize("split", [2, 4, 7, 12, 16])
@pytest.mark.parametrize("kernel,waves", [("valu", 4), ("valu", 8), ("mfma", 4), ("mfma", 8)])
@pytest.mark.parametrize("h,hk", [(32, 8), (32, 1), (8, 2)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_in_launch_merge_is_bit_identical(dtype, h, hk, kernel, waves, split):
    label = f"fused merge {kernel} w{waves} {dtype} H{h}/{hk} sk{split}"
    print(label, flush=True)
    q, cache = _cache(LENS, h, hk, 128, 16, dtype, seed=split + h + hk)
    two, one, cnt = _both(q, cache, split, kernel, waves=waves)
    assert torch.equal(one, two), label
    assert int(cnt.abs().sum()) == 0, f"{label}: counters not left zero"


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_in_launch_merge_against_oracle(dtype, kernel):
    """Head dim 64, pages of 32, one case per kernel also against the oracle."""
    label = f"fused merge oracle {kernel} {dtype} D64"
    print(label, flush=True)
    q, cache = _cache(LENS, 32, 8, 64, 32, dtype, seed=5)
    two, one, cnt = _both(q, cache, 8, kernel)
    assert torch.equal(one, two), label
    ref = ref_attention_paged(q.cpu(), cache.k_cache.cpu(), cache.v_cache.cpu(), cache.page_table.cpu(),
                              cache.seq_lens.cpu(), return_fp32=True)
    assert_parity(one, ref, label=label)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
def test_in_launch_merge_quantised(qdtype, mode):
    label = f"fused merge {mode} {qdtype}"
    print(label, flush=True)
    q, cache, scales = _quant_cache(LENS, 32, 8, 128, 16, qdtype, mode, seed=9)
    for split in (3, 16):
        two, one, cnt = _both(q, cache, split, None, scales=scales)
        assert torch.equal(one, two), f"{label} sk{split}"
        assert int(cnt.abs().sum()) == 0


@pytest.mark.parametrize("T", [2, 5])
def test_in_launch_merge_multi_token(T):
    """q_len > 1: the MFMA kernel's (head, token) columns, counters sized by
    batch * q_len rows."""
    label = f"fused merge multi-token T{T}"
    print(label, flush=True)
    k, v, pt, sl = make_paged(LENS, 8, 128, 16, torch.float16, seed=21, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, 16)
    g = torch.Generator().manual_seed(22)
    q = torch.randn(len(LENS), T, 32, 128, generator=g).half().to(DEV)
    two, one, cnt = _both(q, cache, 8, None)
    assert torch.equal(one, two), label
    assert int(cnt.abs().sum()) == 0


def test_counters_shared_by_launches_in_order():
    """One counter buffer, launches of different split_k, batch and kernel in
    stream order without synchronisation in between: each result equals its
    two-launch counterpart."""
    print("fused merge shared counters", flush=True)
    cases = [_cache(LENS, 32, 8, 128, 16, torch.float16, seed=s) for s in (31, 32)]
    cnt = torch.zeros(1 << 16, dtype=torch.int32, device=DEV)
    plan = [(0, 4, "valu"), (1, 16, "mfma"), (0, 32, "valu"), (1, 3, "valu"), (0, 16, "mfma"), (1, 2, None)]
    outs, refs = [], []
    for i, split, kernel in plan:
        q, cache = cases[i]
        outs.append(paged_decode_launch(q, cache, 128 ** -0.5, split, kernel=kernel, counters=cnt))
    for i, split, kernel in plan:
        q, cache = cases[i]
        refs.append(paged_decode_launch(q, cache, 128 ** -0.5, split, kernel=kernel))
    torch.cuda.synchronize()
    for (i, split, kernel), o, r in zip(plan, outs, refs):
        assert torch.equal(o, r), (i, split, kernel)
    assert int(cnt.abs().sum()) == 0


def test_split_above_16_and_generic_kernel_merge_in_a_second_launch():
    """split_k > 16 and the generic kernel keep the merge kernel: results as
    without counters, which stay zero (untouched)."""
    print("fused merge fallbacks", flush=True)
    q, cache = _cache(LENS, 32, 8, 128, 16, torch.float16, seed=41)
    for split, kernel in ((32, "valu"), (48, "valu"), (64, "mfma"), (8, "generic")):
        two, one, cnt = _both(q, cache, split, kernel)
        assert torch.equal(one, two), (split, kernel)
        assert int(cnt.abs().sum()) == 0


def test_wrappers_use_the_in_launch_merge():
    """paged_decode_attention (cached counters per stream) and DecodeLaunch
    (its own counters) give the two-launch result, run after run."""
    print("fused merge wrappers", flush=True)
    q, cache = _cache(LENS, 32, 8, 128, 16, torch.float16, seed=51)
    ref = paged_decode_launch(q, cache, 128 ** -0.5, 8)
    a = paged_decode_attention(q, cache, config={"split_k": 8, "pages_per_split": 0})
    plan = DecodeLaunch(q, cache, config={"split_k": 8, "pages_per_split": 0})
    b1 = plan.run(q)
    b2 = plan.run(q)
    torch.cuda.synchronize()
    assert torch.equal(a, ref) and torch.equal(b1, ref) and torch.equal(b2, ref)
    assert plan.counters is not None and int(plan.counters.abs().sum()) == 0
    cached = merge_counters(q, 8)
    assert cached is not None and int(cached.abs().sum()) == 0
    assert merge_counters(q, 1) is None


def test_in_launch_merge_in_a_graph():
    """A captured split-K decode with counters, replayed with new queries
    (eager work and synchronisation between replays): every replay equals the
    eager two-launch result and leaves the counters zero."""
    print("fused merge graph", flush=True)
    q, cache = _cache(LENS, 32, 8, 128, 16, torch.float16, seed=61)
    qs = [make_query(len(LENS), 32, 128, torch.float16, seed=70 + i, device=DEV) for i in range(4)]
    cnt = _zeros(q)
    ws = torch.empty(_hip.decode_workspace_bytes(len(LENS), 32, 128, 16), dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)
    static_q = q.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        paged_decode_launch(static_q, cache, 128 ** -0.5, 16, out=out, workspace=ws, counters=cnt)  # warm-up
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_launch(static_q, cache, 128 ** -0.5, 16, out=out, workspace=ws, counters=cnt)
    for qi in qs:
        static_q.copy_(qi)
        graph.replay()
        torch.cuda.synchronize()
        ref = paged_decode_launch(qi, cache, 128 ** -0.5, 16)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert int(cnt.abs().sum()) == 0
