"""Split-K partitions merged inside the decode launch (ticket counters).

With ``split_counters`` the last partition workgroup of each (sequence,
query-head group) to finish merges the partitions by log-sum-exp; without
them ``decode_merge_kernel`` does it in a second launch.  Both take the
maximum over every partition first and then sum the partitions in order, so
they must agree bit for bit.  Every launch must leave its counters at zero
(the next launch and graph replays rely on it).
Reference semantics: flashattn_tile/kernels/decode.py:316-356.
"""

from __future__ import annotations

import pytest
import torch

from _parity import assert_parity, make_paged, make_query
from flashattntile_amd import DecodeLaunch, PagedKVCache, _hip
from oracle.reference import ref_attention_paged, ref_attention_paged_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"
KERNELS = {"valu": _hip.KERNEL_DECODE_VALU, "mfma": _hip.KERNEL_DECODE_MFMA, "generic": _hip.KERNEL_DECODE_GENERIC}


def _launch(q, cache, split, kernel, counters):
    out = torch.empty_like(q)
    ws = torch.empty(_hip.decode_workspace_bytes(q.shape[0], q.shape[-2], q.shape[-1], split), dtype=torch.uint8,
                     device=DEV)
    _hip.paged_decode(q, cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, out, cache.page_size,
                      q.shape[-1] ** -0.5, split, workspace=ws, kernel=kernel, counters=counters)
    return out


@pytest.mark.parametrize("split", [2, 5, 16, 17, 33, 64])
@pytest.mark.parametrize("kernel", list(KERNELS))
@pytest.mark.parametrize("h,hk", [(32, 8), (32, 1)])
def test_in_launch_merge_matches_merge_kernel(h, hk, kernel, split):
    label = f"split merge {kernel} H{h}/{hk} S{split}"
    print(label, flush=True)
    lens = [1, 700, 0, 4096, 33]  # an empty sequence, and more partitions than pages
    k, v, pt, sl = make_paged(lens, hk, 128, 16, torch.float16, seed=split + h + hk, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, 16)
    q = make_query(len(lens), h, 128, torch.float16, seed=split, device=DEV)
    counters = torch.zeros(_hip.decode_ticket_count(len(lens), h), dtype=torch.int32, device=DEV)
    fused = _launch(q, cache, split, KERNELS[kernel], counters)
    second = _launch(q, cache, split, KERNELS[kernel], None)
    again = _launch(q, cache, split, KERNELS[kernel], counters)  # the counters were left at zero
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0, f"{label}: counters not reset"
    assert torch.equal(fused, again), f"{label}: second fused launch differs"
    assert torch.equal(fused, second), f"{label}: differs from the merge kernel"
    assert torch.all(fused[2] == 0), f"{label}: empty sequence not zero"
    keep = [0, 1, 3, 4]  # the oracle takes no empty sequence
    ref = ref_attention_paged(q[keep].cpu(), k.cpu(), v.cpu(), pt[keep].cpu(), sl[keep].cpu(), return_fp32=True)
    assert_parity(fused[keep], ref, label=label)


def test_in_launch_merge_multi_token():
    print("split merge multi-token T3", flush=True)
    lens = [300, 2000]
    k, v, pt, sl = make_paged(lens, 8, 128, 16, torch.bfloat16, seed=7, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, 16)
    g = torch.Generator(device=DEV).manual_seed(8)
    q = torch.randn(2, 3, 32, 128, generator=g, device=DEV).to(torch.bfloat16)
    counters = torch.zeros(_hip.decode_ticket_count(2, 32, 3), dtype=torch.int32, device=DEV)
    fused = _launch(q, cache, 6, _hip.KERNEL_AUTO, counters)
    second = _launch(q, cache, 6, _hip.KERNEL_AUTO, None)
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0
    assert torch.equal(fused, second)
    for b, n in enumerate(lens):
        ref = ref_attention_paged_prefill(q[b].cpu(), k.cpu(), v.cpu(), pt[b:b + 1].cpu(), sl[b:b + 1].cpu(),
                                          [0, 3], return_fp32=True)
        assert_parity(fused[b], ref, label=f"multi-token fused b{b}")


def test_counters_shared_by_launches_of_different_shapes():
    """One stream's counters serve launches of any split and batch in turn."""
    print("split merge shared counters", flush=True)
    counters = torch.zeros(_hip.decode_ticket_count(8, 32), dtype=torch.int32, device=DEV)
    for i, (lens, split) in enumerate((([5000] * 8, 12), ([64, 3000], 3), ([9000], 40), ([128] * 4, 2))):
        k, v, pt, sl = make_paged(lens, 8, 128, 16, torch.float16, seed=30 + i, device=DEV)
        cache = PagedKVCache(k, v, pt, sl, 16)
        q = make_query(len(lens), 32, 128, torch.float16, seed=40 + i, device=DEV)
        fused = _launch(q, cache, split, _hip.KERNEL_AUTO, counters)
        torch.cuda.synchronize()
        assert int(counters.abs().sum()) == 0, f"launch {i}: counters not reset"
        ref = ref_attention_paged(q.cpu(), k.cpu(), v.cpu(), pt.cpu(), sl.cpu(), return_fp32=True)
        assert_parity(fused, ref, label=f"shared counters launch {i} S{split}")


def test_counters_are_validated():
    lens = [100]
    k, v, pt, sl = make_paged(lens, 8, 128, 16, torch.float16, seed=1, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, 16)
    q = make_query(1, 32, 128, torch.float16, seed=2, device=DEV)
    with pytest.raises(ValueError, match="counters"):
        _launch(q, cache, 4, _hip.KERNEL_AUTO, torch.zeros(31, dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError, match="counters"):
        _launch(q, cache, 4, _hip.KERNEL_AUTO, torch.zeros(32, dtype=torch.int64, device=DEV))


def test_plan_with_counters_in_a_graph():
    """DecodeLaunch owns its counters, so a captured plan merges inside the
    launch; every replay (with eager work between) matches an eager run."""
    print("split merge plan graph", flush=True)
    lens = [17, 1000, 255, 4096]
    k, v, pt, sl = make_paged(lens, 8, 128, 16, torch.float16, seed=11, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, 16)
    q = make_query(len(lens), 32, 128, torch.float16, seed=12, device=DEV)
    plan = DecodeLaunch(q, cache, softmax_scale=0.088, config={"split_k": 8})
    assert plan.counters is not None
    out = torch.empty_like(q)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        plan.run(q, out)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run(q, out)
    torch.cuda.synchronize()
    g = torch.Generator(device=DEV).manual_seed(13)
    for i in range(4):
        q.copy_(torch.randn(q.shape, generator=g, device=DEV).half())
        graph.replay()
        ref = torch.empty_like(q)
        plan.run(q, ref)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        assert int(plan.counters.abs().sum()) == 0, f"replay {i}: counters not reset"
