"""HIP-graph capture of the sync-free entry points (paged_decode_launch,
prefill_launch, append_tokens(validate=False)).

A serving loop that captures its per-step launches replays them with no host
work per kernel.  Each test captures once, replays several times with the
program's own eager work and synchronisations between replays (new inputs
written in place), and checks every replay bit for bit against the same
launches run eagerly on the same inputs.
"""

from __future__ import annotations

import pytest
import torch

from _parity import make_paged, make_query, make_varlen
from flashattntile_amd import PagedKVCache, _hip
from flashattntile_amd.autotune import decode_partition
from flashattntile_amd.kernels.decode import paged_decode_launch
from flashattntile_amd.kernels.prefill import prefill_launch
from flashattntile_amd.paging import append_tokens
from flashattntile_amd.quant import quantize_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPLAYS = 4


def _capture(fn):
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # warm-up outside the graph
        fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("h,hk", [(32, 8), (32, 1)])
def test_decode_graph_replays_match_eager(dtype, h, hk):
    label = f"graph decode {dtype} H{h}/{hk}"
    print(label, flush=True)
    lens = [17, 1000, 255, 4096]
    k, v, pt, sl = make_paged(lens, hk, 128, 16, dtype, seed=h + hk, device=DEV)
    cache = PagedKVCache(k, v, pt, sl, 16)
    q = make_query(len(lens), h, 128, dtype, seed=3, device=DEV)
    split, pps = decode_partition(len(lens), h, hk, pt.shape[1], sum(-(-n // 16) for n in lens))
    split = max(split, 3)  # the merge kernel is part of the graph
    ws = torch.empty(_hip.decode_workspace_bytes(len(lens), h, 128, split), dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)
    graph = _capture(lambda: paged_decode_launch(q, cache, 0.088, split, out=out, workspace=ws,
                                                 pages_per_split=pps))
    g = torch.Generator(device=DEV).manual_seed(5)
    for i in range(REPLAYS):
        q.copy_(torch.randn(q.shape, generator=g, device=DEV).to(dtype))
        graph.replay()
        ref = paged_decode_launch(q, cache, 0.088, split, pages_per_split=pps)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"{label}: replay {i}"


def test_prefill_graph_replays_match_eager():
    print("graph prefill", flush=True)
    lens = [300, 1, 1000]
    q, k, v, cu = make_varlen(lens, 32, 8, 128, torch.bfloat16, seed=9, device=DEV)
    out = torch.empty_like(q)
    graph = _capture(lambda: prefill_launch(q, k, v, cu, cu, 1000, 1000, True, 128 ** -0.5, out=out))
    g = torch.Generator(device=DEV).manual_seed(6)
    for i in range(REPLAYS):
        q.copy_(torch.randn(q.shape, generator=g, device=DEV).to(q.dtype))
        v.copy_(torch.randn(v.shape, generator=g, device=DEV).to(v.dtype))
        graph.replay()
        ref = prefill_launch(q, k, v, cu, cu, 1000, 1000, True, 128 ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"graph prefill replay {i}"


@pytest.mark.parametrize("mode", [None, "fp8"])
def test_serving_step_graph_append_then_decode(mode):
    """One captured serving step: append one token per sequence (keeping an
    fp8 copy requantised when `mode`), then decode against the updated cache.
    seq_lens advances on the device, so each replay appends at the next
    position; an eager replica of the cache runs the same steps."""
    label = f"graph append+decode mode={mode}"
    print(label, flush=True)
    lens = [5, 31, 300, 77]
    h, hk, d = 32, 8, 128
    k, v, pt, sl = make_paged(lens, hk, d, 16, torch.float16, seed=11, device=DEV, extra_pages=0, poison=False)
    # room for REPLAYS + 1 more tokens per sequence: extend every table row
    need = max(-(-(n + REPLAYS + 2) // 16) for n in lens)
    extra = len(lens) * need
    k = torch.cat([k, torch.zeros(extra, 16, hk, d, dtype=k.dtype, device=DEV)])
    v = torch.cat([v, torch.zeros_like(k[-extra:])])
    table = torch.zeros(len(lens), need, dtype=torch.int32, device=DEV)
    base = k.shape[0] - extra
    for b, n in enumerate(lens):
        used = -(-n // 16)
        table[b, :used] = pt[b, :used]
        table[b, used:] = torch.arange(base + b * need + used, base + (b + 1) * need, dtype=torch.int32)
    cache = PagedKVCache(k, v, table, sl.clone(), 16)
    twin = PagedKVCache(k.clone(), v.clone(), table.clone(), sl.clone(), 16)
    mirror = twin_mirror = None
    if mode:
        mirror = quantize_cache(cache, mode)  # (qcache, scales)
        twin_mirror = quantize_cache(twin, mode)

    def parts(m):
        return (m[0].k_cache, m[0].v_cache, m[1].k, m[1].v)
    q = make_query(len(lens), h, d, torch.float16, seed=12, device=DEV)
    nk = torch.zeros(len(lens), hk, d, dtype=torch.float16, device=DEV)
    nv = torch.zeros_like(nk)
    split = 2
    ws = torch.empty(_hip.decode_workspace_bytes(len(lens), h, d, split), dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)

    def step(c, m, o):
        append_tokens(c, nk, nv, quantized=m, validate=False)
        return paged_decode_launch(q, c, d ** -0.5, split, out=o, workspace=ws)

    # capture on a scratch copy so the warm-up append does not move `cache`
    scratch = PagedKVCache(cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens.clone(), 16)
    graph = torch.cuda.CUDAGraph()
    step(scratch, mirror, out)  # warm-up (eager) on the scratch lengths
    torch.cuda.synchronize()
    # undo the warm-up's cache writes: restore pages and the quantised copy from the twin
    cache.k_cache.copy_(twin.k_cache)
    cache.v_cache.copy_(twin.v_cache)
    if mode:
        for dst, src in zip(parts(mirror), parts(twin_mirror)):
            dst.copy_(src)
    with torch.cuda.graph(graph):
        step(cache, mirror, out)
    torch.cuda.synchronize()
    assert torch.equal(cache.seq_lens, twin.seq_lens)  # capture launches nothing
    g = torch.Generator(device=DEV).manual_seed(13)
    for i in range(REPLAYS):
        nk.copy_(torch.randn(nk.shape, generator=g, device=DEV).half())
        nv.copy_(torch.randn(nv.shape, generator=g, device=DEV).half())
        q.copy_(torch.randn(q.shape, generator=g, device=DEV).half())
        graph.replay()
        ref = step(twin, twin_mirror, torch.empty_like(q))
        torch.cuda.synchronize()
        assert torch.equal(cache.seq_lens, twin.seq_lens), f"{label}: lengths after replay {i}"
        assert torch.equal(cache.k_cache, twin.k_cache) and torch.equal(cache.v_cache, twin.v_cache), \
            f"{label}: pages after replay {i}"
        if mode:
            for a, b in zip(parts(mirror), parts(twin_mirror)):
                assert torch.equal(a, b), f"{label}: quantised copy after replay {i}"
        assert torch.equal(out, ref), f"{label}: output after replay {i}"


@pytest.mark.parametrize("kind", ["fp16", "bf16-mqa", "int8", "multi"])
def test_decode_launch_plan_runs_match_wrappers(kind):
    """DecodeLaunch (plan once, run per step) gives the wrappers' bits, also
    after seq_lens and the pages change in place between runs."""
    from flashattntile_amd import DecodeLaunch, paged_decode_attention, paged_decode_attention_multi
    from flashattntile_amd import paged_decode_attention_fp8

    print(f"decode plan {kind}", flush=True)
    dtype = torch.bfloat16 if kind == "bf16-mqa" else torch.float16
    hk = 1 if kind == "bf16-mqa" else 8
    lens = [40, 700, 129, 2000]
    k, v, pt, sl = make_paged([n + 8 for n in lens], hk, 128, 16, dtype, seed=21, device=DEV, poison=False)
    sl.copy_(torch.tensor(lens, dtype=torch.int32))
    cache = PagedKVCache(k, v, pt, sl, 16)
    scales = None
    if kind == "int8":
        cache, scales = quantize_cache(cache, "int8")
    g = torch.Generator(device=DEV).manual_seed(22)
    shape = (len(lens), 3, 32, 128) if kind == "multi" else (len(lens), 32, 128)
    q = torch.randn(shape, generator=g, device=DEV).to(dtype)
    plan = DecodeLaunch(q, cache, softmax_scale=0.09, scales=scales, config={"split_k": 3})
    out = torch.empty_like(q)
    for i in range(3):
        q.copy_(torch.randn(shape, generator=g, device=DEV).to(dtype))
        cache.seq_lens.add_(2)  # the engine appends in place; the plan reads lengths on the device
        plan.run(q, out)
        if kind == "multi":
            ref = paged_decode_attention_multi(q, cache, softmax_scale=0.09, config={"split_k": 3})
        elif kind == "int8":
            ref = paged_decode_attention_fp8(q, cache, scales, softmax_scale=0.09, config={"split_k": 3})
        else:
            ref = paged_decode_attention(q, cache, softmax_scale=0.09, config={"split_k": 3})
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"decode plan {kind} run {i}"
    with pytest.raises(ValueError, match="shape"):
        plan.run(q[:2].contiguous())


@pytest.mark.parametrize("mode", [None, "int8"])
def test_append_launch_plan_matches_append_tokens(mode):
    """AppendLaunch.run (plan once) writes the same pages, lengths and
    quantised copy as append_tokens on a twin cache, step after step."""
    from flashattntile_amd import AppendLaunch

    print(f"append plan mode={mode}", flush=True)
    lens = [3, 64, 17, 200]
    k, v, pt, sl = make_paged([n + 8 for n in lens], 8, 128, 16, torch.bfloat16, seed=31, device=DEV,
                              poison=False)
    sl.copy_(torch.tensor(lens, dtype=torch.int32))
    cache = PagedKVCache(k, v, pt, sl, 16)
    twin = PagedKVCache(k.clone(), v.clone(), pt.clone(), sl.clone(), 16)
    m1 = quantize_cache(cache, mode) if mode else None
    m2 = quantize_cache(twin, mode) if mode else None
    plan = AppendLaunch(cache, quantized=m1)
    g = torch.Generator(device=DEV).manual_seed(32)
    for i in range(5):
        nk = torch.randn(len(lens), 8, 128, generator=g, device=DEV).bfloat16()
        nv = torch.randn(len(lens), 8, 128, generator=g, device=DEV).bfloat16()
        plan.run(nk, nv)
        append_tokens(twin, nk, nv, quantized=m2, validate=False)
        torch.cuda.synchronize()
        assert torch.equal(cache.seq_lens, twin.seq_lens) and torch.equal(cache.k_cache, twin.k_cache) \
            and torch.equal(cache.v_cache, twin.v_cache), f"append plan step {i}"
        if mode:
            assert torch.equal(m1[0].k_cache, m2[0].k_cache) and torch.equal(m1[1].v, m2[1].v), f"copy step {i}"
    with pytest.raises(ValueError, match="contiguous"):
        plan.run(nk.float(), nv)
