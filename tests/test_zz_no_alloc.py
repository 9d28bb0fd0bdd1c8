"""The allocation-free decode entry ``fat_paged_decode_noalloc``, through the
C ABI (ctypes), against ``fat_paged_decode`` with a caller workspace.

Both run the same kernels with the same launch, so the outputs must be
bit-identical.  Two calls in a row share the library's device array, the
second with a smaller input; split-K is on, so the array carries the
partials each time.  A launch whose workspace would exceed the array is
rejected with an error before anything runs.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from _parity import assert_parity, make_paged, make_query
from flashattntile_amd import _hip
from oracle.reference import ref_attention_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both(lens, h, hk, split_k, q_dtype=torch.float16, seed=0):
    k, v, pt, sl = make_paged(lens, hk, 128, 16, q_dtype, seed=seed, device=DEV)
    q = make_query(len(lens), h, 128, q_dtype, seed=seed + 1, device=DEV)
    ws = torch.empty(_hip.decode_workspace_bytes(len(lens), h, 128, split_k), dtype=torch.uint8, device=DEV)
    out_ref = torch.empty_like(q)
    out_na = torch.full_like(q, float("nan"))
    stream = _hip.current_stream_handle(q.device)
    a = _hip.decode_args(q, k, v, pt, sl, out_ref, 16, 128 ** -0.5, split_k, workspace=ws)
    _hip.decode_with_args(a, stream)
    b = _hip.decode_args(q, k, v, pt, sl, out_na, 16, 128 ** -0.5, split_k, workspace=None)
    rc = _hip.lib().fat_paged_decode_noalloc(ctypes.byref(b), ctypes.c_void_p(stream))
    assert rc == 0, _hip.lib().fat_last_error().decode()
    torch.cuda.synchronize()
    ref = ref_attention_paged(q.cpu(), k.cpu(), v.cpu(), pt.cpu(), sl.cpu(), return_fp32=True)
    return out_na, out_ref, ref


def test_noalloc_captured_in_a_graph_replays_like_the_allocating_entry():
    """A split-K fat_paged_decode_noalloc call captured in a HIP graph: the
    graph holds no allocation (the partials live in the library's array),
    and each replay, after q and seq_lens change in place on the device,
    equals fat_paged_decode with a caller workspace bit for bit."""
    print("noalloc: graph capture, B4 split 4", flush=True)
    lens = [700, 33, 4096, 1500]
    split = 4
    k, v, pt, sl = make_paged(lens, 8, 128, 16, torch.float16, seed=11, device=DEV)
    q = make_query(len(lens), 32, 128, torch.float16, seed=12, device=DEV)
    out = torch.empty_like(q)
    a = _hip.decode_args(q, k, v, pt, sl, out, 16, 128 ** -0.5, split)
    lib = _hip.lib()

    def launch():
        rc = lib.fat_paged_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(_hip.current_stream_handle(q.device)))
        assert rc == 0, lib.fat_last_error().decode()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the graph (resolves the array once)
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    torch.cuda.synchronize()

    ws = torch.empty(_hip.decode_workspace_bytes(len(lens), 32, 128, split), dtype=torch.uint8, device=DEV)
    ref = torch.empty_like(q)
    b = _hip.decode_args(q, k, v, pt, sl, ref, 16, 128 ** -0.5, split, workspace=ws)
    g = torch.Generator(device=DEV).manual_seed(13)
    full = torch.tensor(lens, dtype=torch.int32, device=DEV)
    for i in range(4):
        q.copy_(torch.randn(q.shape, generator=g, device=DEV).half())
        sl.copy_(torch.randint(1, 1 << 30, sl.shape, generator=g, device=DEV, dtype=torch.int32) % full + 1)
        graph.replay()
        torch.cuda.synchronize()
        _hip.decode_with_args(b, _hip.current_stream_handle(q.device))
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
    assert_parity(out, ref_attention_paged(q.cpu(), k.cpu(), v.cpu(), pt.cpu(), sl.cpu(), return_fp32=True),
                  label="noalloc graph replay")


def test_noalloc_matches_the_allocating_entry_twice():
    print("noalloc: first call, B8 split 8", flush=True)
    out_na, out_ref, ref = _both([4096, 17, 900, 2000, 1, 333, 4095, 64], 32, 8, split_k=8, seed=3)
    assert torch.equal(out_na, out_ref)
    assert_parity(out_na, ref, label="noalloc call 1")
    print("noalloc: second call, smaller (B3 split 4, MQA)", flush=True)
    out_na, out_ref, ref = _both([100, 1000, 7], 32, 1, split_k=4, q_dtype=torch.bfloat16, seed=5)
    assert torch.equal(out_na, out_ref)
    assert_parity(out_na, ref, label="noalloc call 2")


def test_noalloc_without_split_and_oversized_workspace():
    print("noalloc: split 1 (no workspace) and an oversized launch", flush=True)
    out_na, out_ref, ref = _both([300, 40], 32, 8, split_k=1, seed=7)
    assert torch.equal(out_na, out_ref)
    # 1024 rows x 32 heads x 64 partitions x 130 floats = 1.09e9 B > 32 MiB: rejected, nothing launched
    q = torch.zeros(1024, 32, 128, dtype=torch.float16, device=DEV)
    k = torch.zeros(8, 16, 8, 128, dtype=torch.float16, device=DEV)
    pt = torch.zeros(1024, 1, dtype=torch.int32, device=DEV)
    sl = torch.ones(1024, dtype=torch.int32, device=DEV)
    out = torch.zeros_like(q)
    a = _hip.decode_args(q, k, k, pt, sl, out, 16, 1.0, 64)
    rc = _hip.lib().fat_paged_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(_hip.current_stream_handle(q.device)))
    assert rc == 1 and "at most 33554432" in _hip.lib().fat_last_error().decode()
    torch.cuda.synchronize()
    assert torch.all(out == 0)
