"""The C-ABI library: loads, exports every symbol include/fat_abi.h declares,
matches the ctypes struct layout, and rejects bad arguments before touching
the device (no kernel runs here)."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

from flashattntile_amd import _hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fat_abi.h"


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(fat_\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    assert _hip.is_loaded(), _hip.load_error()
    lib = _hip.lib()
    declared = _declared_functions()
    assert set(declared) == set(_hip.EXPORTED_SYMBOLS), declared
    for name in declared:
        assert hasattr(lib, name), name
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", str(_hip.LIB_PATH)], capture_output=True, text=True).stdout
        exported = set(re.findall(r"\bT (fat_\w+)", out))
        assert exported == set(declared)


def test_abi_version_and_workspace_sizes():
    lib = _hip.lib()
    assert lib.fat_abi_version() == _hip.ABI_VERSION
    assert _hip.decode_workspace_bytes(32, 32, 128, 1) == 0
    assert _hip.decode_workspace_bytes(32, 32, 128, 4) == 32 * 32 * 4 * 130 * 4
    assert _hip.prefill_workspace_bytes(1, 1, 128) >= 0
    # one int32 counter per (query row, head); the Python wrappers size
    # their cached counter buffers with this formula
    for rows, heads in ((0, 32), (1, 1), (32, 32), (128 * 4, 8)):
        assert _hip.decode_counters_bytes(rows, heads) == 4 * rows * heads


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layout_matches_ctypes(tmp_path):
    src = tmp_path / "layout.c"
    fields = {
        "fat_decode_args": [f for f, _ in _hip.DecodeArgs._fields_],
        "fat_prefill_args": [f for f, _ in _hip.PrefillArgs._fields_],
        "fat_prefill_paged_args": [f for f, _ in _hip.PrefillPagedArgs._fields_],
        "fat_quantize_args": [f for f, _ in _hip.QuantizeArgs._fields_],
        "fat_append_args": [f for f, _ in _hip.AppendArgs._fields_],
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for struct, names in fields.items():
        lines.append(f'  printf("{struct} size %zu\\n", sizeof({struct}));')
        for n in names:
            lines.append(f'  printf("{struct} {n} %zu\\n", offsetof({struct}, {n}));')
    lines.append("  return 0; }")
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        struct, name, val = line.split()
        got[(struct, name)] = int(val)
    for struct, cls in (("fat_decode_args", _hip.DecodeArgs), ("fat_prefill_args", _hip.PrefillArgs),
                        ("fat_prefill_paged_args", _hip.PrefillPagedArgs),
                        ("fat_quantize_args", _hip.QuantizeArgs), ("fat_append_args", _hip.AppendArgs)):
        assert got[(struct, "size")] == ctypes.sizeof(cls)
        for n, _ in cls._fields_:
            assert got[(struct, n)] == getattr(cls, n).offset, (struct, n)


def _err() -> str:
    return _hip.lib().fat_last_error().decode()


def test_decode_argument_errors_are_reported():
    lib = _hip.lib()
    assert lib.fat_paged_decode(None, None) == 1
    assert "NULL" in _err()
    a = _hip.DecodeArgs()
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 1
    assert "pointer is NULL" in _err()
    # Non-null fake pointers: every rejection below happens before any launch.
    for f in ("q", "k_cache", "v_cache", "page_table", "seq_lens", "out"):
        setattr(a, f, 0x1000)
    a.batch, a.num_heads, a.num_kv_heads, a.head_dim = 1, 4, 3, 128
    a.page_size, a.num_pages, a.max_pages, a.split_k = 16, 1, 1, 1
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 1 and "divisible" in _err()
    a.num_kv_heads = 2
    a.split_k = 65
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 1 and "split_k" in _err()
    a.split_k = 2
    a.q_dtype = a.kv_dtype = _hip.DT_F16
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 1 and "workspace" in _err()
    a.split_k = 1
    a.head_dim = 96
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 2 and "head_dim" in _err()
    a.head_dim = 128
    a.page_size = 0
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 1 and "page_size" in _err()
    # pages of 2 rows exist only for the generic kernel
    a.page_size, a.kernel = 2, _hip.KERNEL_DECODE_MFMA
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 2 and "GENERIC" in _err()
    a.page_size, a.kernel = 16, _hip.KERNEL_AUTO
    a.kv_dtype = _hip.DT_I8
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 1 and "scale" in _err()
    a.k_scale = a.v_scale = 0x2000
    a.num_heads, a.kernel = 16, _hip.KERNEL_DECODE_VALU  # 8-bit cache, GQA group 8
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 2 and "VALU decode takes int8/fp8" in _err()
    a.num_heads, a.kernel = 4, _hip.KERNEL_AUTO
    a.q_dtype = _hip.DT_F32  # fp32 queries take an fp32 cache only
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 2 and "kv_dtype" in _err()
    a.k_scale = a.v_scale = None
    a.kv_dtype = _hip.DT_F16
    a.q_dtype = 9
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 2 and "q_dtype" in _err()
    a.q_dtype = _hip.DT_F16
    a.kernel = 4
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 1 and "kernel" in _err()
    a.kernel, a.q_len = _hip.KERNEL_DECODE_VALU, 2
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 2 and "VALU" in _err()
    a.kernel = _hip.KERNEL_DECODE_GENERIC  # one query per sequence only
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 2 and "multi-token" in _err()
    a.kernel, a.q_len = _hip.KERNEL_AUTO, 0
    a.k_stride_slot = 3  # 6-byte rows: misaligned for 16-byte loads
    assert lib.fat_paged_decode(ctypes.byref(a), None) == 1 and "aligned" in _err()


def test_prefill_argument_errors_are_reported():
    lib = _hip.lib()
    assert lib.fat_prefill_varlen(None, None) == 1
    a = _hip.PrefillArgs()
    assert lib.fat_prefill_varlen(ctypes.byref(a), None) != 0
    assert _err()
    for f in ("q", "k", "v", "cu_seqlens_q", "cu_seqlens_k", "out"):
        setattr(a, f, 0x1000)
    a.batch, a.num_heads, a.num_kv_heads, a.head_dim, a.dtype = 1, 4, 2, 128, _hip.DT_F16
    a.kernel = 6
    assert lib.fat_prefill_varlen(ctypes.byref(a), None) == 1 and "kernel" in _err()
    p = _hip.PrefillPagedArgs()
    for f in ("q", "k_cache", "v_cache", "page_table", "seq_lens", "cu_seqlens_q", "out"):
        setattr(p, f, 0x1000)
    p.batch, p.num_heads, p.num_kv_heads, p.head_dim, p.dtype, p.page_size = 1, 4, 2, 128, _hip.DT_F16, 16
    p.num_pages, p.max_pages = 1, 1
    p.kernel = -1
    assert lib.fat_prefill_paged(ctypes.byref(p), None) == 1 and "kernel" in _err()
    p.kernel, p.rows = _hip.KERNEL_AUTO, 3
    assert lib.fat_prefill_paged(ctypes.byref(p), None) == 1 and "rows" in _err()


def _paged_sizes(lens_q, cap, dtype, d=128, h=32, hk=8, page=16, causal=1, kernel=0):
    p = _hip.PrefillPagedArgs()
    p.batch, p.total_q, p.num_heads, p.num_kv_heads, p.head_dim = len(lens_q), sum(lens_q), h, hk, d
    p.page_size, p.max_pages, p.num_pages = page, cap // page, len(lens_q) * cap // page
    p.max_seqlen_q, p.causal, p.dtype, p.kernel = max(lens_q), causal, dtype, kernel
    return p


def test_paged_prefill_staging_plan():
    """Which paged launches copy their K/V rows for the wide kernel (no
    device access: sizes only).  Long chunks at head_dim 128 do (fp16 causal
    from a mean of 4096 queries, bf16 from 2048, as the packed kernel
    choice); short chunks after long prefixes, head_dim 64, fp32, forced
    paged kernels and tables far larger than the queries do not."""
    lib = _hip.lib()
    need = lambda p: lib.fat_prefill_paged_workspace_bytes(ctypes.byref(p))  # noqa: E731
    f16, bf16 = _hip.DT_F16, _hip.DT_BF16
    kv = 8192 * 8 * 128 * 2
    assert need(_paged_sizes([8192], 8192, f16)) == 256 + 2 * kv
    assert need(_paged_sizes([8192], 8192, bf16)) > 3 * kv  # + the V pre-pass's fp16 copy
    assert need(_paged_sizes([2048] * 4, 2048, bf16)) > 0
    assert need(_paged_sizes([2048] * 4, 2048, f16)) == 0  # fp16 causal: mean below 4096
    assert need(_paged_sizes([2048] * 4, 2048, f16, causal=0)) > 0
    assert need(_paged_sizes([512] * 16, 4096, bf16)) == 0  # chunks of 512 after 3584
    assert need(_paged_sizes([8192], 8192, f16, d=64)) == 0
    assert need(_paged_sizes([8192], 8192, _hip.DT_F32)) == 0
    assert need(_paged_sizes([8192], 8192, f16, kernel=_hip.KERNEL_PREFILL_PINGPONG)) == 0
    assert need(_paged_sizes([8192], 65536, f16)) == 0  # table capacity 8x the queries
    assert need(_paged_sizes([100], 128, f16, h=8, hk=2, kernel=_hip.KERNEL_PREFILL_WIDE)) > 0


def test_paged_prefill_wide_needs_the_staging_workspace():
    lib = _hip.lib()
    p = _paged_sizes([100], 128, _hip.DT_F16, d=64, h=8, hk=2, kernel=_hip.KERNEL_PREFILL_WIDE)
    for f in ("q", "k_cache", "v_cache", "page_table", "seq_lens", "cu_seqlens_q", "out"):
        setattr(p, f, 0x1000)
    p.q_stride_t, p.q_stride_h, p.out_stride_t, p.out_stride_h = 8 * 64, 64, 8 * 64, 64
    p.k_stride_page, p.k_stride_slot, p.k_stride_head = 16 * 2 * 64, 2 * 64, 64
    p.v_stride_page, p.v_stride_slot, p.v_stride_head = 16 * 2 * 64, 2 * 64, 64
    assert lib.fat_prefill_paged(ctypes.byref(p), None) == 2 and "packed copies" in _err()
    p.head_dim = 128
    assert lib.fat_prefill_paged(ctypes.byref(p), None) == 2 and "packed copies" in _err()  # no workspace
    p.workspace = 0x1080
    assert lib.fat_prefill_paged(ctypes.byref(p), None) == 1 and "256-byte aligned" in _err()


def test_cache_stats_argument_errors():
    """fat_cache_stats rejects missing pointers and inconsistent sizes before
    any device access."""
    lib = _hip.lib()
    assert lib.fat_cache_stats(None, None) == 1
    a = _hip.CacheStatsArgs()
    assert lib.fat_cache_stats(ctypes.byref(a), None) == 1 and "NULL" in _err()
    a.seq_lens, a.page_table, a.out = 0x1000, 0x1000, 0x1000
    a.batch, a.max_pages, a.page_size, a.page_table_stride = 2, 4, 0, 4
    assert lib.fat_cache_stats(ctypes.byref(a), None) == 1 and "page_size" in _err()
    a.page_size, a.page_table_stride = 16, 3
    assert lib.fat_cache_stats(ctypes.byref(a), None) == 1 and "page_table_stride" in _err()


def test_prefill_args_block_fields():
    """prefill_args fills the fat_prefill_args block from the tensors
    (addresses, element strides, shape, dtype code, scale, kernel) without a
    launch; a head-strided output keeps its own strides."""
    q = torch.zeros(30, 8, 64, dtype=torch.bfloat16)
    k = torch.zeros(50, 2, 64, dtype=torch.bfloat16)
    v = torch.zeros(50, 2, 64, dtype=torch.bfloat16)
    cq = torch.tensor([0, 10, 30], dtype=torch.int32)
    ck = torch.tensor([0, 20, 50], dtype=torch.int32)
    out = torch.zeros(30, 8, 72, dtype=torch.bfloat16)[:, :, 4:68]
    ws = torch.zeros(512, dtype=torch.uint8)
    a = _hip.prefill_args(q, k, v, cq, ck, out, 20, 30, True, 0.125, workspace=ws,
                          kernel=_hip.KERNEL_PREFILL_PINGPONG)
    assert (a.q, a.k, a.v, a.out, a.workspace) == (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                                   ws.data_ptr())
    assert (a.cu_seqlens_q, a.cu_seqlens_k) == (cq.data_ptr(), ck.data_ptr())
    assert (a.q_stride_t, a.q_stride_h, a.k_stride_t, a.k_stride_h) == (512, 64, 128, 64)
    assert (a.out_stride_t, a.out_stride_h) == (8 * 72, 72)
    assert (a.batch, a.total_q, a.total_k, a.num_heads, a.num_kv_heads, a.head_dim) == (2, 30, 50, 8, 2, 64)
    assert (a.max_seqlen_q, a.max_seqlen_k, a.causal, a.dtype) == (20, 30, 1, _hip.DT_BF16)
    assert a.softmax_scale == 0.125 and a.kernel == _hip.KERNEL_PREFILL_PINGPONG
    assert _hip.prefill_args(q, k, v, cq, ck, q, 20, 30, False, 0.5).workspace is None


def test_quantize_argument_errors_are_reported():
    lib = _hip.lib()
    assert lib.fat_quantize_pages(None, None) == 1 and "required" in _err()
    a = _hip.QuantizeArgs()
    a.src, a.dst, a.scale = 0x1000, 0x2000, 0x3000
    a.num_pages, a.page_size, a.num_kv_heads, a.head_dim = 1, 0, 1, 128
    assert lib.fat_quantize_pages(ctypes.byref(a), None) == 1 and "positive" in _err()
    a.page_size = 16
    a.src_dtype, a.dst_dtype = _hip.DT_F16, _hip.DT_F16
    assert lib.fat_quantize_pages(ctypes.byref(a), None) == 2 and "dst_dtype" in _err()
    a.src_dtype, a.dst_dtype = _hip.DT_I8, _hip.DT_I8
    assert lib.fat_quantize_pages(ctypes.byref(a), None) == 2 and "src_dtype" in _err()
    # No pages: nothing to launch, success.
    a.src_dtype, a.num_pages = _hip.DT_F32, 0
    assert lib.fat_quantize_pages(ctypes.byref(a), None) == 0 and _err() == ""


def test_append_argument_errors_are_reported():
    lib = _hip.lib()
    assert lib.fat_append_kv(None, None) == 1 and "required" in _err()
    a = _hip.AppendArgs()
    for f in ("new_k", "new_v", "k_cache", "v_cache", "page_table", "seq_lens"):
        setattr(a, f, 0x1000)
    a.batch, a.num_kv_heads, a.head_dim, a.page_size, a.num_pages, a.max_pages = 2, 2, 128, 16, 0, 4
    assert lib.fat_append_kv(ctypes.byref(a), None) == 1 and "positive" in _err()
    a.num_pages = 8
    a.max_pages = 1 << 28
    assert lib.fat_append_kv(ctypes.byref(a), None) == 1 and "overflows" in _err()
    a.max_pages = 4
    a.dtype = _hip.DT_I8
    assert lib.fat_append_kv(ctypes.byref(a), None) == 2 and "fp16 or bf16" in _err()
    a.dtype = _hip.DT_BF16
    a.quant_k_cache = 0x4000  # a quantised copy needs both code tensors and both scales
    a.quant_dtype = _hip.DT_I8
    assert lib.fat_append_kv(ctypes.byref(a), None) == 1 and "quantised copy" in _err()
    a.quant_v_cache, a.k_scale, a.v_scale = 0x5000, 0x6000, 0x7000
    a.quant_dtype = _hip.DT_F16
    assert lib.fat_append_kv(ctypes.byref(a), None) == 1 and "quantised copy" in _err()
    # Empty batch: nothing to launch, success.
    a.quant_dtype, a.batch = _hip.DT_FP8E4M3, 0
    assert lib.fat_append_kv(ctypes.byref(a), None) == 0 and _err() == ""


def test_integration_stubs_match_the_abi():
    """The ctypes stubs the integration guide shows a maintainer lay out
    their structs exactly as the bindings (and so the header) do."""
    text = (ROOT / "INTEGRATION.md").read_text()
    found = 0
    for block in re.findall(r"```python\n(.*?)```", text, re.S):
        for cls in ("DecodeArgs", "AppendArgs"):
            m = re.search(rf"class {cls}\(ctypes.Structure\):.*?\n\n", block, re.S)
            if not m:
                continue
            ns = {"ctypes": ctypes}
            exec(m.group(0), ns)  # the documentation's own struct definition
            stub, mine = ns[cls], getattr(_hip, cls)
            assert ctypes.sizeof(stub) == ctypes.sizeof(mine), cls
            for name, _ in mine._fields_:
                assert getattr(stub, name).offset == getattr(mine, name).offset, (cls, name)
            found += 1
    assert found == 2
