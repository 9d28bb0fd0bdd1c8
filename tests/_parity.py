"""Shared helpers: seeded input builders and the parity criterion.

Parity criterion (north-star tolerance 2e-3 max-abs for fp16/bf16 outputs):
the kernel writes ``round_to_dtype(r_k)`` where ``r_k`` is its fp32 result;
the oracle's fp32 result is ``r_o``.  We require ``|r_k - r_o| <= 2e-3``,
checked as ``|out - r_o| <= 2e-3 + ulp(out)/2`` -- the final rounding to the
output dtype adds at most half an ulp and is not a kernel error.  Against the
oracle's own output in that dtype (``reference.py:140`` casts at the end) the
bound is ``2e-3 + ulp`` (each side rounds once); both are asserted
elementwise, and the worst of each per dtype is printed at the end of the run
(conftest.py).
"""

from __future__ import annotations

import math

import torch

TOL = 2e-3
_MANT = {torch.float16: 10, torch.bfloat16: 7}
_EMIN = {torch.float16: -14, torch.bfloat16: -126}


def ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Spacing of ``dtype`` numbers around ``|x|`` (normal range; subnormals use the min)."""
    ax = x.abs().clamp_min(1e-30)
    e = torch.floor(torch.log2(ax)).clamp_min(_EMIN[dtype])
    return torch.exp2(e - _MANT[dtype])


# Every assert_parity call of the session: (label, dtype, raw_max_abs,
# max_abs_vs_fp32).  conftest.py prints the worst per dtype at the end of the
# run, so the figures show under ``pytest -q`` too.
RECORDS: list[tuple[str, str, float, float]] = []


def parity(out: torch.Tensor, ref32: torch.Tensor, tol: float = TOL) -> dict:
    out32 = out.detach().float().cpu()
    r32 = ref32.detach().float().cpu()
    assert out32.shape == r32.shape, (out32.shape, r32.shape)
    assert torch.isfinite(out32).all(), "non-finite kernel output"
    diff = (out32 - r32).abs()
    mag = torch.maximum(out32.abs(), r32.abs())
    bound = tol + 0.5 * ulp(mag, out.dtype)
    # Against the oracle's own output in the output dtype (reference.py:140
    # casts at the end): both sides are rounded once, so a kernel within
    # `tol` of the fp32 result is within tol + one ulp of it.
    raw_diff = (out32 - r32.to(out.dtype).float()).abs()
    raw_bound = tol + ulp(mag, out.dtype)
    return {
        "raw_max_abs": raw_diff.max().item(),
        "max_abs_vs_fp32": diff.max().item(),
        "excess": (diff - bound).max().item(),
        "raw_excess": (raw_diff - raw_bound).max().item(),
    }


def assert_parity(out, ref32, tol: float = TOL, label: str = "") -> dict:
    rep = parity(out, ref32, tol)
    RECORDS.append((label, str(out.dtype).replace("torch.", ""), rep["raw_max_abs"], rep["max_abs_vs_fp32"]))
    print(f"{label} raw_max_abs={rep['raw_max_abs']:.3e} vs_fp32={rep['max_abs_vs_fp32']:.3e}", flush=True)
    assert rep["excess"] <= 0.0, f"{label}: parity failed {rep}"
    assert rep["raw_excess"] <= 0.0, f"{label}: parity against the oracle's {out.dtype} output failed {rep}"
    return rep


def make_paged(lens, num_kv_heads, head_dim, page_size, dtype, seed=0, scale=1.0, extra_pages=3,
               device="cpu", pad=0, poison=True):
    """K/V pages ~ N(0,1)*scale in ``dtype`` scattered by a seeded permutation.

    Returns (k_cache, v_cache, page_table, seq_lens).  Table entries past a
    sequence's pages hold ``pad``.  With ``poison`` the slots past each
    sequence's length in its last page get K = 30*scale and V = 500: a kernel
    that let them through the mask would be far off.
    """
    g = torch.Generator().manual_seed(seed)
    pages_per = [math.ceil(n / page_size) for n in lens]
    maxp = max(1, max(pages_per))
    num_pages = sum(pages_per) + extra_pages
    shape = (num_pages, page_size, num_kv_heads, head_dim)
    k = (torch.randn(shape, generator=g) * scale).to(dtype)
    v = (torch.randn(shape, generator=g) * scale).to(dtype)
    perm = torch.randperm(num_pages, generator=g)
    table = torch.full((len(lens), maxp), pad, dtype=torch.int32)
    at = 0
    for b, n in enumerate(pages_per):
        table[b, :n] = perm[at:at + n].to(torch.int32)
        at += n
        used = lens[b] - (n - 1) * page_size
        if poison and n > 0 and used < page_size and dtype.is_floating_point:
            last = int(table[b, n - 1])
            k[last, used:] = 30.0 * scale
            v[last, used:] = 500.0
    seq = torch.tensor(lens, dtype=torch.int32)
    return k.to(device), v.to(device), table.to(device), seq.to(device)


def make_query(batch, num_heads, head_dim, dtype, seed=1, scale=1.0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(batch, num_heads, head_dim, generator=g) * scale).to(dtype).to(device)


def make_varlen(lens, num_heads, num_kv_heads, head_dim, dtype, seed=0, scale=1.0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    total = sum(lens)
    q = (torch.randn(total, num_heads, head_dim, generator=g) * scale).to(dtype)
    k = (torch.randn(total, num_kv_heads, head_dim, generator=g) * scale).to(dtype)
    v = (torch.randn(total, num_kv_heads, head_dim, generator=g) * scale).to(dtype)
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0).tolist()), dtype=torch.int32)
    return q.to(device), k.to(device), v.to(device), cu.to(device)


def force_decode_knobs(monkeypatch, **knobs):
    """Make every decode wrapper call in this test launch with ``knobs``
    (``kernel``, ``num_warps``) on top of the launch it resolves; the choice
    reaches the library through the ``kernel`` / ``waves_per_group`` fields
    of ``fat_decode_args``."""
    import flashattntile_amd.kernels.decode as dec

    resolve = dec._resolve_config

    def forced(config, q, cache, max_len, total_pages, q_len=1):
        return {**resolve(config, q, cache, max_len, total_pages, q_len), **knobs}

    monkeypatch.setattr(dec, "_resolve_config", forced)


def force_prefill_knobs(monkeypatch, **knobs):
    """The same for the prefill wrappers (``kernel``, and ``rows`` for paged
    prefill)."""
    import flashattntile_amd.kernels.prefill as pre

    resolve = pre._resolve_config

    def forced(config, kind=None, signature=None, defaults=pre.DEFAULT_CONFIG):
        cfg = resolve(config, kind, signature, defaults)
        return {**cfg, **{k: v for k, v in knobs.items() if k in cfg}}

    monkeypatch.setattr(pre, "_resolve_config", forced)
