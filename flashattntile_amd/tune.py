"""Fill the gfx950 tuned-config store on an MI355X.

``python -m flashattntile_amd.tune [--out FILE] [--only decode|prefill]``
times, for each benchmark shape, the untuned launch (what the wrappers pick
from their heuristics) against every candidate of
:func:`flashattntile_amd.autotune.build_config_space`, and stores the winner
under the wrapper's own signature, so ``config=None`` calls of that shape use
it.  The reference fills its store the same way from
``scripts/benchmark.py:240-270`` (``autotune(..., save=True)``).

Timing is that of a serving loop: launches back to back between two HIP
events (:func:`~flashattntile_amd.autotune.time_back_to_back`), the decode
launches cycling over enough copies of the cache that consecutive launches
cannot be served from the 256 MB MALL.  The fastest candidate is then timed
again, interleaved with the untuned launch over several rounds, and replaces
it only when it is at least ``--min-gain`` faster (default 3 %) in that
confirmation: candidates within a few percent of each other, or a candidate
that is the untuned launch spelled out, keep the untuned entry.

Shapes (synthetic, seeded, N(0, 1) values, randomly permuted page pools):
decode fp16 32/8 heads D128 P16 for B in {1, 8, 32, 128} x ctx in {128,
1024, 4096, 16384}; int8 and fp8 decode B128 ctx16384; B1 ctx131072; MQA
32/1 B32 ctx4096; 4-token decode B32 ctx4096; bf16 and D64 decode B32
ctx4096; the skewed batch of 64 log-uniform lengths in [16, 65536] (the
benchmark's own draw); causal prefill of one fp16
sequence, L in {512, ..., 8192}; paged prefill L8192 at page size 16.
"""

from __future__ import annotations

import argparse
import math
import json
import statistics
import sys

import torch

from . import _hip
from .autotune import (TUNED_CONFIGS_PATH, autotune, build_config_space, bytes_decode_paged, decode_partition,
                       decode_signature, flops_attention, initialize_store, prefill_paged_signature,
                       prefill_signature, save_best, time_back_to_back)
from .kernels.decode import merge_counters, paged_decode_launch
from .kernels.prefill import paged_prefill_launch, prefill_launch
from .paging import PagedKVCache
from .quant import quantize_cache

# (batch, ctx, query heads, KV heads, quantised dtype, q_len[, head_dim, dtype])
DECODE_SHAPES = [(b, ctx, 32, 8, None, 1) for b in (1, 8, 32, 128) for ctx in (128, 1024, 4096, 16384)] + [
    (128, 16384, 32, 8, torch.int8, 1),
    (128, 16384, 32, 8, torch.float8_e4m3fn, 1),
    (1, 131072, 32, 8, None, 1),
    (32, 4096, 32, 1, None, 1),
    (32, 4096, 32, 8, None, 4),
    (32, 4096, 32, 8, None, 1, 128, torch.bfloat16),
    (32, 4096, 32, 8, None, 1, 64, torch.float16),
]
PREFILL_LENS = (512, 1024, 2048, 4096, 8192)
D, P = 128, 16


def skewed_lens() -> list[int]:
    """The long-context stress config's skewed batch, as
    ``bench.py --all-configs`` draws it: 64 log-uniform lengths in [16, 65536]
    (seed 64)."""
    g = torch.Generator().manual_seed(64)
    logs = torch.rand(64, generator=g) * (math.log(65536) - math.log(16)) + math.log(16)
    return [int(math.exp(x)) for x in logs.tolist()]


# the skewed batch: (batch, "skewed", query heads, KV heads, quantised dtype, q_len)
DECODE_SHAPES.append((64, "skewed", 32, 8, None, 1))


def _ragged_cache(lens: list[int], hkv: int, gen: torch.Generator, device, d: int = D,
                  dtype=torch.float16) -> PagedKVCache:
    """A paged cache holding sequences of the given lengths, pages randomly
    permuted over one pool."""
    per = [-(-n // P) for n in lens]
    num_pages = sum(per)
    perm = torch.randperm(num_pages, generator=gen, device=device).to(torch.int32)
    table = torch.zeros(len(lens), max(per), dtype=torch.int32, device=device)
    at = 0
    for b, n in enumerate(per):
        table[b, :n] = perm[at:at + n]
        at += n
    k = torch.randn(num_pages, P, hkv, d, generator=gen, device=device, dtype=torch.float32).to(dtype)
    v = torch.randn(num_pages, P, hkv, d, generator=gen, device=device, dtype=torch.float32).to(dtype)
    return PagedKVCache(k_cache=k, v_cache=v, page_table=table,
                        seq_lens=torch.tensor(lens, dtype=torch.int32, device=device), page_size=P)


def _paged_cache(batch: int, ctx: int, hkv: int, gen: torch.Generator, device, d: int = D,
                 dtype=torch.float16) -> PagedKVCache:
    pages = -(-ctx // P)
    num_pages = batch * pages
    perm = torch.randperm(num_pages, generator=gen, device=device).to(torch.int32)
    k = torch.randn(num_pages, P, hkv, d, generator=gen, device=device, dtype=torch.float32).to(dtype)
    v = torch.randn(num_pages, P, hkv, d, generator=gen, device=device, dtype=torch.float32).to(dtype)
    return PagedKVCache(k_cache=k, v_cache=v, page_table=perm.view(batch, pages).contiguous(),
                        seq_lens=torch.full((batch,), ctx, dtype=torch.int32, device=device), page_size=P)


MALL_BYTES = 256 << 20


def _copies(pool_bytes: int) -> int:
    """Cache copies to cycle (at least 1 GiB in all, at most 16) so that
    back-to-back launches read from HBM, as the benchmark's do."""
    return max(1, min(16, -(-4 * MALL_BYTES // max(1, pool_bytes))))


def _timer(fn):
    return time_back_to_back(fn, warmup=3, reps=5, per_rep=20)


def _pick(problem: dict, rows: list[dict], default: dict, keys, min_gain: float,
          rounds: int = 3) -> tuple[dict, dict]:
    """The fastest candidate if, timed again interleaved with the untuned
    launch over ``rounds`` rounds, it beats it by at least ``min_gain``."""
    best = {k: rows[0][k] for k in keys}
    base = {k: default.get(k) for k in keys}
    t_base, t_best = [], []
    for _ in range(rounds):
        t_base += _timer(lambda: problem["runner"](base))
        t_best += _timer(lambda: problem["runner"](best))
    ms_base, ms_best = statistics.median(t_base), statistics.median(t_best)
    chosen, ms = (best, ms_best) if ms_base > ms_best * (1.0 + min_gain) else (base, ms_base)
    metrics = {"latency_ms": ms, "default_ms": ms_base, "best_ms": ms_best,
               "gbytes_per_s": problem["bytes"] / (ms * 1e-3) / 1e9,
               "tflops": problem["flops"] / (ms * 1e-3) / 1e12}
    return chosen, metrics


def tune_decode(device, out_path, min_gain: float) -> None:
    for shape in DECODE_SHAPES:
        batch, ctx, hq, hkv, qdt, q_len = shape[:6]
        d, dtype = shape[6:] if len(shape) > 6 else (D, torch.float16)
        lens = skewed_lens() if ctx == "skewed" else [ctx] * batch
        gen = torch.Generator(device=device).manual_seed(batch * 7919 + max(lens))
        pool_bytes = sum(lens) * hkv * d * 2 * (1 if qdt is not None else 2)
        caches, scale_list = [], []
        for _ in range(_copies(pool_bytes)):
            cache = (_ragged_cache(lens, hkv, gen, device, d, dtype) if ctx == "skewed"
                     else _paged_cache(batch, ctx, hkv, gen, device, d, dtype))
            scales = None
            if qdt is not None:
                cache, scales = quantize_cache(cache, "int8" if qdt == torch.int8 else "fp8")
            caches.append(cache)
            scale_list.append(None if scales is None else {"k": scales.k, "v": scales.v})
        cache = caches[0]
        qshape = (batch, q_len, hq, d) if q_len > 1 else (batch, hq, d)
        q = torch.randn(*qshape, generator=gen, device=device, dtype=torch.float32).to(dtype)
        out = torch.empty_like(q)
        ws = torch.empty(_hip.decode_workspace_bytes(batch * q_len, hq, d, 64), dtype=torch.uint8, device=device)
        max_pages = -(-max(lens) // P)
        total = sum(-(-n // P) for n in lens)
        quantized = qdt is not None
        split, pps = decode_partition(batch, hq, hkv, max_pages, total, quantized=quantized, q_len=q_len)
        default = {"split_k": split, "pages_per_split": pps, "num_warps": None, "kernel": None}
        cands = [default] + build_config_space("decode", batch=batch, num_heads=hq, num_kv_heads=hkv,
                                               max_pages=max_pages, total_pages=total, quantized=quantized,
                                               q_len=q_len)
        turn = [0]

        def run(cfg):
            i = turn[0] = (turn[0] + 1) % len(caches)
            paged_decode_launch(q, caches[i], d ** -0.5, cfg["split_k"], out=out, workspace=ws,
                                scales=scale_list[i], waves_per_group=cfg["num_warps"],
                                pages_per_split=cfg["pages_per_split"], kernel=cfg["kernel"],
                                counters=merge_counters(q, cfg["split_k"]))

        nbytes = bytes_decode_paged(lens, hq * q_len, hkv, d, kv_elem_bytes=1 if quantized else 2,
                                    page_size=P, quantized=quantized)
        sig = decode_signature(batch, hq, hkv, d, P, max(lens), total, cache.k_cache.dtype, q_len)
        problem = {"kind": "decode", "signature": sig, "runner": run, "bytes": nbytes,
                   "flops": 4 * hq * q_len * d * sum(lens)}
        rows = autotune(problem, cands, save=False, timer=_timer)
        cfg, metrics = _pick(problem, rows, default, list(default), min_gain)
        save_best("decode", sig, cfg, metrics, path=out_path)
        print(json.dumps({"decode": sig, "config": cfg, "copies": len(caches),
                          **{k: round(v, 5) for k, v in metrics.items()}}), flush=True)
        del cache, caches, scale_list, q, out, ws
        torch.cuda.empty_cache()


def tune_prefill(device, out_path, min_gain: float) -> None:
    hq, hkv = 32, 8
    for L in PREFILL_LENS + (-8192,):
        paged = L < 0
        L = abs(L)
        gen = torch.Generator(device=device).manual_seed(L)
        q = torch.randn(L, hq, D, generator=gen, device=device, dtype=torch.float16)
        cu = torch.tensor([0, L], dtype=torch.int32, device=device)
        out = torch.empty_like(q)
        flops = flops_attention(hq, D, L, L, causal=True)
        default = {"kernel": None}
        cands = [default] + build_config_space("prefill_paged" if paged else "prefill")
        if paged:
            cache = _paged_cache(1, L, hkv, gen, device)
            sig = prefill_paged_signature(1, hq, hkv, D, P, L, True)

            def run(cfg):
                paged_prefill_launch(q, cache, cu, L, True, D ** -0.5, out=out, kernel=cfg["kernel"])
        else:
            k = torch.randn(L, hkv, D, generator=gen, device=device, dtype=torch.float16)
            v = torch.randn(L, hkv, D, generator=gen, device=device, dtype=torch.float16)
            sig = prefill_signature(1, hq, hkv, D, L, L, True)

            def run(cfg):
                prefill_launch(q, k, v, cu, cu, L, L, True, D ** -0.5, out=out, kernel=cfg["kernel"])
        kind = "prefill_paged" if paged else "prefill"
        problem = {"kind": kind, "signature": sig, "runner": run, "flops": flops,
                   "bytes": 2 * L * (hq + 2 * hkv) * D * 2}
        rows = autotune(problem, cands, save=False, timer=_timer)
        cfg, metrics = _pick(problem, rows, default, ["kernel"], min_gain)
        save_best(kind, sig, cfg, metrics, path=out_path)
        print(json.dumps({kind: sig, "config": cfg, **{k: round(v, 5) for k, v in metrics.items()}}), flush=True)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", default=str(TUNED_CONFIGS_PATH), help="store file to write")
    ap.add_argument("--only", choices=("decode", "prefill"), default=None)
    ap.add_argument("--min-gain", type=float, default=0.03)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("tune: needs a ROCm GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda", 0)
    arch = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
    initialize_store(f"Tuned on {torch.cuda.get_device_name(device)} ({arch}) by python -m flashattntile_amd.tune: "
                     f"median of 5 samples of 20 back-to-back launches (HIP events), decode launches cycling "
                     f"over cache copies totalling >= 1 GiB (at most 16); the fastest candidate replaces the "
                     f"untuned launch only when >= {args.min_gain:.0%} faster when the two are timed again, "
                     f"interleaved, over 3 rounds.", path=args.out)
    if args.only in (None, "decode"):
        tune_decode(device, args.out, args.min_gain)
    if args.only in (None, "prefill"):
        tune_prefill(device, args.out, args.min_gain)
    torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
