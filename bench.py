"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline (BASELINE.json ``metric``, configs[1]): fp16 single-query paged
decode, B=32, ctx 4096 for every sequence, 32 query / 8 KV heads, head_dim
128, page_size 16, K/V ~ N(0,1) scattered through a seeded permutation of
the page pool.  ``value`` is decode GB/s = algorithmic bytes (q + K + V + o,
flashattn_tile/autotune.py:76-106) / measured time, inputs resident in HBM.
Two copies of the 537 MB pool alternate between steps so the 256 MB
Infinity Cache cannot serve a step from the previous one.

A step is one ``fat_paged_decode`` call through the C ABI (decode kernel,
plus the log-sum-exp merge kernel when split_k > 1); HIP events on the
launch stream bracket the K timed steps.  Split-K / waves-per-workgroup are
chosen among a few candidates during warm-up (timed the same way) and
reported in ``config``.  The prefill leg (causal varlen, seq 8192, 32/8
heads, D128, fp16) is reported under ``prefill``.  ``cpu_baseline`` times the
fp32 oracle (oracle/reference.py) on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"f16": 2516.6, "bf16": 2516.6}


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--legs", default="decode,prefill,cpu",
                    help="comma list of decode, prefill, cpu (the JSON line needs decode)")
    ap.add_argument("--tune", action="store_true",
                    help="time a few split_k / waves candidates in warm-up and keep the fastest")
    ap.add_argument("--split-k", type=int, default=0, help="force split_k (0 = pick during warm-up)")
    ap.add_argument("--waves", type=int, default=0, help="force waves per workgroup (0 = pick)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 1 GiB copy kernel (torch.neg on fp32) three times, the known-size "
                         "reference that rocprofv3 FETCH_SIZE / WRITE_SIZE readings are scaled by")
    return ap.parse_args()


def copy_calibration(device, nbytes=1 << 30):
    """A plain elementwise copy of known size: reads and writes ``nbytes``."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    return nbytes


def _decode_inputs(batch, ctx, hq, hkv, d, page, dtype, seed, device, copies=2):
    g = torch.Generator(device="cpu").manual_seed(seed)
    pages_per = (ctx + page - 1) // page
    num_pages = batch * pages_per
    table = torch.randperm(num_pages, generator=g).to(torch.int32).view(batch, pages_per).to(device)
    lens = torch.full((batch,), ctx, dtype=torch.int32, device=device)
    q = torch.randn(batch, hq, d, generator=g).to(dtype).to(device)
    gd = torch.Generator(device=device).manual_seed(seed + 1)
    pools = []
    for _ in range(copies):
        k = torch.randn((num_pages, page, hkv, d), generator=gd, device=device, dtype=torch.float32).to(dtype)
        v = torch.randn((num_pages, page, hkv, d), generator=gd, device=device, dtype=torch.float32).to(dtype)
        pools.append((k, v))
    return q, pools, table, lens


def _time_steps(fn, steps, warmup, stream):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def bench_decode(args, device):
    from flashattntile_amd import _hip
    from flashattntile_amd.autotune import bytes_decode_paged, decode_split_k

    B, CTX, HQ, HKV, D, P = 32, 4096, 32, 8, 128, 16
    dtype = torch.float16
    q, pools, table, lens = _decode_inputs(B, CTX, HQ, HKV, D, P, dtype, seed=1, device=device)
    out = torch.empty_like(q)
    nbytes = bytes_decode_paged([CTX] * B, HQ, HKV, D)
    scale = D ** -0.5
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)
    ws = torch.empty(_hip.decode_workspace_bytes(B, HQ, D, 64), dtype=torch.uint8, device=device)

    def make(split, waves):
        def step(i):
            k, v = pools[i % len(pools)]
            _hip.paged_decode(q, k, v, table, lens, out, P, scale, split, workspace=ws, stream=handle,
                              waves_per_group=waves)
        return step

    if args.tune:
        cands = [(s, w) for s in (1, 2, 3, 4, 8) for w in (4, 8)]
    else:
        cands = [(args.split_k or decode_split_k(B, HQ, HKV, (CTX + P - 1) // P), args.waves or 0)]
    tuning = {}
    if len(cands) > 1:
        for cand in cands:
            tuning[cand] = _time_steps(make(*cand), max(5, args.warmup // 4), 2, stream)
    s, w = min(tuning, key=tuning.get) if tuning else cands[0]
    torch.cuda.synchronize()
    ms = _time_steps(make(s, w), args.steps, args.warmup, stream)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "ms": ms,
        "gbs": gbs,
        "bytes": nbytes,
        "split_k": s,
        "waves_per_group": w,
        "tuning_ms": {f"sk{a}_w{b}": round(t, 5) for (a, b), t in tuning.items()},
        "shape": {"batch": B, "ctx": CTX, "num_heads": HQ, "num_kv_heads": HKV, "head_dim": D, "page_size": P},
    }


def bench_prefill(args, device, seq=8192):
    from flashattntile_amd import _hip
    from flashattntile_amd.autotune import flops_attention

    HQ, HKV, D = 32, 8, 128
    dtype = torch.float16
    g = torch.Generator(device=device).manual_seed(7)
    q = torch.randn(seq, HQ, D, generator=g, device=device).to(dtype)
    k = torch.randn(seq, HKV, D, generator=g, device=device).to(dtype)
    v = torch.randn(seq, HKV, D, generator=g, device=device).to(dtype)
    cu = torch.tensor([0, seq], dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    ws_bytes = _hip.prefill_workspace_bytes(seq, HKV, D)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)

    def step(i):
        _hip.prefill_varlen(q, k, v, cu, cu, out, seq, seq, True, D ** -0.5, workspace=ws, stream=handle)

    steps = max(5, args.steps // 10)
    ms = _time_steps(step, steps, max(3, args.warmup // 4), stream)
    flops = flops_attention(HQ, D, seq, seq, causal=True)
    tflops = flops / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tflops, "flops": flops, "seq": seq, "steps": steps,
            "mfma_peak_tflops": MFMA_PEAK_TFLOPS["f16"], "frac": tflops / MFMA_PEAK_TFLOPS["f16"]}


def cpu_baseline_decode(budget_s=12.0):
    """fp32 oracle (oracle/reference.py) on a bounded sample of the decode
    workload: 4 of the 32 sequences (ctx 4096, 32/8 heads, D128, fp16 pages
    upcast), timed with perf_counter, min over repetitions within ~budget_s."""
    from flashattntile_amd.autotune import bytes_decode_paged
    from oracle.reference import ref_attention_paged

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        cores = os.cpu_count() or 1
    cores = min(cores, 16)
    torch.set_num_threads(cores)
    B, CTX, HQ, HKV, D, P = 4, 4096, 32, 8, 128, 16
    q, pools, table, lens = _decode_inputs(B, CTX, HQ, HKV, D, P, torch.float16, seed=1, device="cpu", copies=1)
    k, v = pools[0]
    for _ in range(2):
        ref_attention_paged(q, k, v, table, lens)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        ref_attention_paged(q, k, v, table, lens)
        times.append(time.perf_counter() - t0)
        if len(times) >= 21:
            break
    nbytes = bytes_decode_paged([CTX] * B, HQ, HKV, D)
    best = min(times)
    return {
        "value": nbytes / best / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"fp32 oracle ref_attention_paged on 4 of the 32 sequences (ctx 4096, 32/8 heads, D128, "
                  f"page 16, fp16 pages upcast); min of {len(times)} runs after 2 warm-ups",
        "ms": best * 1e3,
    }


def _traffic_from_profiles(workload: str):
    """HBM bytes per launch measured by rocprofv3 PMC runs, if committed."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as fh:
            data = json.load(fh)
        return data.get(workload, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); every MI355X box here has "
              "one GPU and the attention path needs no collectives.  Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    from flashattntile_amd import _hip

    if not _hip.is_loaded():
        print(f"bench.py: HIP library unavailable: {_hip.load_error()}", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        n = copy_calibration(device)
        print(f"# copy calibration: 3 x torch.neg over {n} bytes read + {n} bytes written", file=sys.stderr,
              flush=True)
    legs = set(args.legs.split(","))
    if args.no_prefill:
        legs.discard("prefill")
    if args.no_cpu_baseline:
        legs.discard("cpu")
    dec = None
    if "decode" in legs:
        dec = bench_decode(args, device)
        print(f"# decode: {dec['gbs']:.1f} GB/s ({dec['ms'] * 1e3:.1f} us/step, split_k={dec['split_k']}, "
              f"waves={dec['waves_per_group']})", file=sys.stderr, flush=True)
    pre = None
    if "prefill" in legs:
        try:
            pre = bench_prefill(args, device)
            print(f"# prefill seq8192: {pre['tflops']:.1f} TFLOP/s ({pre['ms']:.3f} ms)", file=sys.stderr,
                  flush=True)
        except RuntimeError as exc:  # prefill kernel not available in this build
            pre = {"error": str(exc)}
    cpu = None
    if "cpu" in legs:
        cpu = cpu_baseline_decode()
        print(f"# cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} cores", file=sys.stderr, flush=True)
    if dec is None:
        return

    workload = "decode_fp16_b32_ctx4096_h32_kv8_d128_p16"
    line = {
        "metric": "decode GB/s (% of 8 TB/s HBM) B=32 ctx4096; prefill TFLOP/s at seq 8192",
        "value": round(dec["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": workload,
            **dec["shape"],
            "split_k": dec["split_k"],
            "waves_per_group": dec["waves_per_group"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec["gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": _traffic_from_profiles(workload),
            "algorithmic_bytes": dec["bytes"],
        },
        "cpu_baseline": None if cpu is None else {k: v for k, v in cpu.items() if k != "ms"},
        "prefill": pre,
        "decode_tuning_ms": dec["tuning_ms"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
