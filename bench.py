"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline (BASELINE.json ``metric``, configs[1]): fp16 single-query paged
decode, B=32, ctx 4096 for every sequence, 32 query / 8 KV heads, head_dim
128, page_size 16, K/V ~ N(0,1) scattered through a seeded permutation of
the page pool.  ``value`` is decode GB/s = algorithmic bytes (q + K + V + o,
flashattn_tile/autotune.py:76-106) / measured time, inputs resident in HBM.
Two copies of the 537 MB pool alternate between steps so the 256 MB
Infinity Cache cannot serve a step from the previous one.

A step is one ``fat_paged_decode`` call through the C ABI (the decode
kernel, plus the log-sum-exp merge kernel when split_k > 1); HIP events on
the launch stream bracket the K timed steps.  The launch (split_k, waves,
kernel) is the one the decode wrappers make for this shape: the tuned store's
entry, else the MI355X heuristic (``--tune`` times a few candidates).  The
prefill leg (causal varlen, seq 8192, 32/8 heads, D128, fp16 and bf16) is
reported under ``prefill`` with its own MFMA roofline.  ``cpu_baseline``
times the fp32 oracle (oracle/reference.py) on a bounded sample of the
headline workload on this host's cores.

``--all-configs`` measures every BASELINE.json configuration (decode sweep,
prefill lengths and mixed pack, int8/fp8 decode, long-context / skewed /
MQA / D64 / page-size stress), each next to a CPU-oracle sample, and writes
the table to ``--report`` (JSON) as well as stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

import torch

from flashattntile_amd.env import MI355X, peak_hbm_gbs, peak_mfma_tflops  # noqa: E402

HBM_PEAK_GBS = peak_hbm_gbs()
MFMA_PEAK_TFLOPS = peak_mfma_tflops("fp16")  # dense fp16 / bf16
VALU_FP32_PEAK_TFLOPS = MI355X["vector_fp32_tflops"]  # the generic fp32 prefill kernel's bound
MALL_BYTES = 256 << 20
FLUSH_BYTES = 512 << 20


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
    ap.add_argument("--split-k", type=int, default=0, help="force split_k (0 = heuristic)")
    ap.add_argument("--waves", type=int, default=0, help="force waves per workgroup (0 = library choice)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 1 GiB copy kernel (torch.neg on fp32) three times, the known-size "
                         "reference that rocprofv3 FETCH_SIZE / WRITE_SIZE readings are scaled by")
    ap.add_argument("--all-configs", action="store_true", help="measure every BASELINE.json configuration")
    ap.add_argument("--report", default="", help="with --all-configs: write the table to this JSON file")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU-oracle timing per sample")
    ap.add_argument("--only", default="", help="with --all-configs: run only rows whose name contains this text")
    ap.add_argument("--row-warm-ms", type=float, default=100.0,
                    help="with --all-configs: ms of each row's own launches run before its warm-up and timing "
                         "(0: time from an idle GPU, as the default run does)")
    ap.add_argument("--source-digests", action="store_true",
                    help="print the kernel-source digests that profiles/traffic.json entries are stamped with, "
                         "and exit")
    return ap.parse_args()


def _host() -> dict:
    """Affinity core count, os.cpu_count(), cgroup CPU quota and the full CPU
    model of this host (flashattntile_amd.env.host_info)."""
    from flashattntile_amd.env import host_info

    return host_info()


def _cores(info: dict | None = None) -> int:
    """Threads for the CPU baselines: every core this process may run on,
    bounded only by a cgroup CPU quota when one is set (more threads than the
    quota only time-slice)."""
    from flashattntile_amd.env import cpu_threads

    return cpu_threads(info or _host())


def copy_calibration(device, nbytes=1 << 30):
    """A plain elementwise copy of known size: reads and writes ``nbytes``."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    return nbytes


# ---------------------------------------------------------------------------
# Inputs and timing
# ---------------------------------------------------------------------------
def _paged_inputs(lens, hq, hkv, d, page, dtype, seed, device, copies=1, quant=None):
    """Seeded paged decode inputs: q, [(k, v, k_scale, v_scale)] x copies, table, seq_lens
    (device) and table, seq_lens (host).

    Tables are a seeded permutation of the pool; with ``quant`` the pages are
    drawn in fp32 and quantised per (page, KV head) by the product's
    ``quantize_kv_pages`` (int8: absmax/127, fp8: absmax/448)."""
    from flashattntile_amd.quant import quantize_kv_pages

    g = torch.Generator(device="cpu").manual_seed(seed)
    pages_per = [max(1, math.ceil(n / page)) for n in lens]
    maxp = max(pages_per)
    num_pages = sum(pages_per)
    perm = torch.randperm(num_pages, generator=g).to(torch.int32)
    table = torch.zeros(len(lens), maxp, dtype=torch.int32)
    at = 0
    for b, n in enumerate(pages_per):
        table[b, :n] = perm[at:at + n]
        at += n
    q = torch.randn(len(lens), hq, d, generator=g).to(dtype).to(device)
    gd = torch.Generator(device=device).manual_seed(seed + 1)
    pools = []
    for _ in range(copies):
        shape = (num_pages, page, hkv, d)
        if quant is None:
            k = torch.randn(shape, generator=gd, device=device, dtype=torch.float32).to(dtype)
            v = torch.randn(shape, generator=gd, device=device, dtype=torch.float32).to(dtype)
            pools.append((k, v, None, None))
        else:
            kf = torch.randn(shape, generator=gd, device=device, dtype=torch.float32)
            vf = torch.randn(shape, generator=gd, device=device, dtype=torch.float32)
            qk, qv, sk, sv, _ = quantize_kv_pages(kf, vf, quant)
            del kf, vf
            pools.append((qk, qv, sk, sv))
    seq = torch.tensor(lens, dtype=torch.int32)
    return q, pools, table.to(device), seq.to(device), table, seq


# --all-configs rows first run their own launches for this many ms of GPU
# time: each row follows seconds of CPU-oracle work that leave the GPU idle,
# and an HBM-bound launch reads up to 5 % slower in the first tens of ms of
# load after that (the memory side warms up).  The default run (the
# headline's contract: exactly `--warmup` untimed steps) keeps 0.
ROW_WARM_MS = 0.0


# The default run's extra sustained-load figures (the decode headline's
# `sustained` object, the prefill leg's main numbers) are timed after this
# many ms of the same launches.
SUSTAIN_MS = 200.0

# Seconds of GPU idle before a timed leg when no CPU baseline runs there.
IDLE_GAP_S = 10.0


def _prewarm(fn, stream, warm_ms=None):
    """Run ``fn`` back to back until ``warm_ms`` (default ROW_WARM_MS) of GPU
    time has passed."""
    warm_ms = ROW_WARM_MS if warm_ms is None else warm_ms
    done, n, i = 0.0, 4, 0
    while done < warm_ms:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn(i)
            i += 1
        e1.record(stream)
        e1.synchronize()
        done += e0.elapsed_time(e1)
        n = min(2 * n, 64)


def _time_steps(fn, steps, warmup, stream, warm_ms=None):
    """Back-to-back steps bracketed by two HIP events on ``stream``; ms/step."""
    _prewarm(fn, stream, warm_ms)
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
    return start.elapsed_time(end) / steps


def _time_steps_flushed(fn, steps, warmup, stream, flush):
    """Median over steps, each timed by its own event pair after a 512 MB
    read that evicts the Infinity Cache (for working sets the MALL could
    otherwise hold).  The flush only reads (a max-reduction into 8 bytes), so
    it leaves no dirty lines for the timed kernel to write back.  The median,
    not the mean: one launch delayed by the system (seen once at 0.7 ms for a
    30 us launch) would otherwise dominate a row of ~20 samples."""
    _prewarm(fn, stream)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    evs = []
    sink = torch.empty((), dtype=flush.dtype, device=flush.device)
    for i in range(steps):
        torch.amax(flush, dim=0, out=sink)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn(i)
        e1.record(stream)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in evs)


def _time_cpu(fn, budget_s, max_reps=21):
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return min(times), len(times)


# ---------------------------------------------------------------------------
# Headline legs
# ---------------------------------------------------------------------------
def _product_launch(q, pools, table, lens, page, max_len, total_pages, q_len=1):
    """What the decode wrappers launch for this shape (tuned store, else the
    heuristic): (split_k, pages_per_split, waves or 0, kernel code, source)."""
    from flashattntile_amd import PagedKVCache, _hip
    from flashattntile_amd.autotune import best_config, decode_signature
    from flashattntile_amd.kernels.decode import resolve_decode_config

    k, v = pools[0][0], pools[0][1]
    cache = PagedKVCache(k, v, table, lens, page)
    cfg = resolve_decode_config(q, cache, max_len, total_pages, q_len=q_len)
    sig = decode_signature(q.shape[0], q.shape[-2], k.shape[2], q.shape[-1], page, max_len, total_pages, k.dtype,
                           q_len)
    source = "tuned store" if best_config("decode", sig) else "heuristic"
    code = {None: _hip.KERNEL_AUTO, "valu": _hip.KERNEL_DECODE_VALU, "mfma": _hip.KERNEL_DECODE_MFMA}[cfg["kernel"]]
    return cfg["split_k"], cfg["pages_per_split"], cfg["num_warps"] or 0, code, source


def _auto_waves(kernel, batch, group, hkv, split, pps, max_pages, page):
    """Waves per workgroup the library picks when none is requested
    (fat_paged_decode in csrc/decode.hip)."""
    mfma = kernel == 2 or (kernel == 0 and group >= 8)
    wgs = split * hkv * batch * (-(-group // 32) if mfma else 1)
    per_wg = pps if pps > 0 else -(-max_pages // split)
    if not mfma:
        return 8 if wgs < 512 or per_wg * page >= 1024 else 4
    return 8 if wgs < 512 and per_wg * page >= 2048 else 4


def bench_decode(args, device):
    from flashattntile_amd import _hip
    from flashattntile_amd.kernels.decode import merge_counters
    from flashattntile_amd.autotune import bytes_decode_paged

    B, CTX, HQ, HKV, D, P = 32, 4096, 32, 8, 128, 16
    q, pools, table, lens, _, _ = _paged_inputs([CTX] * B, HQ, HKV, D, P, torch.float16, seed=1, device=device,
                                                copies=2)
    out = torch.empty_like(q)
    nbytes = bytes_decode_paged([CTX] * B, HQ, HKV, D)
    scale = D ** -0.5
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)
    ws = torch.empty(_hip.decode_workspace_bytes(B, HQ, D, 64), dtype=torch.uint8, device=device)

    pages = (CTX + P - 1) // P
    auto_split, auto_chunk, auto_waves, auto_kernel, source = _product_launch(q, pools, table, lens, P, CTX,
                                                                               B * pages)

    def make(split, waves, kernel):
        pps = auto_chunk if split == auto_split else 0
        cnt = merge_counters(q, split)  # split-K: the product's merge inside the decode launch

        def step(i):
            k, v, _, _ = pools[i % len(pools)]
            _hip.paged_decode(q, k, v, table, lens, out, P, scale, split, workspace=ws, stream=handle,
                              waves_per_group=waves, pages_per_split=pps, kernel=kernel, counters=cnt)
        return step

    if args.tune:
        cands = [(s, w, auto_kernel) for s in (1, 2, 3, 4, 8) for w in (4, 8)]
    elif args.split_k or args.waves:
        cands = [(args.split_k or auto_split, args.waves or auto_waves, auto_kernel)]
    else:
        cands = [(auto_split, auto_waves, auto_kernel)]
    tuning = {}
    if len(cands) > 1:
        for cand in cands:
            tuning[cand] = _time_steps(make(*cand), max(5, args.warmup // 4), 2, stream)
    s, w, kern = min(tuning, key=tuning.get) if tuning else cands[0]
    torch.cuda.synchronize()
    # The contract's timing: exactly `warmup` untimed steps, then `steps`.
    ms = _time_steps(make(s, w, kern), args.steps, args.warmup, stream, warm_ms=0.0)
    gbs = nbytes / (ms * 1e-3) / 1e9
    # Beside it, the same launches after SUSTAIN_MS of load (a serving loop's
    # steady state; the first tens of ms after an idle GPU run slower).
    ms_sus = _time_steps(make(s, w, kern), args.steps, 0, stream, warm_ms=SUSTAIN_MS)
    del pools
    return {
        "ms": ms,
        "gbs": gbs,
        "sustained_ms": ms_sus,
        "sustained_gbs": nbytes / (ms_sus * 1e-3) / 1e9,
        "bytes": nbytes,
        "split_k": s,
        "waves_per_group": w or _auto_waves(kern, B, HQ // HKV, HKV, s, auto_chunk if s == auto_split else 0,
                                            pages, P),
        "kernel": {0: "auto", 1: "valu", 2: "mfma"}[kern],
        "config_source": source if not (args.tune or args.split_k or args.waves) else "command line",
        "tuning_ms": {f"sk{a}_w{b}": round(t, 5) for (a, b, _), t in tuning.items()},
        "shape": {"batch": B, "ctx": CTX, "num_heads": HQ, "num_kv_heads": HKV, "head_dim": D, "page_size": P},
    }


def _prefill_case(lens, hq, hkv, d, dtype, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    total = sum(lens)
    q = torch.randn(total, hq, d, generator=g, device=device).to(dtype)
    k = torch.randn(total, hkv, d, generator=g, device=device).to(dtype)
    v = torch.randn(total, hkv, d, generator=g, device=device).to(dtype)
    cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens), 0).tolist(), dtype=torch.int32, device=device)
    return q, k, v, cu


def run_prefill(lens, dtype, device, steps, warmup, hq=32, hkv=8, d=128, seed=7, sustain_ms=None):
    """Prefill TFLOP/s over `steps` back-to-back launches after `warmup`
    untimed ones (the contract's timing; without `sustain_ms` the row's own
    ROW_WARM_MS of launches come first).  With `sustain_ms` the same steps are
    timed again after that many ms of load (`sustained_*`)."""
    from flashattntile_amd import _hip
    from flashattntile_amd.autotune import flops_attention_varlen

    q, k, v, cu = _prefill_case(lens, hq, hkv, d, dtype, seed, device)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)
    mx = max(lens)
    # The argument block is built once: a step is one ctypes call, so rows
    # whose kernel takes ~15 us are not bound by Python building it.  The
    # workspace is the one the product path (kernels/prefill.py:
    # prefill_launch) passes: what the library says this launch uses.
    args = _hip.prefill_args(q, k, v, cu, cu, out, mx, mx, True, d ** -0.5)
    need = _hip.prefill_varlen_workspace_bytes(args)
    ws = torch.empty(need, dtype=torch.uint8, device=device) if need else None
    if ws is not None:
        args.workspace = ws.data_ptr()
    launch, ref, hs = _hip.lib().fat_prefill_varlen, ctypes.byref(args), ctypes.c_void_p(handle)

    def step(i):
        if launch(ref, hs) != 0:
            raise RuntimeError(_hip.lib().fat_last_error().decode(errors="replace"))

    flops = flops_attention_varlen(hq, d, lens, lens, causal=True)
    extra = {"workspace_bytes": need}
    if sustain_ms is not None:
        ms = _time_steps(step, steps, warmup, stream, warm_ms=0.0)
        ms_sus = _time_steps(step, steps, 0, stream, warm_ms=sustain_ms)
        extra.update(sustained_ms=ms_sus, sustained_tflops=flops / (ms_sus * 1e-3) / 1e12)
    else:
        ms = _time_steps(step, steps, warmup, stream)
    tflops = flops / (ms * 1e-3) / 1e12
    peak = VALU_FP32_PEAK_TFLOPS if dtype == torch.float32 else MFMA_PEAK_TFLOPS
    return {"ms": ms, "tflops": tflops, "flops": flops, "frac": tflops / peak, "peak": peak, **extra}


PREFILL_SEQ = 8192


def bench_prefill_leg(args, device, name, dtype, seq=PREFILL_SEQ):
    """One dtype of the prefill leg, timed as the decode headline is, from an
    idle GPU: exactly --warmup untimed launches, then --steps timed ones (the
    main figures and the roofline), then the same steps after SUSTAIN_MS of
    load (`sustained`)."""
    steps = args.steps
    warmup = args.warmup
    r = run_prefill([seq], dtype, device, steps, warmup, sustain_ms=SUSTAIN_MS)
    workload = f"prefill_causal_seq{seq}_h32_kv8_d128"
    entry_wl = workload if name == "f16" else f"{workload}_bf16"
    return {
        "workload": entry_wl,
        "steps": steps,
        "warmup": warmup,
        "ms": round(r["ms"], 4),
        "tflops": round(r["tflops"], 1),
        "workspace_bytes": r["workspace_bytes"],
        "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 1), "peak": MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(r["frac"], 4), "flops_per_launch": r["flops"],
                     "traffic": _traffic_from_profiles(entry_wl),
                     "mfma_busy": _profile_entry(entry_wl)[0].get("mfma_busy"),
                     "counters_source": _profile_entry(entry_wl)[1]},
        "sustained": {"ms": round(r["sustained_ms"], 4), "tflops": round(r["sustained_tflops"], 1),
                      "frac": round(r["sustained_tflops"] / MFMA_PEAK_TFLOPS, 4), "after_ms_of_load": SUSTAIN_MS},
    }


def cpu_baseline_decode(budget_s=12.0):
    """fp32 oracle (oracle/reference.py) on a bounded sample of the decode
    workload: 4 of the 32 sequences (ctx 4096, 32/8 heads, D128, fp16 pages
    upcast), timed with perf_counter, min over repetitions within ~budget_s.
    Records the threads used, the affinity core count, os.cpu_count(), the
    cgroup CPU quota and the CPU model."""
    from flashattntile_amd.autotune import bytes_decode_paged
    from oracle.reference import ref_attention_paged

    host = _host()
    cores = _cores(host)
    torch.set_num_threads(cores)
    B, CTX, HQ, HKV, D, P = 4, 4096, 32, 8, 128, 16
    q, pools, _, _, table, lens = _paged_inputs([CTX] * B, HQ, HKV, D, P, torch.float16, seed=1, device="cpu")
    k, v, _, _ = pools[0]
    best, reps = _time_cpu(lambda: ref_attention_paged(q, k, v, table, lens), budget_s)
    nbytes = bytes_decode_paged([CTX] * B, HQ, HKV, D)
    return {
        "value": nbytes / best / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"fp32 oracle ref_attention_paged on 4 of the 32 sequences (ctx 4096, 32/8 heads, D128, "
                  f"page 16, fp16 pages upcast); min of {reps} runs after 1 warm-up; {cores} torch threads",
        "host": host,
        "ms": best * 1e3,
    }


def cpu_baseline_prefill(budget_s=8.0, seq=PREFILL_SEQ):
    """fp32 oracle (oracle/reference.py ref_attention_varlen) on a bounded
    sample of the prefill workload: one KV head and its 4 query heads of the
    causal seq-8192 sequence (fp16 inputs upcast), min over repetitions
    within ~budget_s.  TFLOP/s counts the same algorithmic causal FLOPs as
    the GPU figure (flashattn_tile/autotune.py:31-73) for that sample."""
    from flashattntile_amd.autotune import flops_attention_varlen
    from oracle.reference import ref_attention_varlen

    host = _host()
    cores = _cores(host)
    torch.set_num_threads(cores)
    q, k, v, cu = _prefill_case([seq], 4, 1, 128, torch.float16, 7, "cpu")
    best, reps = _time_cpu(lambda: ref_attention_varlen(q, k, v, cu, cu, causal=True), budget_s, max_reps=9)
    flops = flops_attention_varlen(4, 128, [seq], [seq], causal=True)
    return {
        "value": flops / best / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": f"fp32 oracle ref_attention_varlen on one KV head and its 4 query heads of the causal seq-{seq} "
                  f"sequence (D128, fp16 inputs upcast): 1/8 of the GPU leg's work; min of {reps} runs after 1 "
                  f"warm-up; {cores} torch threads",
        "cpu_model": host.get("cpu_model"),
        "ms": best * 1e3,
    }


def op_latency_decode(device, reps=100, warmup=25):
    """Latency of the op-level decode calls at the headline shape, as the
    reference's benchmark times its wrapper (scripts/benchmark_gpu.py:57-59,
    178: triton's do_bench, median of 100 calls after 25 warm-ups, cache
    flushed before each): HIP events around each call, after a 512 MB read
    that evicts L2 and the Infinity Cache.  Each call includes the wrapper's
    validation (one device->host sync), the tuned-store lookup and the
    launch, so this is what a caller of the op waits for per call."""
    from flashattntile_amd import PagedKVCache
    from flashattntile_amd.autotune import bytes_decode_paged
    from flashattntile_amd.kernels.decode import paged_decode_attention, resolve_decode_config

    B, CTX, HQ, HKV, D, P = 32, 4096, 32, 8, 128, 16
    q, pools, table, lens, _, _ = _paged_inputs([CTX] * B, HQ, HKV, D, P, torch.float16, seed=1, device=device)
    k, v = pools[0][0], pools[0][1]
    cache = PagedKVCache(k, v, table, lens, P)
    split = resolve_decode_config(q, cache, CTX, B * (CTX // P))["split_k"]
    flush = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=device)
    sink = torch.empty((), dtype=flush.dtype, device=device)
    stream = torch.cuda.current_stream(device)
    scale = D ** -0.5
    calls = {
        "paged_decode_attention": lambda: paged_decode_attention(q, cache),
        "torch.ops.flashattn_tile.paged_decode": lambda: torch.ops.flashattn_tile.paged_decode(
            q, k, v, table, lens, P, scale, split),
    }
    res = {}
    for name, fn in calls.items():
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        evs = []
        for _ in range(reps):
            torch.amax(flush, dim=0, out=sink)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            evs.append((e0, e1))
        torch.cuda.synchronize()
        ms = statistics.median(a.elapsed_time(b) for a, b in evs)
        res[name] = {"ms": round(ms, 5), "gbs": round(bytes_decode_paged([CTX] * B, HQ, HKV, D) / (ms * 1e-3) / 1e9,
                                                        1)}
    res["method"] = (f"HIP events around each call, median of {reps} after {warmup} warm-ups, each after a "
                     f"{FLUSH_BYTES >> 20} MB read; split_k {split} (the launch the wrapper resolves); validation "
                     "sync included")
    del pools, flush
    return res


# ---------------------------------------------------------------------------
# Every BASELINE.json configuration
# ---------------------------------------------------------------------------
def _decode_row(name, lens, hq, hkv, d, page, device, args, flush, split=None, quant=None, cpu_seqs=2,
                dtype=torch.float16):
    if args.only and args.only not in name:
        return None
    from flashattntile_amd import _hip
    from flashattntile_amd.kernels.decode import merge_counters
    from flashattntile_amd.autotune import bytes_decode_paged
    from oracle.reference import ref_attention_paged

    kv_elem = 1 if quant else torch.tensor([], dtype=dtype).element_size()
    pool_bytes = sum(lens) * hkv * d * 2 * kv_elem
    copies = 1 if pool_bytes >= 2 * MALL_BYTES else 2
    q, pools, table, seq, table_cpu, seq_cpu = _paged_inputs(lens, hq, hkv, d, page, dtype, seed=11,
                                                             device=device, copies=copies, quant=quant)
    maxp = table.shape[1]
    total_pages = sum(math.ceil(n / page) for n in lens)
    waves, kern, source = 0, 0, "command line"
    if split:
        sk, pps = split, 0
    else:
        sk, pps, waves, kern, source = _product_launch(q, pools, table, seq, page, max(lens), total_pages)
    out = torch.empty_like(q)
    ws = torch.empty(max(1, _hip.decode_workspace_bytes(len(lens), hq, d, sk)), dtype=torch.uint8, device=device)
    cnt = merge_counters(q, sk)  # the product's split-K merge inside the decode launch
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)

    def step(i):
        k, v, ks, vs = pools[i % copies]
        _hip.paged_decode(q, k, v, table, seq, out, page, d ** -0.5, sk, workspace=ws, stream=handle,
                          k_scale=ks, v_scale=vs, pages_per_split=pps, waves_per_group=waves, kernel=kern,
                          counters=cnt)

    steps = max(20, args.steps // 4)
    if pool_bytes * copies < 2 * MALL_BYTES:
        ms = _time_steps_flushed(step, steps, 5, stream, flush)
        timing = "median of per-launch events, each after a 512 MB cache flush"
    else:
        ms = _time_steps(step, steps, 5, stream)
        timing = f"back-to-back, {copies} pool copies alternating"
    nbytes = bytes_decode_paged(lens, hq, hkv, d, kv_elem_bytes=kv_elem, page_size=page, quantized=bool(quant))
    gbs = nbytes / (ms * 1e-3) / 1e9
    # CPU oracle on the first `cpu_seqs` sequences (dequantised to fp16 first for 8-bit caches)
    nb = min(cpu_seqs, len(lens))
    k0, v0, ks0, vs0 = pools[0]
    used = table_cpu[:nb].flatten().unique().long()
    kc, vc = k0[used.to(device)].cpu(), v0[used.to(device)].cpu()
    remap = torch.full((k0.shape[0],), -1, dtype=torch.int64)
    remap[used] = torch.arange(used.numel())
    tab = remap[table_cpu[:nb].long()].clamp_min(0).to(torch.int32)
    if quant:
        from oracle.quant_ref import dequantize_pages
        kc = dequantize_pages(kc, ks0[used.to(device)].cpu(), torch.float16)
        vc = dequantize_pages(vc, vs0[used.to(device)].cpu(), torch.float16)
    qc = q[:nb].cpu()
    best, reps = _time_cpu(lambda: ref_attention_paged(qc, kc, vc, tab, seq_cpu[:nb]), args.cpu_budget / 4)
    cpu_bytes = bytes_decode_paged(lens[:nb], hq, hkv, d, kv_elem_bytes=kv_elem, page_size=page,
                                   quantized=bool(quant))
    del pools
    torch.cuda.empty_cache()
    return {"config": name, "kind": "decode", "value": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "us": round(ms * 1e3, 2), "bytes": nbytes, "split_k": sk,
            "pages_per_split": pps, "launch": {"waves": waves, "kernel": kern, "source": source},
            "timing": timing,
            "cpu": {"value": round(cpu_bytes / best / 1e9, 3), "unit": "GB/s",
                    "sample": f"{nb} of {len(lens)} sequences, min of {reps}"}}


def _configs0_row(device, args, flush):
    """BASELINE configs[0], the reference's CPU workload: B4, 32/8 heads, D128,
    page 16, ctx ~ U{64..512} (seeded), a 256-page pool and a seeded
    randperm(256) table sliced to [4, 32], fp16 pages.  The GPU decode (the
    product's launch for the shape) and the fp32 oracle over the whole batch
    (min of 21 runs after 3 warm-ups, the reference's CPU convention)."""
    name = "decode fp16 configs[0] B4 ctx U[64,512] pool256"
    if args.only and args.only not in name:
        return None
    from flashattntile_amd import _hip
    from flashattntile_amd.kernels.decode import merge_counters
    from flashattntile_amd.autotune import bytes_decode_paged
    from oracle.reference import ref_attention_paged

    g = torch.Generator().manual_seed(0)
    lens = torch.randint(64, 513, (4,), generator=g).to(torch.int32)
    table = torch.randperm(256, generator=g)[:128].to(torch.int32).view(4, 32)
    k = torch.randn(256, 16, 8, 128, generator=g).half()
    v = torch.randn(256, 16, 8, 128, generator=g).half()
    q = torch.randn(4, 32, 128, generator=g).half()
    kd, vd, qd = k.to(device), v.to(device), q.to(device)
    td, ld = table.to(device), lens.to(device)
    pools = [(kd, vd, None, None)]
    sk, pps, waves, kern, source = _product_launch(qd, pools, td, ld, 16, int(lens.max()), 256)
    out = torch.empty_like(qd)
    ws = torch.empty(max(1, _hip.decode_workspace_bytes(4, 32, 128, sk)), dtype=torch.uint8, device=device)
    cnt = merge_counters(qd, sk)
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)

    def step(i):
        _hip.paged_decode(qd, kd, vd, td, ld, out, 16, 128 ** -0.5, sk, workspace=ws, stream=handle,
                          pages_per_split=pps, waves_per_group=waves, kernel=kern, counters=cnt)

    ms = _time_steps_flushed(step, max(20, args.steps // 4), 5, stream, flush)
    nbytes = bytes_decode_paged(lens.tolist(), 32, 8, 128)
    for _ in range(2):
        ref_attention_paged(q, k, v, table, lens)
    best, reps = _time_cpu(lambda: ref_attention_paged(q, k, v, table, lens), args.cpu_budget, max_reps=21)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"config": name, "kind": "decode", "value": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "us": round(ms * 1e3, 2), "bytes": nbytes, "split_k": sk,
            "pages_per_split": pps, "launch": {"waves": waves, "kernel": kern, "source": source},
            "lens": lens.tolist(),
            "timing": "median of per-launch events, each after a 512 MB cache flush",
            "cpu": {"value": round(nbytes / best / 1e9, 3), "unit": "GB/s", "us": round(best * 1e6, 1),
                    "sample": f"the whole configs[0] batch, min of {reps} after 3 warm-ups, {_cores()} threads"}}


def _prefill_row(name, lens, dtype, device, args, hq=32, hkv=8, d=128):
    if args.only and args.only not in name:
        return None
    from flashattntile_amd.autotune import flops_attention_varlen
    from oracle.reference import ref_attention_varlen

    r = run_prefill(lens, dtype, device, max(10, args.steps // 10), 3, hq=hq, hkv=hkv, d=d)
    # CPU oracle: the query heads of one KV head over the first sequence
    group = hq // hkv
    L = lens[0]
    g = torch.Generator().manual_seed(3)
    qc = torch.randn(L, group, d, generator=g).to(dtype)
    kc = torch.randn(L, 1, d, generator=g).to(dtype)
    vc = torch.randn(L, 1, d, generator=g).to(dtype)
    cu = torch.tensor([0, L], dtype=torch.int32)
    best, reps = _time_cpu(lambda: ref_attention_varlen(qc, kc, vc, cu, cu, causal=True), args.cpu_budget / 4,
                           max_reps=5)
    cpu_flops = flops_attention_varlen(group, d, [L], [L], causal=True)
    torch.cuda.empty_cache()
    return {"config": name, "kind": "prefill", "value": round(r["tflops"], 1), "unit": "TFLOP/s",
            "frac": round(r["frac"], 4), "peak": r["peak"], "us": round(r["ms"] * 1e3, 2), "flops": r["flops"],
            "cpu": {"value": round(cpu_flops / best / 1e12, 5), "unit": "TFLOP/s",
                    "sample": f"{group} query heads / 1 KV head of sequence 0 (L={L}), min of {reps}"}}


def _paged_prefill_row(name, lens_k, lens_q, dtype, device, args, page=16, hq=32, hkv=8, d=128):
    """fat_prefill_paged: each sequence's q_len-token chunk attends to its
    kv_len keys read through the page table (permuted pool)."""
    if args.only and args.only not in name:
        return None
    from flashattntile_amd import _hip
    from flashattntile_amd.autotune import flops_attention_varlen
    from oracle.reference import ref_attention_paged_prefill

    gen = torch.Generator(device=device).manual_seed(12)
    pages_per = [math.ceil(n / page) for n in lens_k]
    num_pages = sum(pages_per)
    k = torch.randn(num_pages, page, hkv, d, device=device, generator=gen).to(dtype)
    v = torch.randn(num_pages, page, hkv, d, device=device, generator=gen).to(dtype)
    perm = torch.randperm(num_pages, device=device, generator=gen).to(torch.int32)
    table = torch.zeros(len(lens_k), max(pages_per), dtype=torch.int32, device=device)
    at = 0
    for b, n in enumerate(pages_per):
        table[b, :n] = perm[at:at + n]
        at += n
    seq = torch.tensor(lens_k, dtype=torch.int32, device=device)
    q = torch.randn(sum(lens_q), hq, d, device=device, generator=gen).to(dtype)
    cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens_q), 0).tolist(), dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)
    mq = max(lens_q)
    # The product's launch (kernels/prefill.py paged_prefill_launch): the
    # workspace the library asks for (packed K/V copies for long chunks),
    # allocated once outside the timed steps.
    a = _hip.prefill_paged_args(q, k, v, table, seq, cu, out, page, mq, True, d ** -0.5)
    need = _hip.prefill_paged_workspace_bytes(a)
    ws = torch.empty(need, dtype=torch.uint8, device=device) if need else None
    if ws is not None:
        a.workspace = ws.data_ptr()
    launch, ref, hs = _hip.lib().fat_prefill_paged, ctypes.byref(a), ctypes.c_void_p(handle)

    def step(i):
        if launch(ref, hs) != 0:
            raise RuntimeError(_hip.lib().fat_last_error().decode(errors="replace"))

    ms = _time_steps(step, max(10, args.steps // 10), 3, stream)
    flops = flops_attention_varlen(hq, d, lens_q, lens_k, causal=True)
    tflops = flops / (ms * 1e-3) / 1e12
    # CPU oracle: one KV head's query heads of the first sequence
    group = hq // hkv
    q0 = q[: lens_q[0], :group].cpu()
    k0 = k[:, :, :1].cpu()
    v0 = v[:, :, :1].cpu()
    best, reps = _time_cpu(lambda: ref_attention_paged_prefill(q0, k0, v0, table[:1].cpu(), seq[:1].cpu(),
                                                               [0, lens_q[0]], causal=True), args.cpu_budget / 4,
                           max_reps=5)
    cpu_flops = flops_attention_varlen(group, d, lens_q[:1], lens_k[:1], causal=True)
    del k, v
    torch.cuda.empty_cache()
    return {"config": name, "kind": "prefill_paged", "value": round(tflops, 1), "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_PEAK_TFLOPS, 4), "us": round(ms * 1e3, 2), "flops": flops,
            "workspace_bytes": need,
            "cpu": {"value": round(cpu_flops / best / 1e12, 5), "unit": "TFLOP/s",
                    "sample": f"{group} query heads / 1 KV head of sequence 0, min of {reps}"}}


def _multi_decode_row(name, lens, T, device, args, hq=32, hkv=8, d=128, page=16):
    """Multi-token decode (q_len = T) through fat_paged_decode: bytes = K/V
    read once + T queries and outputs per sequence."""
    if args.only and args.only not in name:
        return None
    from flashattntile_amd import _hip
    from flashattntile_amd.kernels.decode import merge_counters
    from flashattntile_amd.autotune import bytes_decode_paged
    from oracle.reference import ref_attention_paged_prefill

    q1, pools, table, seq, table_cpu, seq_cpu = _paged_inputs(lens, hq, hkv, d, page, torch.float16, seed=13,
                                                               device=device, copies=2)
    gen = torch.Generator(device=device).manual_seed(14)
    q = torch.randn(len(lens), T, hq, d, device=device, generator=gen).half()
    out = torch.empty_like(q)
    total_pages = sum(math.ceil(n / page) for n in lens)
    sk, pps, waves, kern, source = _product_launch(q, pools, table, seq, page, max(lens), total_pages, q_len=T)
    ws = torch.empty(max(1, _hip.decode_workspace_bytes(len(lens) * T, hq, d, sk)), dtype=torch.uint8,
                     device=device)
    cnt = merge_counters(q, sk)
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)

    def step(i):
        k, v, _, _ = pools[i % 2]
        _hip.paged_decode(q, k, v, table, seq, out, page, d ** -0.5, sk, workspace=ws, stream=handle,
                          pages_per_split=pps, waves_per_group=waves, kernel=kern, counters=cnt)

    ms = _time_steps(step, max(20, args.steps // 4), 5, stream)
    nbytes = bytes_decode_paged(lens, hq, hkv, d) + 2 * len(lens) * (T - 1) * hq * d * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    k0, v0, _, _ = pools[0]
    used = table_cpu[:1].flatten().unique().long()
    kc, vc = k0[used.to(device)].cpu(), v0[used.to(device)].cpu()
    remap = torch.full((k0.shape[0],), -1, dtype=torch.int64)
    remap[used] = torch.arange(used.numel())
    tab = remap[table_cpu[:1].long()].clamp_min(0).to(torch.int32)
    qc = q[:1].reshape(T, hq, d).cpu()
    best, reps = _time_cpu(lambda: ref_attention_paged_prefill(qc, kc, vc, tab, seq_cpu[:1], [0, T]),
                           args.cpu_budget / 4)
    cpu_bytes = bytes_decode_paged(lens[:1], hq, hkv, d) + 2 * (T - 1) * hq * d * 2
    del pools
    torch.cuda.empty_cache()
    return {"config": name, "kind": "decode_multi", "value": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "us": round(ms * 1e3, 2), "bytes": nbytes, "split_k": sk,
            "pages_per_split": pps, "q_len": T, "launch": {"waves": waves, "kernel": kern, "source": source},
            "cpu": {"value": round(cpu_bytes / best / 1e9, 3), "unit": "GB/s",
                    "sample": f"1 of {len(lens)} sequences, min of {reps}"}}


def _graph_decode_row(name, B, ctx, device, args, hq=32, hkv=8, d=128, page=16, layers=32):
    """Per-launch cost of a small decode in a step of `layers` launches (one
    per model layer; all on the same cache here): launched eagerly from Python
    (paged_decode_launch: ctypes argument block + launch) and replayed from
    one HIP graph that captured the whole step."""
    if args.only and args.only not in name:
        return None
    from flashattntile_amd import PagedKVCache, _hip
    from flashattntile_amd.kernels.decode import merge_counters, paged_decode_launch

    q, pools, table, seq, _, _ = _paged_inputs([ctx] * B, hq, hkv, d, page, torch.float16, seed=17, device=device,
                                               copies=1)
    k, v, _, _ = pools[0]
    cache = PagedKVCache(k, v, table, seq, page)
    sk, pps, waves, kern, _ = _product_launch(q, pools, table, seq, page, ctx, B * table.shape[1])
    kname = {0: None, 1: "valu", 2: "mfma"}[kern]
    out = torch.empty_like(q)
    ws = torch.empty(max(1, _hip.decode_workspace_bytes(B, hq, d, sk)), dtype=torch.uint8, device=device)
    cnt = merge_counters(q, sk)

    def launch():
        paged_decode_launch(q, cache, d ** -0.5, sk, out=out, workspace=ws, waves_per_group=waves,
                            pages_per_split=pps, kernel=kname, counters=cnt)

    def step():
        for _ in range(layers):
            launch()

    from flashattntile_amd.kernels.decode import DecodeLaunch

    plan = DecodeLaunch(q, cache, d ** -0.5, config={"split_k": sk, "pages_per_split": pps,
                                                     "num_warps": waves or None, "kernel": kname},
                        max_len=ctx, total_pages=B * table.shape[1])
    handle = int(torch.cuda.current_stream(device).cuda_stream)

    def plan_step():
        for _ in range(layers):
            plan.run(q, out, stream=handle)

    stream = torch.cuda.current_stream(device)
    steps = max(10, args.steps // 20)
    eager = _time_steps(lambda i: step(), steps, 3, stream) / layers
    planned = _time_steps(lambda i: plan_step(), steps, 3, stream) / layers
    side = torch.cuda.Stream(device)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        step()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    replay = _time_steps(lambda i: graph.replay(), steps, 3, stream) / layers
    nbytes = 4096 * B * ctx + 16384 * B
    del pools, cache
    torch.cuda.empty_cache()
    return {"config": name, "kind": "decode_graph", "value": round(replay * 1e3, 2), "unit": "us/call",
            "frac": round(nbytes / (replay * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "us": round(replay * 1e3, 2),
            "eager_us": round(eager * 1e3, 2), "plan_us": round(planned * 1e3, 2), "bytes": nbytes, "split_k": sk,
            "cpu": None}


def _quantize_row(name, src_dtype, mode, device, args, pages=8192, page=16, hkv=8, d=128):
    """fat_quantize_pages over a whole K pool (the headline cache's 8192 pages);
    two pools alternate.  Bytes = read src + write codes + write scales."""
    if args.only and args.only not in name:
        return None
    from flashattntile_amd import _hip
    from oracle.quant_ref import quantize_pages

    gen = torch.Generator(device=device).manual_seed(5)
    srcs = [torch.randn(pages, page, hkv, d, device=device, generator=gen).to(src_dtype) for _ in range(2)]
    qdt = torch.int8 if mode == "int8" else torch.float8_e4m3fn
    codes = torch.empty(pages, page, hkv, d, dtype=qdt, device=device)
    scale = torch.empty(pages, hkv, dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream(device)
    handle = int(stream.cuda_stream)

    def step(i):
        _hip.quantize_pages(srcs[i % 2], codes, scale, stream=handle)

    ms = _time_steps(step, max(20, args.steps // 4), 5, stream)
    elem = srcs[0].element_size()
    nbytes = pages * page * hkv * d * (elem + 1) + pages * hkv * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    sample = srcs[0][:256].cpu()
    best, reps = _time_cpu(lambda: quantize_pages(sample, mode), args.cpu_budget / 4)
    cpu_bytes = 256 * page * hkv * d * (elem + 1) + 256 * hkv * 4
    del srcs
    torch.cuda.empty_cache()
    return {"config": name, "kind": "kv_write", "value": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "us": round(ms * 1e3, 2), "bytes": nbytes,
            "cpu": {"value": round(cpu_bytes / best / 1e9, 3), "unit": "GB/s",
                    "sample": f"256 of {pages} pages, min of {reps}"}}


def _append_row(name, mode, device, args, B=32, ctx=4000, page=16, hkv=8, d=128):
    """append_tokens (HIP, validate=False: no host sync) of one token per
    sequence into the headline-shaped cache, optionally keeping an fp8/int8
    copy requantised; latency per call.  Bytes = rows written + touched
    (page, head) units re-read and re-quantised."""
    if args.only and args.only not in name:
        return None
    from flashattntile_amd.paging import PagedKVCache, append_tokens
    from flashattntile_amd.quant import quantize_cache

    maxp = (ctx + 64) // page + 1
    gen = torch.Generator(device=device).manual_seed(6)
    k = torch.randn(B * maxp, page, hkv, d, device=device, generator=gen).half()
    v = torch.randn_like(k)
    perm = torch.randperm(B * maxp, device=device, generator=gen).to(torch.int32)
    lens = torch.full((B,), ctx, dtype=torch.int32, device=device)
    cache = PagedKVCache(k, v, perm.view(B, maxp), lens, page)
    mirror = quantize_cache(cache, mode=mode) if mode else None
    nk = torch.randn(B, hkv, d, device=device, generator=gen).half()
    nv = torch.randn_like(nk)
    stream = torch.cuda.current_stream(device)

    def step(i):
        if i % 64 == 0:
            lens.fill_(ctx)  # stay inside the table (64 appends per refill)
        append_tokens(cache, nk, nv, quantized=mirror, validate=False)

    steps = max(64, args.steps // 2)
    ms = _time_steps(step, steps, 8, stream)
    from flashattntile_amd.paging import AppendLaunch

    plan = AppendLaunch(cache, quantized=mirror)
    handle = int(stream.cuda_stream)

    def plan_step(i):
        if i % 64 == 0:
            lens.fill_(ctx)
        plan.run(nk, nv, stream=handle)

    plan_ms = _time_steps(plan_step, steps, 8, stream)
    nbytes = 2 * B * hkv * d * 2
    if mode:
        nbytes += 2 * B * hkv * (page * d * (2 + 1) + 4)
    # CPU: the torch path of append_tokens on a CPU copy of 4 sequences (no copy maintained)
    kc = k[: 4 * maxp].cpu()
    vc = v[: 4 * maxp].cpu()
    tab = torch.arange(4 * maxp, dtype=torch.int32).view(4, maxp)
    lc = torch.full((4,), ctx, dtype=torch.int32)
    ccache = PagedKVCache(kc, vc, tab, lc, page)
    nkc, nvc = nk[:4].cpu(), nv[:4].cpu()

    def cpu_step():
        lc.fill_(ctx)
        append_tokens(ccache, nkc, nvc)

    best, reps = _time_cpu(cpu_step, args.cpu_budget / 8)
    del cache, mirror, k, v
    torch.cuda.empty_cache()
    us = ms * 1e3
    return {"config": name, "kind": "kv_write", "value": round(us, 2), "unit": "us/call",
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "us": round(us, 2), "bytes": nbytes,
            "plan_us": round(plan_ms * 1e3, 2),
            "cpu": {"value": round(best * 1e6, 1), "unit": "us/call (torch path, 4 sequences)",
                    "sample": f"4 of {B} sequences, min of {reps}"}}


def all_configs(args, device):
    flush = torch.ones(FLUSH_BYTES // 8, dtype=torch.float64, device=device)
    rows = []

    def emit(row):
        if row is None:
            return
        rows.append(row)
        tail = (f"cpu {row['cpu']['value']} {row['cpu']['unit']}"
                + (f"; AppendLaunch.run {row['plan_us']} us/call" if "plan_us" in row else "") if row.get("cpu")
                else f"eager Python launch {row.get('eager_us')} us/call, DecodeLaunch.run {row.get('plan_us')} us/call")
        print(f"# {row['config']:46s} {row['value']:9.1f} {row['unit']:8s} ({100 * row['frac']:5.1f}% of peak, "
              f"{row['us']:9.1f} us)  {tail}", file=sys.stderr, flush=True)

    # the reference's CPU workload, GPU decode next to the fp32 oracle
    emit(_configs0_row(device, args, flush))
    # fp16 decode sweep (and bf16 at the headline shape)
    for B in (1, 8, 32, 128):
        for ctx in (128, 1024, 4096, 16384):
            emit(_decode_row(f"decode fp16 B{B} ctx{ctx}", [ctx] * B, 32, 8, 128, 16, device, args, flush))
    emit(_decode_row("decode bf16 B32 ctx4096", [4096] * 32, 32, 8, 128, 16, device, args, flush,
                     dtype=torch.bfloat16))
    # prefill fp16 / bf16, L in 512..8192 and the mixed pack
    g = torch.Generator().manual_seed(2024)
    mixed = torch.randint(1, 4097, (8,), generator=g).tolist()
    mixed[0] |= 1
    for dt, dn in ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        for L in (512, 1024, 2048, 4096, 8192):
            emit(_prefill_row(f"prefill {dn} causal L{L}", [L], dt, device, args))
        emit(_prefill_row(f"prefill {dn} causal mixed8 {sum(mixed)} tok", mixed, dt, device, args))
    # fp32 prefill: the generic VALU kernel (its bound is the 157.3 TFLOP/s fp32 vector peak)
    for L in (1024, 4096):
        emit(_prefill_row(f"prefill fp32 causal L{L} (generic)", [L], torch.float32, device, args))
    # quantised decode B128 ctx16384
    for mode, mn in (("int8", "int8"), ("float8_e4m3fn", "fp8")):
        emit(_decode_row(f"decode {mn} B128 ctx16384", [16384] * 128, 32, 8, 128, 16, device, args, flush,
                         quant=mode, cpu_seqs=1))
    # stress
    emit(_decode_row("decode fp16 B1 ctx131072 split16", [131072], 32, 8, 128, 16, device, args, flush, split=16,
                     cpu_seqs=1))
    emit(_decode_row("decode fp16 B1 ctx131072", [131072], 32, 8, 128, 16, device, args, flush, cpu_seqs=1))
    from flashattntile_amd.tune import skewed_lens  # the tuner's draw, so its store entry matches
    skew = skewed_lens()
    emit(_decode_row(f"decode fp16 skewed64 sum{sum(skew)}", skew, 32, 8, 128, 16, device, args, flush))
    emit(_decode_row("decode fp16 MQA 32/1 B32 ctx4096", [4096] * 32, 32, 1, 128, 16, device, args, flush))
    emit(_decode_row("decode fp16 D64 B32 ctx4096", [4096] * 32, 32, 8, 64, 16, device, args, flush))
    for page in (32, 64):
        emit(_decode_row(f"decode fp16 P{page} B32 ctx4096", [4096] * 32, 32, 8, 128, page, device, args, flush))
    # the generic decode kernel (LDS-tiled, any page size): fp32, and pages of 1 and 5 rows
    for dt, dn in ((torch.float32, "fp32"), (torch.float16, "fp16")):
        for page in (1, 5):
            emit(_decode_row(f"decode {dn} generic P{page} B32 ctx4096", [4096] * 32, 32, 8, 128, page, device,
                             args, flush, dtype=dt))
    emit(_decode_row("decode fp32 generic P16 B32 ctx4096", [4096] * 32, 32, 8, 128, 16, device, args, flush,
                     dtype=torch.float32))
    # Multi-token (speculative) decode: T query tokens per sequence
    for T in (2, 4, 8):
        emit(_multi_decode_row(f"decode fp16 multi-token T{T} B32 ctx4096", [4096] * 32, T, device, args))
    # small decodes: Python-launched vs replayed from a HIP graph
    for B, ctx in ((1, 1024), (8, 1024), (32, 128)):
        emit(_graph_decode_row(f"decode fp16 B{B} ctx{ctx} graph replay (32/step)", B, ctx, device, args))
    # Paged (chunked) prefill: K/V through the page table (page 16)
    for dt, dn in ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        emit(_paged_prefill_row(f"prefill paged {dn} causal L8192 P16", [8192], [8192], dt, device, args))
        emit(_paged_prefill_row(f"prefill paged {dn} chunk 512 after 3584 B16", [4096] * 16, [512] * 16, dt,
                                device, args))
    # KV write path (flashattn_tile/quant.py:84-142, paging.py:172-210): quantise the headline
    # pool; one-token append
    for dt, dn in ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        for mode, mn in (("int8", "int8"), ("float8_e4m3fn", "fp8")):
            emit(_quantize_row(f"kvwrite quantize {dn}->{mn} 8192 pages", dt, mode, device, args))
    emit(_append_row("kvwrite append B32", None, device, args))
    emit(_append_row("kvwrite append B32 + fp8 copy", "float8_e4m3fn", device, args))
    return rows


# Kernel sources behind each profiled workload.  A profiles/traffic.json
# entry records the digest of these files at the commit its rocprofv3 PMC
# passes ran on; the bench line carries its figures only while the files
# still hash to that digest (otherwise the kernel changed since).
PROFILE_SOURCES = {
    "decode": ["flashattntile_amd/csrc/decode.hip", "flashattntile_amd/csrc/decode_params.h",
               "flashattntile_amd/csrc/fat_common.h"],
    "prefill": ["flashattntile_amd/csrc/prefill.hip", "flashattntile_amd/csrc/prefill_wide.hip",
                "flashattntile_amd/csrc/prefill_common.h", "flashattntile_amd/csrc/fat_common.h"],
    "kvwrite": ["flashattntile_amd/csrc/kvwrite.hip", "flashattntile_amd/csrc/fat_common.h"],
}


def source_digest(family: str) -> str:
    """sha256 (first 16 hex digits) over the path and bytes of each source
    file of a kernel family, in PROFILE_SOURCES order."""
    import hashlib

    root = os.path.dirname(os.path.abspath(__file__))
    h = hashlib.sha256()
    for rel in PROFILE_SOURCES[family]:
        h.update(rel.encode())
        with open(os.path.join(root, rel), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def _profile_entry(workload: str) -> tuple[dict, str]:
    """The rocprofv3 PMC measurements of a workload (profiles/traffic.json)
    and where they come from; ({}, reason) when absent or measured on other
    kernel sources than this tree's."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as fh:
            entry = json.load(fh).get(workload, {})
    except (OSError, ValueError):
        return {}, "profiles/traffic.json unreadable"
    if not entry:
        return {}, f"no PMC entry for {workload}"
    family = entry.get("family")
    if family not in PROFILE_SOURCES or entry.get("source_digest") != source_digest(family):
        return {}, (f"stale: {workload}'s PMC passes ran on kernel sources with digest "
                    f"{entry.get('source_digest')}, this tree's are {source_digest(family) if family in PROFILE_SOURCES else '?'}")
    return entry, entry.get("source", "profiles/traffic.json")


def _traffic_from_profiles(workload: str):
    """HBM bytes per launch measured by rocprofv3 PMC runs on this tree's
    kernel sources (None when stale or absent)."""
    return _profile_entry(workload)[0].get("bytes_per_launch")


def _mfma_busy_from_profiles(workload: str, dtype: str):
    """Fraction of the kernel's cycles the MFMA pipe was busy (PMC run on
    this tree's kernel sources; None when stale or absent)."""
    return _profile_entry(workload)[0].get("mfma_busy", {}).get(dtype)


def main():
    args = _parse()
    if args.source_digests:
        print(json.dumps({f: source_digest(f) for f in PROFILE_SOURCES}))
        return
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
    torch.set_num_threads(_cores())

    if args.all_configs:
        global ROW_WARM_MS
        ROW_WARM_MS = args.row_warm_ms
        rows = all_configs(args, device)
        report = {"cores": _cores(), "host": _host(), "rows": rows, "row_warm_ms": ROW_WARM_MS,
                  "device": torch.cuda.get_device_name(device)}
        if args.report:
            with open(args.report, "w") as fh:
                json.dump(report, fh, indent=1)
        return

    if args.copy_calibration:
        n = copy_calibration(device)
        print(f"# copy calibration: 3 x torch.neg over {n} bytes read + {n} bytes written", file=sys.stderr,
              flush=True)
    legs = set(args.legs.split(","))
    if args.no_prefill:
        legs.discard("prefill")
    if args.no_cpu_baseline:
        legs.discard("cpu")

    def idle_gap(cpu_leg):
        """Leave the GPU idle before the next timed leg, so that every leg's
        contract timing starts from an idle GPU as the decode leg's does: the
        CPU baseline when it runs, else IDLE_GAP_S of sleep."""
        if cpu_leg is not None and "cpu" in legs:
            return cpu_leg()
        time.sleep(IDLE_GAP_S)
        return None

    dec = None
    if "decode" in legs:
        dec = bench_decode(args, device)
        print(f"# decode: {dec['gbs']:.1f} GB/s ({dec['ms'] * 1e3:.1f} us/step, split_k={dec['split_k']}, "
              f"waves={dec['waves_per_group']}); after {SUSTAIN_MS:.0f} ms of load {dec['sustained_gbs']:.1f} GB/s "
              f"({dec['sustained_ms'] * 1e3:.1f} us/step)", file=sys.stderr, flush=True)
        dec["op_latency"] = op_latency_decode(device)
        print(f"# decode op latency: {json.dumps(dec['op_latency'])}", file=sys.stderr, flush=True)
    cpu = idle_gap(lambda: cpu_baseline_decode(args.cpu_budget)) if ("prefill" in legs or "cpu" in legs) else None
    if cpu is not None:
        print(f"# cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} cores", file=sys.stderr, flush=True)
    pre = None
    if "prefill" in legs:
        pre = {"f16": bench_prefill_leg(args, device, "f16", torch.float16)}
        cpu_pre = idle_gap(lambda: cpu_baseline_prefill(min(args.cpu_budget, 8.0)))
        pre["bf16"] = bench_prefill_leg(args, device, "bf16", torch.bfloat16)
        if cpu_pre is not None:
            pre["cpu_baseline"] = {k: v for k, v in cpu_pre.items() if k != "ms"}
        pre["timing"] = (f"each dtype from an idle GPU (after seconds of CPU baseline or {IDLE_GAP_S:.0f} s of "
                         f"sleep): ms / tflops / roofline over the contract's steps right after the warm-up steps; "
                         f"`sustained` the same steps after {SUSTAIN_MS:.0f} ms of load")
        print(f"# prefill seq{PREFILL_SEQ}: fp16 {pre['f16']['tflops']:.1f} TFLOP/s ({pre['f16']['ms']:.3f} ms), "
              f"bf16 {pre['bf16']['tflops']:.1f}; sustained fp16 {pre['f16']['sustained']['tflops']:.1f}, "
              f"bf16 {pre['bf16']['sustained']['tflops']:.1f}"
              + (f"; cpu {cpu_pre['value']:.3f} TFLOP/s" if cpu_pre else ""), file=sys.stderr, flush=True)
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
            "kernel": dec["kernel"],
            "launch_from": dec["config_source"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec["gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": _traffic_from_profiles(workload),
            "traffic_source": _profile_entry(workload)[1],
            "algorithmic_bytes": dec["bytes"],
        },
        "sustained": {"value": round(dec["sustained_gbs"], 2), "ms_per_step": round(dec["sustained_ms"], 5),
                      "frac": round(dec["sustained_gbs"] / HBM_PEAK_GBS, 4), "after_ms_of_load": SUSTAIN_MS,
                      "note": "the same steps timed again after sustained load; `value` is the contract's timing"},
        "cpu_baseline": None if cpu is None else {k: v for k, v in cpu.items() if k != "ms"},
        "op_latency": dec["op_latency"],
        "prefill": pre,
    }
    if dec["tuning_ms"]:
        line["decode_tuning_ms"] = dec["tuning_ms"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
