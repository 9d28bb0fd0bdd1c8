"""Analytic work accounting and the MI355X launch heuristics.

The FLOP and byte formulas are the reference's roofline numerators
(``flashattn_tile/autotune.py:31-106``) so achieved-throughput figures are
comparable:

* ``flops = 4 * B * H * D * pairs`` (QK^T and PV, 2 FLOP per MAC; softmax
  excluded), ``pairs = q*kv`` or, causal bottom-right,
  ``q*(kv - q) + q*(q + 1)/2``;
* decode bytes = q + K + V + o; prefill bytes = q + k + v + o.

The reference's Triton knob search (BLOCK_M/N, num_warps, num_stages) has no
meaning for the HIP kernels.  What matters on MI355X is how many workgroups a
decode launch puts on the 256 CUs and which kernel family runs, so:

* split-K is derived from the shape and the CU count
  (:func:`decode_partition`), with no device synchronisation;
* the tuned-config store of ``autotune.py:376-419`` (``best_config``,
  ``save_best``, ``initialize_store``) keeps the same JSON schema but is
  re-keyed for gfx950: decode signatures carry the cache dtype, the query
  length and whether the batch is ragged, and the stored knobs are the gfx950
  ones (``split_k``, ``pages_per_split``, ``num_warps`` = waves per workgroup,
  ``kernel``).  :func:`autotune` times candidates from
  :func:`build_config_space` with HIP events and stores the winner; the decode
  and prefill wrappers consult the store when ``config`` is None and fall
  back to the heuristic on a miss.
"""

from __future__ import annotations

import json
import math
import os
import time
import warnings
from datetime import datetime, timezone
from pathlib import Path

__all__ = [
    "flops_attention",
    "flops_attention_varlen",
    "bytes_attention",
    "bytes_decode_paged",
    "arithmetic_intensity",
    "decode_split_k",
    "decode_partition",
    "decode_heads_per_workgroup",
    "decode_signature",
    "prefill_signature",
    "prefill_paged_signature",
    "is_ragged",
    "best_config",
    "save_best",
    "initialize_store",
    "build_config_space",
    "time_callable",
    "time_back_to_back",
    "summarize_times",
    "autotune",
    "TUNED_CONFIGS_PATH",
    "MI355X_CUS",
]

MI355X_CUS = 256


def _causal_pairs(q_len: int, kv_len: int) -> int:
    """Query/key pairs visible under bottom-right causal alignment."""
    if q_len <= 0 or kv_len <= 0:
        return 0
    if kv_len < q_len:
        raise ValueError("causal accounting requires kv_len >= q_len")
    return q_len * (kv_len - q_len) + q_len * (q_len + 1) // 2


def flops_attention(num_heads: int, head_dim: int, q_len: int, kv_len: int,
                    causal: bool = False, batch: int = 1) -> int:
    """``4 * batch * H * D * pairs`` (``autotune.py:40-55``)."""
    pairs = _causal_pairs(q_len, kv_len) if causal else q_len * kv_len
    return int(4 * batch * num_heads * head_dim * pairs)


def flops_attention_varlen(num_heads: int, head_dim: int, q_lens, kv_lens, causal: bool = False) -> int:
    """Sum of :func:`flops_attention` over a ragged batch (``autotune.py:58-73``)."""
    if len(q_lens) != len(kv_lens):
        raise ValueError("q_lens and kv_lens must have the same length")
    return int(sum(flops_attention(num_heads, head_dim, int(q), int(k), causal=causal)
                   for q, k in zip(q_lens, kv_lens)))


def bytes_attention(mode: str, batch: int, q_len: int, kv_len: int, num_heads: int,
                    num_kv_heads: int, head_dim: int, elem_bytes: int = 2) -> int:
    """HBM bytes of the fused kernel: q + K + V + o (``autotune.py:76-106``)."""
    if mode == "decode":
        if q_len != 1:
            raise ValueError("decode accounting assumes q_len == 1")
        q_bytes = batch * num_heads * head_dim * elem_bytes
        kv_bytes = batch * kv_len * num_kv_heads * head_dim * 2 * elem_bytes
        return int(2 * q_bytes + kv_bytes)
    if mode == "prefill":
        q_bytes = batch * q_len * num_heads * head_dim * elem_bytes
        kv_bytes = batch * kv_len * num_kv_heads * head_dim * 2 * elem_bytes
        return int(2 * q_bytes + kv_bytes)
    raise ValueError(f"unknown mode {mode!r}")


def bytes_decode_paged(seq_lens, num_heads: int, num_kv_heads: int, head_dim: int,
                       q_elem_bytes: int = 2, kv_elem_bytes: int = 2, page_size: int | None = None,
                       quantized: bool = False) -> int:
    """Decode bytes for a ragged batch: q + o + sum_b ctx_b * (K + V).

    For a quantised cache the fp32 scales of every touched (page, KV head) are
    added (2 * 4 bytes each), the scale term of ``kv_bytes_per_token``
    (``quant.py:205-208``).  The page table is excluded, as in the reference.
    """
    lens = [int(x) for x in seq_lens]
    batch = len(lens)
    qo = 2 * batch * num_heads * head_dim * q_elem_bytes
    kv = sum(lens) * num_kv_heads * head_dim * 2 * kv_elem_bytes
    scales = 0
    if quantized:
        if page_size is None:
            raise ValueError("quantized accounting needs page_size")
        pages = sum(math.ceil(n / page_size) for n in lens)
        scales = pages * num_kv_heads * 2 * 4
    return int(qo + kv + scales)


def arithmetic_intensity(flops: float, nbytes: float) -> float:
    if nbytes <= 0:
        return float("inf")
    return float(flops) / float(nbytes)


def decode_split_k(batch: int, num_heads: int, num_kv_heads: int, max_pages: int,
                   num_cus: int = MI355X_CUS, min_pages_per_split: int = 8, max_split: int = 16) -> int:
    """Split-K partitions for a decode launch on MI355X.

    One workgroup handles one GQA group of up to 8 query heads for one
    partition, so a launch has ``batch * groups * split`` workgroups.  The
    rule asks for about one workgroup per CU, never fewer than
    ``min_pages_per_split`` pages per partition (shorter partitions spend more
    on the merge than they gain) and at most ``max_split`` partitions.  It was
    fitted on an MI355X sweep of B in {1, 8, 32, 128} x ctx in {128, 1024,
    4096, 16384} (32/8 heads, D128, page 16, fp16), where it picks the fastest
    measured split or one within 2 % of it.  It needs only host-known sizes,
    so it never synchronises with the device.
    """
    group = max(1, num_heads // max(1, num_kv_heads))
    heads_per_wg = 8 if group >= 8 else 4
    groups = num_kv_heads * math.ceil(group / heads_per_wg)
    base = max(1, batch * groups)
    split = math.ceil(num_cus / base)
    split = min(split, max_split, max(1, max_pages // min_pages_per_split))
    return int(max(1, split))


def decode_heads_per_workgroup(group: int, quantized: bool = False) -> int:
    """Query heads one decode workgroup serves: the MFMA decode (every int8 /
    fp8 cache, and fp16/bf16 caches with group >= 8) takes up to 32, the VALU
    decode (fp16/bf16, group < 8) 4."""
    if quantized or group >= 8:
        return 32
    return 4


def decode_partition(batch: int, num_heads: int, num_kv_heads: int, max_pages: int, total_pages: int,
                     num_cus: int = MI355X_CUS, min_pages_per_split: int = 8,
                     max_split: int = 16, quantized: bool = False, q_len: int = 1) -> tuple[int, int]:
    """``(split_k, pages_per_split)`` for a possibly ragged batch on MI355X.

    Every partition holds the same number of pages and split_k covers the
    longest sequence.  A uniform batch (``batch * max_pages`` below twice
    ``total_pages``) is spread over about one workgroup per CU with at most
    ``max_split`` partitions -- the same launch as :func:`decode_split_k` --
    or up to 64 when every partition still holds at least 256 pages.  A
    skewed batch gets about 4 workgroups per CU (up to 64 partitions), so
    the long sequences are streamed by many workgroups and the dispatcher
    balances the uneven rest, and an odd split_k: workgroups go to the 8 XCDs
    round-robin with the partition index fastest, so with an even split_k the
    only non-empty partition of every short sequence (partition 0) lands on
    half of the XCDs or fewer.  Both regimes were measured on MI355X (32/8
    heads, D128, page 16: the B x ctx sweep; 64 log-uniform lengths in [16,
    65536], 2 x 65536 + 30 x 512 and 128 log-uniform lengths in [16, 16384],
    where this rule with 4-wave workgroups ran 533 / 176 / 324 us against 674
    / 497 / 334 us for 16 workgroups per CU and 8 waves).
    """
    group = max(1, num_heads // max(1, num_kv_heads))
    rows = group * max(1, int(q_len))  # (query head, token) rows per KV head
    heads_per_wg = 32 if q_len > 1 else decode_heads_per_workgroup(group, quantized)
    groups = num_kv_heads * math.ceil(rows / heads_per_wg)
    max_pages = max(1, int(max_pages))
    total_pages = max(1, int(total_pages))
    skewed = is_ragged(batch, max_pages, total_pages)
    target_wgs = 4 * num_cus if skewed else num_cus
    chunk = max(min_pages_per_split, math.ceil(total_pages * groups / target_wgs))
    # Partitions of at least 256 pages may number up to 64: the merge is then
    # negligible and one long sequence still reaches every CU (B1 ctx131072:
    # 32 partitions run 11 % faster than 16 on MI355X).
    cap = 64 if skewed or chunk >= 256 else max_split
    split = math.ceil(max_pages / chunk)
    if split > cap:
        split = cap
        chunk = math.ceil(max_pages / split)
    if skewed and split > 1:
        if split % 2 == 0:
            split = split + 1 if split < cap else split - 1
        chunk = math.ceil(max_pages / split)  # equal partitions of the longest sequence
    return int(max(1, split)), int(chunk)


def is_ragged(batch: int, max_pages: int, total_pages: int) -> bool:
    """A batch whose longest sequence holds at least twice the mean page
    count: :func:`decode_partition` then cuts many short partitions."""
    return int(batch) * max(1, int(max_pages)) >= 2 * max(1, int(total_pages))


# ---------------------------------------------------------------------------
# Tuned-config store (schema of flashattn_tile/autotune.py:376-419, gfx950 keys)
# ---------------------------------------------------------------------------
TUNED_CONFIGS_PATH = Path(__file__).resolve().with_name("tuned_configs_gfx950.json")
_STORE_ENV = "FAT_TUNED_CONFIGS"  # another store file; "" or "none" disables lookups
_STORE_CACHE: dict[str, tuple[int, int, dict]] = {}

_DTYPE_TAGS = {"float16": "fp16", "bfloat16": "bf16", "int8": "int8", "float8_e4m3fn": "fp8"}


def _dtype_tag(dtype) -> str:
    name = str(dtype).replace("torch.", "")
    return _DTYPE_TAGS.get(name, name)


def decode_signature(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                     max_len: int, total_pages: int, kv_dtype, q_len: int = 1) -> str:
    """Store key of a decode launch.  The reference's key
    (``decode.py:525-530``) plus what changes the best gfx950 launch: the
    cache dtype, the query length and whether the batch is ragged."""
    max_pages = -(-int(max_len) // int(page_size))
    sig = (f"B{batch}_H{num_heads}_Hkv{num_kv_heads}_D{head_dim}_P{page_size}_L{max_len}"
           f"_{_dtype_tag(kv_dtype)}")
    if q_len > 1:
        sig += f"_T{q_len}"
    if is_ragged(batch, max_pages, total_pages):
        sig += "_ragged"
    return sig


def prefill_signature(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, max_seqlen_q: int,
                      max_seqlen_k: int, causal: bool) -> str:
    """Store key of a packed prefill launch, the reference's (``prefill.py:276``)."""
    return (f"B{batch}_H{num_heads}_Hkv{num_kv_heads}_D{head_dim}_Lq{max_seqlen_q}_Lk{max_seqlen_k}"
            f"_c{int(bool(causal))}")


def prefill_paged_signature(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                            max_seqlen_q: int, causal: bool) -> str:
    """Store key of a paged prefill launch (no reference counterpart)."""
    return (f"B{batch}_H{num_heads}_Hkv{num_kv_heads}_D{head_dim}_P{page_size}_Lq{max_seqlen_q}"
            f"_c{int(bool(causal))}")


def _store_path(path: Path | str | None = None) -> Path | None:
    if path is not None:
        return Path(path)
    env = os.environ.get(_STORE_ENV)
    if env is not None:
        return None if env.strip().lower() in ("", "none") else Path(env)
    return TUNED_CONFIGS_PATH


def _empty_store() -> dict:
    return {"_meta": {"schema_version": 1, "arch": "gfx950"}, "configs": {}}


def _load_store(path: Path | str | None = None) -> dict:
    """The store as a dict; a missing or unreadable file is an empty store."""
    p = _store_path(path)
    if p is None:
        return _empty_store()
    try:
        st = p.stat()
    except OSError:
        return _empty_store()
    key = str(p)
    hit = _STORE_CACHE.get(key)
    if hit is not None and hit[0] == st.st_mtime_ns and hit[1] == st.st_size:
        return hit[2]
    try:
        data = json.loads(p.read_text())
        if not isinstance(data, dict):
            raise ValueError("not a JSON object")
    except (OSError, ValueError):
        data = _empty_store()
    data.setdefault("configs", {})
    data.setdefault("_meta", {"schema_version": 1, "arch": "gfx950"})
    _STORE_CACHE[key] = (st.st_mtime_ns, st.st_size, data)
    return data


def _write_store(data: dict, path: Path | str | None) -> None:
    p = _store_path(path)
    if p is None:
        raise ValueError(f"the tuned-config store is disabled ({_STORE_ENV}={os.environ.get(_STORE_ENV)!r})")
    data["_meta"]["updated_utc"] = datetime.now(timezone.utc).isoformat()
    tmp = p.with_name(p.name + ".tmp")
    tmp.write_text(json.dumps(data, indent=2) + "\n")
    tmp.replace(p)
    _STORE_CACHE.pop(str(p), None)


def save_best(kind: str, signature: str, config: dict, metrics: dict | None = None,
              path: Path | str | None = None) -> None:
    """Persist the winning config for one problem shape (``autotune.py:390-402``)."""
    data = json.loads(json.dumps(_load_store(path)))  # private copy of the cached store
    data["configs"][f"{kind}:{signature}"] = {
        "kind": kind,
        "signature": signature,
        "config": dict(config),
        "metrics": dict(metrics or {}),
        "recorded_utc": datetime.now(timezone.utc).isoformat(),
    }
    _write_store(data, path)


def best_config(kind: str, signature: str, path: Path | str | None = None) -> dict | None:
    """The persisted winner for ``kind:signature``; ``None`` when nothing was
    tuned (``autotune.py:405-408``).  Reads the file once per modification."""
    entry = _load_store(path)["configs"].get(f"{kind}:{signature}")
    if not isinstance(entry, dict) or not isinstance(entry.get("config"), dict):
        return None
    return dict(entry["config"])


def initialize_store(note: str, path: Path | str | None = None) -> None:
    """Create or refresh the store with a meta block (``autotune.py:411-419``)."""
    data = json.loads(json.dumps(_load_store(path)))
    data["_meta"].update({"schema_version": 1, "arch": "gfx950", "note": note})
    _write_store(data, path)


# ---------------------------------------------------------------------------
# Config space and timing (autotune.py:121-300, gfx950 knobs)
# ---------------------------------------------------------------------------
def build_config_space(kind: str, *, batch: int = 1, num_heads: int = 32, num_kv_heads: int = 8,
                       max_pages: int = 1, total_pages: int | None = None, quantized: bool = False,
                       q_len: int = 1, split_k_choices=(1, 2, 3, 4, 8, 16, 32, 64),
                       num_warps_choices=(4, 8)) -> list[dict]:
    """Candidate launch configs for one shape.

    ``decode``: every split-K count that leaves at least one page per
    partition (the reference's ``ceil(pages / split_k)`` partitioning) times
    4/8-wave workgroups times the VALU and MFMA kernel families, plus the
    :func:`decode_partition` pick; the VALU kernel is left out for
    multi-token decode, which only the MFMA kernel serves.  ``prefill`` and
    ``prefill_paged``: the 8-wave ping-pong, the 4-wave kernel and its 8-wave
    key-split form (and, packed only, the 64-rows-per-wave "wide" kernel).
    """
    if kind == "prefill":
        return [{"kernel": "pingpong"}, {"kernel": "wide"}, {"kernel": "4wave"}, {"kernel": "4wave_split"}]
    if kind == "prefill_paged":
        return [{"kernel": "pingpong"}, {"kernel": "4wave"}, {"kernel": "4wave_split"}]
    if kind != "decode":
        raise ValueError(f"unknown kind {kind!r}")
    max_pages = max(1, int(max_pages))
    total = int(total_pages) if total_pages is not None else int(batch) * max_pages
    kernels = ("mfma",) if q_len > 1 else ("valu", "mfma")
    out: list[dict] = []
    seen = set()
    heur = decode_partition(batch, num_heads, num_kv_heads, max_pages, total, quantized=quantized, q_len=q_len)
    parts = [heur] + [(s, 0) for s in split_k_choices if s <= max_pages]
    for split, pps in parts:
        for warps in num_warps_choices:
            for kern in kernels:
                key = (split, pps, warps, kern)
                if key in seen:
                    continue
                seen.add(key)
                out.append({"split_k": int(split), "pages_per_split": int(pps), "num_warps": int(warps),
                            "kernel": kern})
    return out


def time_callable(fn, warmup: int = 10, iters: int = 50, flush=None) -> list[float]:
    """Per-call latencies of ``fn`` in milliseconds (the role of
    ``autotune.py:241-271``).

    On a ROCm device every call is bracketed by its own pair of HIP events on
    torch's current stream (where the kernels are enqueued); all ``iters``
    calls are enqueued first and the events are read after one final
    synchronisation, so no host round trip sits between two calls.
    ``flush`` (e.g. clearing a 512 MiB buffer) is enqueued before each timed
    call, outside its events, so the 256 MB MALL does not serve a working set
    that fits in it.  Without a device the calls are timed on the host clock.
    Timing inside a graph capture is refused."""
    import torch

    if warmup < 1 or iters < 1:
        raise ValueError("warmup and iters must be >= 1")
    on_device = torch.cuda.is_available()
    if on_device and torch.cuda.is_current_stream_capturing():
        raise RuntimeError("time_callable cannot time inside a graph capture")
    for _ in range(warmup):
        fn()
    if not on_device:
        out = []
        for _ in range(iters):
            t0 = time.perf_counter_ns()
            fn()
            out.append((time.perf_counter_ns() - t0) / 1e6)
        return out
    torch.cuda.synchronize()
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for begin, end in marks:
        if flush is not None:
            flush()
        begin.record()
        fn()
        end.record()
    torch.cuda.synchronize()
    return [float(begin.elapsed_time(end)) for begin, end in marks]


def summarize_times(times: list[float]) -> dict:
    """``median_ms`` / ``mean_ms`` / ``min_ms`` / ``p90_ms`` (nearest-rank
    90th percentile) and ``iters`` of a list of latencies (the columns of
    ``autotune.py:274-287``)."""
    vals = sorted(float(t) for t in times)
    n = len(vals)
    if n == 0:
        raise ValueError("no timings")
    half = n // 2
    median = vals[half] if n % 2 else 0.5 * (vals[half - 1] + vals[half])
    rank90 = -(-9 * n // 10)  # smallest rank r with r / n >= 0.9
    return {"median_ms": median, "mean_ms": math.fsum(vals) / n, "min_ms": vals[0], "p90_ms": vals[rank90 - 1],
            "iters": n}


def time_back_to_back(fn, warmup: int = 3, reps: int = 5, per_rep: int = 20) -> list[float]:
    """``reps`` samples of the mean latency (ms) of ``per_rep`` launches
    enqueued back to back between two HIP events on torch's current stream:
    the steady state of a serving loop, without the per-launch event and
    host round trip of :func:`time_callable`."""
    import torch

    if warmup < 0 or reps < 1 or per_rep < 1:
        raise ValueError("warmup must be >= 0, reps and per_rep >= 1")
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(per_rep):
            fn()
        end.record()
        end.synchronize()
        out.append(float(start.elapsed_time(end)) / per_rep)
    return out


def autotune(problem: dict, candidates: list[dict], warmup: int = 10, iters: int = 50, save: bool = True,
             flush=None, path: Path | str | None = None, timer=None) -> list[dict]:
    """Time every candidate and return the rows ranked by median latency.

    ``problem`` keys (``autotune.py:263-373``): ``kind``, ``signature``,
    ``runner`` (callable taking a config dict), ``flops``, ``bytes``, and
    optionally ``default`` (the config the wrapper would use untuned; its
    latency is stored beside the winner's).  The reference returns a pandas
    DataFrame; this returns a list of dicts with the same columns (``rank``,
    the config keys, ``latency_ms``, ``min_ms``, ``p90_ms``, ``tflops``,
    ``gbytes_per_s``).  A candidate the library rejects (``RuntimeError``,
    ``ValueError``) is skipped.  ``timer`` (a callable taking the launch and
    returning latencies in ms, e.g. :func:`time_back_to_back`) replaces
    :func:`time_callable`.  With ``save`` the winner goes to the store.
    """
    required = {"kind", "signature", "runner", "flops", "bytes"}
    missing = required - set(problem)
    if missing:
        raise ValueError(f"problem is missing keys: {sorted(missing)}")
    if not candidates:
        raise ValueError("no candidates")
    rows = []
    for cfg in candidates:
        try:
            launch = lambda: problem["runner"](cfg)  # noqa: E731
            times = timer(launch) if timer is not None else time_callable(launch, warmup=warmup, iters=iters,
                                                                            flush=flush)
        except (RuntimeError, ValueError) as exc:
            warnings.warn(f"autotune: candidate {cfg} skipped: {exc}", RuntimeWarning, stacklevel=2)
            continue
        stats = summarize_times(times)
        lat = stats["median_ms"]
        rows.append({
            **cfg,
            "latency_ms": lat,
            "min_ms": stats["min_ms"],
            "p90_ms": stats["p90_ms"],
            "tflops": problem["flops"] / (lat * 1e-3) / 1e12,
            "gbytes_per_s": problem["bytes"] / (lat * 1e-3) / 1e9,
            "flops": problem["flops"],
            "bytes": problem["bytes"],
        })
    if not rows:
        raise RuntimeError(f"autotune: every candidate failed for {problem['kind']}:{problem['signature']}")
    rows.sort(key=lambda r: r["latency_ms"])
    for i, r in enumerate(rows):
        r["rank"] = i + 1
    if save:
        win = rows[0]
        keys = list(candidates[0].keys())
        metrics = {"latency_ms": win["latency_ms"], "gbytes_per_s": win["gbytes_per_s"], "tflops": win["tflops"]}
        default = problem.get("default")
        if default is not None:
            match = [r for r in rows if all(r.get(k) == default.get(k) for k in keys)]
            if match:
                metrics["default_ms"] = match[0]["latency_ms"]
        save_best(problem["kind"], problem["signature"], {k: win[k] for k in keys}, metrics, path=path)
    return rows
