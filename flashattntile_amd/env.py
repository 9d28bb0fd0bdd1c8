"""MI355X spec peaks and the host/device facts a measurement records.

Replaces the NVIDIA tables of ``flashattn_tile/env.py:31-56``: the roofline
denominators here are AMD's published MI355X figures (dense, no sparsity),
and :func:`host_info` / :func:`cpu_threads` describe the CPU the oracle
baseline runs on (``bench.py`` takes both from here).
"""

from __future__ import annotations

import math
import os
import platform

MI355X = {
    "name": "AMD Instinct MI355X",
    "arch": "gfx950",
    "compute_units": 256,
    "xcds": 8,
    "lds_bytes_per_cu": 160 * 1024,
    "hbm_bytes": 288 * 1024**3,
    "hbm_gbs": 8000.0,
    "mfma_dense_tflops": {"fp16": 2516.6, "bf16": 2516.6, "fp8": 5033.2, "int8": 5033.2},
    "vector_fp32_tflops": 157.3,
}


def peak_hbm_gbs() -> float:
    return MI355X["hbm_gbs"]


def peak_mfma_tflops(dtype: str = "fp16") -> float:
    return MI355X["mfma_dense_tflops"][dtype]


def _cgroup_cpu_quota() -> float | None:
    """CPUs this process may use per the cgroup v2 ``cpu.max`` quota (None
    when unlimited or unreadable)."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as fh:
            quota, period = fh.read().split()[:2]
    except (OSError, ValueError):
        return None
    if quota == "max":
        return None
    try:
        return float(quota) / float(period)
    except (ValueError, ZeroDivisionError):
        return None


def host_info() -> dict:
    """Affinity core count, ``os.cpu_count()``, the cgroup CPU quota and the
    full CPU model string of this host."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover - non-Linux
        cores = os.cpu_count() or 1
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:  # pragma: no cover
        pass
    return {"affinity_cores": cores, "os_cpu_count": os.cpu_count(), "cgroup_cpu_quota": _cgroup_cpu_quota(),
            "cpu_model": model}


def cpu_threads(info: dict | None = None) -> int:
    """Threads for a CPU baseline: the affinity cores, bounded by the cgroup
    quota when one is set (more threads than the quota only time-slice)."""
    info = info or host_info()
    n = info["affinity_cores"]
    quota = info.get("cgroup_cpu_quota")
    if quota:
        n = min(n, max(1, math.floor(quota)))
    return max(1, n)


def device_info() -> dict:
    import torch

    info = {"torch": torch.__version__, "hip": getattr(torch.version, "hip", None), **host_info()}
    if torch.cuda.is_available():
        props = torch.cuda.get_device_properties(0)
        info.update({
            "device": props.name,
            "gcn_arch": getattr(props, "gcnArchName", ""),
            "compute_units": props.multi_processor_count,
            "total_memory": props.total_memory,
        })
    return info
