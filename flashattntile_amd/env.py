"""MI355X spec peaks and a small device probe.

Replaces the NVIDIA tables of ``flashattn_tile/env.py:31-56``: the roofline
denominators here are AMD's published MI355X figures (dense, no sparsity).
"""

from __future__ import annotations

import os
import platform

import torch

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


def host_info() -> dict:
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
    return {"affinity_cores": cores, "os_cpu_count": os.cpu_count(), "cpu_model": model}


def device_info() -> dict:
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
