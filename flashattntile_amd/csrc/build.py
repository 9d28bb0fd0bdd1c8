"""Build libfat_hip.so for gfx950 with hipcc (no torch extension machinery).

Usage: python -m flashattntile_amd.csrc.build   (or build() from Python).
The library lands next to this file's package as flashattntile_amd/_lib/.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
REPO = PKG.parent
LIB_DIR = PKG / "_lib"
LIB_NAME = "libfat_hip.so"
SOURCES = ["abi.hip", "decode.hip", "decode_generic.hip", "prefill.hip", "prefill_wide.hip", "prefill_generic.hip",
           "prefill_stage.hip", "kvwrite.hip", "validate.hip"]
ARCH = os.environ.get("FAT_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops is switched off: the kernels use scalar fp32 FMAs only.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
    "-munsafe-fp-atomics",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link libfat_hip.so; returns its path."""
    cc = hipcc()
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    include = ["-I", str(REPO / "include"), "-I", str(HERE)]
    procs = []
    objs = []
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, *include, "-c", str(HERE / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    errors = []
    for src, proc in procs:
        out, _ = proc.communicate()
        if proc.returncode != 0:
            errors.append(f"--- {src} ---\n{out}")
        elif verbose and out.strip():
            print(out)
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
    lib = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + res.stdout)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
