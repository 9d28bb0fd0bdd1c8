"""Test bootstrap: in-tree imports, the ``gpu`` marker and shared fixtures."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

# config=None launches use the library's heuristics, not the committed tuned
# store: a stored `kernel` would override the kernel-forcing fixtures.  The
# store tests point FAT_TUNED_CONFIGS at a file of their own.
os.environ["FAT_TUNED_CONFIGS"] = "none"

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm device in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Worst parity figures of the run per output dtype (tests/_parity.py)."""
    try:
        from _parity import RECORDS
    except ImportError:  # pragma: no cover
        return
    if not RECORDS:
        return
    terminalreporter.write_sep("-", "parity against the fp32 oracle (worst per output dtype)")
    for dt in sorted({r[1] for r in RECORDS}):
        rows = [r for r in RECORDS if r[1] == dt]
        raw = max(rows, key=lambda r: r[2])
        fp = max(rows, key=lambda r: r[3])
        terminalreporter.write_line(
            f"{dt}: {len(rows)} checks; max |out - oracle({dt})| = {raw[2]:.3e} ({raw[0]}); "
            f"max |out - oracle(fp32)| = {fp[3]:.3e} ({fp[0]})")
