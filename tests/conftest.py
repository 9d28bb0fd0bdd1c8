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
