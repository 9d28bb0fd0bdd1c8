"""The reference's import paths, resolved to this build's modules.

A caller of the reference imports ``flashattn_tile`` and its submodules
(``flashattn_tile/__init__.py:22-39``; ``flashattn_tile.kernels.decode``,
``.kernels.prefill``, ``.paging``, ``.quant``, ``.backend``, ``.ops``,
``.autotune``, ``.native``, ``.env``).  Importing this package registers each
of those names in ``sys.modules`` as the *same module object* as its
:mod:`flashattntile_amd` counterpart, so ``from flashattn_tile.kernels.decode
import paged_decode_attention`` (or ``import flashattn_tile.paging as p``)
gets the MI355X implementation, monkeypatching either name patches both, and
the custom ops are registered under ``torch.ops.flashattn_tile`` as the
reference registers them.

Not provided: ``flashattn_tile.reference``, the reference's fp32 oracle.  Its
restatement is test infrastructure here (``oracle/reference.py``) and the
product never imports it.
"""

from __future__ import annotations

import importlib
import sys

import flashattntile_amd as _impl
from flashattntile_amd import *  # noqa: F401,F403  (the public API, same objects)
from flashattntile_amd import __all__, __version__  # noqa: F401

SUBMODULES = ("ops", "paging", "quant", "backend", "autotune", "native", "env", "kernels", "kernels.decode",
              "kernels.prefill")

for _name in SUBMODULES:
    _mod = importlib.import_module(f"{_impl.__name__}.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _mod
    if "." not in _name:
        globals()[_name] = _mod
del _name, _mod
