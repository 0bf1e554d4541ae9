"""Drop-in import name of the reference package (``autosage/__init__.py:1-17``).

The implementation lives in ``autosage_amd``.  This package re-exports its
public names and registers its modules under the reference's module paths
(``autosage.ops``, ``autosage._auto``, ``autosage._cache``,
``autosage.config``, ``autosage.conv``, ``autosage.utils``,
``autosage.utils.csr``, ``autosage._version``), so that code written against
the reference — ``from autosage._auto import _prepare_spmm_baseline,
_run_spmm_choice, _time_cuda`` (``scripts/benchmark.py:16-24``,
``scripts/probe_overhead.py:11-12``, ``scripts/sweep_hubs.py:11-12``) or
``from autosage._cache import ScheduleCache`` (``tests/test_cache.py:7``) —
runs unchanged.  Each alias is the same module object, so state such as the
loaded library and the schedule-cache memos is shared with ``autosage_amd``.
"""

from __future__ import annotations

import importlib
import sys

import autosage_amd as _impl
from autosage_amd import (
    AutoSAGEConv,
    __version__,
    calibrate_full,
    csr_attention_forward,
    load_native,
    native_available,
    sddmm_csr_auto,
    spmm_csr,
    spmm_csr_auto,
    validate_csr,
)

# Submodules of the reference package, plus the two private modules of this
# implementation that hold the native bindings and the backward formulas.
_ALIASED = ("_version", "config", "ops", "_cache", "_auto", "conv", "utils", "utils.csr", "_native", "_autograd")


def _alias_submodules() -> None:
    for name in _ALIASED:
        module = importlib.import_module(f"{_impl.__name__}.{name}")
        sys.modules[f"{__name__}.{name}"] = module
        parent, _, leaf = name.rpartition(".")
        owner = sys.modules[f"{__name__}.{parent}"] if parent else sys.modules[__name__]
        setattr(owner, leaf, module)


_alias_submodules()

__all__ = [
    "AutoSAGEConv",
    "__version__",
    "calibrate_full",
    "csr_attention_forward",
    "load_native",
    "native_available",
    "sddmm_csr_auto",
    "spmm_csr",
    "spmm_csr_auto",
    "validate_csr",
]
