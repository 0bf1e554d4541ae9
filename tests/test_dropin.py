"""The drop-in import name ``autosage``: every module path and private name
that the reference's scripts and tests import resolves, and to the same
objects as the implementation package."""

from __future__ import annotations

import importlib

import pytest

import autosage_amd

# (module, names) imported by the reference's callers:
# scripts/benchmark.py:16-24, scripts/probe_overhead.py:11-12,
# scripts/sweep_hubs.py:11-12, tests/test_cache.py:7, tests/test_cpu.py:6-8,
# tests/test_cuda.py:6-7, tests/test_scheduler.py:5-6
REFERENCE_IMPORTS = [
    ("autosage", ["calibrate_full", "csr_attention_forward", "load_native", "native_available", "spmm_csr_auto",
                  "sddmm_csr_auto", "spmm_csr", "AutoSAGEConv", "__version__"]),
    ("autosage._auto", ["_prepare_spmm_baseline", "_run_spmm_choice", "_time_cuda", "_csr_row_softmax",
                        "sddmm_csr_auto", "_spmm_candidates"]),
    ("autosage._cache", ["ScheduleCache", "cache_directory", "graph_signature"]),
    ("autosage.config", ["SchedulerConfig"]),
    ("autosage.utils.csr", ["edge_index_to_csr"]),
    ("autosage.ops", ["load_native", "native_available", "native_op", "native_load_error", "spmm_csr"]),
    ("autosage.conv", ["AutoSAGEConv"]),
]


@pytest.mark.parametrize("module, names", REFERENCE_IMPORTS)
def test_reference_imports_resolve_to_the_implementation(module, names):
    aliased = importlib.import_module(module)
    impl = importlib.import_module(module.replace("autosage", "autosage_amd", 1))
    for name in names:
        assert getattr(aliased, name) is getattr(impl, name), f"{module}.{name}"


def test_submodules_are_the_same_objects():
    import autosage

    for name in ("ops", "_auto", "_cache", "config", "conv", "utils", "_version"):
        assert getattr(autosage, name) is getattr(autosage_amd, name)
    assert autosage.utils.csr is autosage_amd.utils.csr
    from autosage import _auto as aliased_auto

    assert aliased_auto is autosage_amd._auto
