"""Shared helpers for the GPU parity tests."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import autosage_amd
from autosage_amd import synth


def require_gpu():
    """Skips without a GPU; with a GPU the HIP library must load (no silent
    fallback), otherwise the test fails."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not autosage_amd.load_native():
        from autosage_amd.ops import native_load_error

        pytest.fail(f"HIP library failed to load on a GPU machine: {native_load_error()}")


def case_graph(rows: int, degree: float, seed: int, hubs: int = 0, hub_degree: int = 0, empty: float = 0.0):
    crow, col = synth.random_csr(rows, degree, seed=seed, hub_rows=hubs, hub_degree=hub_degree, empty_fraction=empty)
    return crow, col


def to_dev(*arrays):
    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def bitwise_equal(gpu: torch.Tensor, ref: np.ndarray) -> bool:
    got = gpu.detach().cpu().numpy()
    return got.shape == ref.shape and np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def mismatch_report(gpu: torch.Tensor, ref: np.ndarray) -> str:
    got = gpu.detach().cpu().numpy()
    bad = np.argwhere(got != ref)
    return f"{len(bad)} mismatches, first {bad[:5].tolist()}: got {got[tuple(bad[0])] if len(bad) else None}"
