"""The native induced-sample passes (``as_induced_sample_count/_fill``)
against the reference's torch composition, on the same device and the same
seeded row sample: integer outputs identical, values bit for bit.  The CPU
restatement, fed the same sample, gives the same sub-graph too."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from autosage_amd import _native
from autosage_amd._auto import _induced_sample_csr, _induced_subgraph_torch
from tests.gpu_common import case_graph, require_gpu, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _sample(rows: int, fraction: float, minimum: int, seed: int) -> torch.Tensor:
    size = min(max(int(rows * fraction), minimum, 1), rows)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randperm(rows, generator=g, device="cuda")[:size].sort().values


def _same(a, b):
    if a is None or b is None:
        return a is None and b is None
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize(
    "rows, degree, hubs, fraction, minimum",
    [(5000, 12, 4, 0.03, 512), (5000, 12, 4, 0.5, 512), (300, 6, 1, 0.03, 512), (20000, 3, 10, 0.1, 64)],
)
def test_native_sample_equals_torch_composition(rows, degree, hubs, fraction, minimum, weighted):
    crow, col = case_graph(rows, degree, seed=rows + hubs, hubs=hubs, hub_degree=min(rows, 3000), empty=0.1)
    val = np.random.default_rng(1).standard_normal(col.size).astype(np.float32) if weighted else None
    d_crow, d_col, d_val = to_dev(crow, col, val)
    selected = _sample(rows, fraction, minimum, seed=7)
    native = _native.induced_sample(d_crow, d_col, d_val, selected)
    torch_path = _induced_subgraph_torch(d_crow, d_col, d_val, selected)
    for got, want in zip(native, torch_path):
        assert _same(got, want)
    # the scheduler's entry point takes the native path on the GPU
    s_crow, s_col, s_val, s_sel = _induced_sample_csr(d_crow, d_col, d_val, fraction=fraction, minimum_rows=minimum,
                                                      seed=7)
    assert torch.equal(s_sel, selected) and _same(s_crow, native[0]) and _same(s_col, native[1])
    assert _same(s_val, native[2])
    # the CPU composition with the same sample gives the same sub-graph
    cpu = _induced_subgraph_torch(torch.from_numpy(crow), torch.from_numpy(col),
                                  None if val is None else torch.from_numpy(val), selected.cpu())
    for got, want in zip(native, cpu):
        assert _same(got, want)


def test_native_sample_edge_cases():
    # no edges at all
    crow = torch.zeros(101, dtype=torch.long, device="cuda")
    col = torch.zeros(0, dtype=torch.long, device="cuda")
    sel = _sample(100, 0.5, 1, 0)
    new_crow, new_col, new_val = _native.induced_sample(crow, col, None, sel)
    assert torch.count_nonzero(new_crow).item() == 0 and new_col.numel() == 0 and new_val is None
    # every row sampled: the graph itself
    c, k = case_graph(700, 5, seed=3)
    d_crow, d_col = to_dev(c, k)
    new_crow, new_col, _ = _native.induced_sample(d_crow, d_col, None, torch.arange(700, device="cuda"))
    assert torch.equal(new_crow, d_crow) and torch.equal(new_col, d_col)
    # a column outside [0, N) is dropped, not read out of bounds
    bad = k.copy()
    bad[0] = 700
    new_crow, new_col, _ = _native.induced_sample(d_crow, torch.from_numpy(bad).cuda(), None,
                                                  torch.arange(700, device="cuda"))
    assert new_col.numel() == k.size - 1 and torch.equal(new_col, d_col[1:])
