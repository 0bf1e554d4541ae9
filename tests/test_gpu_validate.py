"""The device CSR structure check (``validate_csr`` / ``as_csr_validate``)
and the ``AUTOSAGE_VALIDATE`` switch on the operators.  Every malformed
graph here is built so that the check itself stays in bounds: it reads
exactly the ``crow`` and ``col`` tensors handed to it."""

from __future__ import annotations

import pytest
import torch

import autosage_amd
from autosage_amd import validate_csr

from gpu_common import case_graph, require_gpu, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    require_gpu()


def _graph(rows=3000, seed=7):
    crow, col = case_graph(rows, 9.0, seed, hubs=2, hub_degree=2000, empty=0.05)
    return to_dev(crow, col)


def test_valid_graphs_pass():
    crow, col = _graph()
    validate_csr(crow, col)
    validate_csr(crow.to(torch.int32), col.to(torch.int32))
    # empty graphs: no rows, and rows without edges
    validate_csr(torch.zeros(1, dtype=torch.long, device="cuda"), torch.zeros(0, dtype=torch.long, device="cuda"))
    validate_csr(torch.zeros(5, dtype=torch.long, device="cuda"), torch.zeros(0, dtype=torch.long, device="cuda"))


@pytest.mark.parametrize(
    "mutate, message",
    [
        (lambda crow, col: crow.__setitem__(0, 1), "crow[0] must be 0"),
        (lambda crow, col: crow.__setitem__(1500, crow[1500] + 40), "crow must be non-decreasing"),
        (lambda crow, col: crow.__setitem__(-1, crow[-1] - 1), "crow[-1] must equal the number of nonzeros"),
        (lambda crow, col: col.__setitem__(col.numel() // 2, 3000), "column indices must lie in [0, N)"),
        (lambda crow, col: col.__setitem__(-1, -1), "column indices must lie in [0, N)"),
    ],
)
def test_each_rule_is_reported(mutate, message):
    crow, col = _graph()
    mutate(crow, col)
    with pytest.raises(ValueError) as info:
        validate_csr(crow, col)
    assert message in str(info.value)


def test_several_rules_at_once_and_rectangular_columns():
    crow, col = _graph()
    crow[0] = 2
    col[0] = 5000
    with pytest.raises(ValueError) as info:
        validate_csr(crow, col)
    text = str(info.value)
    assert "crow[0] must be 0" in text and "column indices" in text
    # a wider column space accepts the same column
    crow, col = _graph()
    col[0] = 5000
    validate_csr(crow, col, n_cols=5001)


def test_operators_validate_under_the_switch(monkeypatch):
    crow, col = _graph()
    x = torch.randn(3000, 64, device="cuda")
    col[10] = 3000  # out of range: must be rejected before any gather
    monkeypatch.setenv("AUTOSAGE_VALIDATE", "1")
    with pytest.raises(ValueError, match="column indices"):
        torch.ops.autosage.spmm_csr(crow, col, None, x)
    with pytest.raises(ValueError, match="column indices"):
        torch.ops.autosage.sddmm_csr(crow, col, x, x)
    with pytest.raises(ValueError, match="column indices"):
        autosage_amd.csr_attention_forward(crow, col, x, x, x)
    col[10] = 0
    y = torch.ops.autosage.spmm_csr(crow, col, None, x)
    monkeypatch.delenv("AUTOSAGE_VALIDATE")
    assert torch.equal(y, torch.ops.autosage.spmm_csr(crow, col, None, x))
