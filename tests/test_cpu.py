"""CPU behaviour of the public API, exercised through the drop-in ``autosage``
import name.

The known answers are the reference suite's (``tests/test_cpu.py:16-85`` of
the reference): destination-row orientation, weighted rows with an empty row,
the CPU info dictionary, the SDDMM values [4, 7, 10], the softmax of a
one-edge row, the convolution's reordered weights [[90], [20], [0]] and the
rejection of fractional indices.  Every float expected here is exact in
fp32, so results are compared bit for bit.
"""

from __future__ import annotations

import pytest
import torch

import autosage
import autosage_amd
from autosage._auto import _csr_row_softmax, sddmm_csr_auto
from autosage.utils.csr import edge_index_to_csr

REFERENCE_EXPORTS = (
    "AutoSAGEConv",
    "__version__",
    "calibrate_full",
    "csr_attention_forward",
    "load_native",
    "native_available",
    "sddmm_csr_auto",
    "spmm_csr",
    "spmm_csr_auto",
)


def _csr_from_rows(rows: list[list[tuple[int, float]]]) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """CSR (crow, col, val) of a graph given as per-row (column, weight) lists."""
    lengths = torch.tensor([0] + [len(r) for r in rows], dtype=torch.long)
    col = torch.tensor([c for r in rows for c, _ in r], dtype=torch.long)
    val = torch.tensor([w for r in rows for _, w in r], dtype=torch.float32)
    return lengths.cumsum(0), col, val


def test_drop_in_surface():
    assert autosage.__version__ == "0.1.0"
    for name in REFERENCE_EXPORTS:
        assert name in autosage.__all__ and hasattr(autosage, name)
    assert autosage.spmm_csr is autosage_amd.spmm_csr
    assert callable(autosage.spmm_csr)


def test_rows_are_destinations():
    # a directed 4-cycle i -> i+1: node i receives the features of node i-1
    src = torch.arange(4)
    edge_index = torch.stack([src, (src + 1) % 4])
    crow, col = edge_index_to_csr(edge_index, 4)
    x = torch.arange(12, dtype=torch.float32).reshape(4, 3)
    assert torch.equal(autosage.spmm_csr(crow, col, None, x), x.roll(1, dims=0))
    # rows_by="src" is the transpose: node i receives from node i+1
    crow_s, col_s = edge_index_to_csr(edge_index, 4, rows_by="src")
    assert torch.equal(autosage.spmm_csr(crow_s, col_s, None, x), x.roll(-1, dims=0))


def test_weighted_rows_and_an_empty_row():
    crow, col, val = _csr_from_rows([[(1, 0.5), (2, 2.0)], [], [(0, -1.0)]])
    x = torch.tensor([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]])
    want = torch.tensor([[11.5, 14.0], [0.0, 0.0], [-1.0, -2.0]])
    assert torch.equal(autosage.spmm_csr(crow, col, val, x), want)


def test_auto_scheduler_on_cpu_reports_the_baseline():
    crow, col, _ = _csr_from_rows([[(1, 1.0)], [(0, 1.0)]])
    x = torch.randn(2, 4)
    y, info = autosage.spmm_csr_auto(crow, col, None, x)
    assert torch.equal(y, x.flip(0))
    assert info == {
        "operation": "spmm",
        "schema_version": 3,
        "choice": "baseline",
        "baseline": "torch CPU",
        "from_cache": False,
        "reason": "AutoSAGE scheduling is CUDA-only",
    }


def test_sddmm_values_and_row_softmax():
    crow, col, _ = _csr_from_rows([[(0, 1.0), (1, 1.0)], [(0, 1.0)]])
    query = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
    key = torch.tensor([[2.0, 1.0], [1.0, 3.0]])
    scores, info = sddmm_csr_auto(crow, col, query, key)
    # <q0,k0> = 4, <q0,k1> = 7, <q1,k0> = 10
    assert torch.equal(scores, torch.tensor([4.0, 7.0, 10.0]))
    assert (info["choice"], info["baseline"]) == ("baseline", "gather-dot")
    probs = _csr_row_softmax(crow, scores)
    assert torch.allclose(probs[:2], torch.softmax(torch.tensor([4.0, 7.0]), 0))
    assert torch.equal(probs[2:], torch.ones(1))


def test_convolution_shapes_and_telemetry():
    layer = autosage.AutoSAGEConv(3, 2)
    x = torch.randn(2, 3)
    edge_index = torch.tensor([[0, 1], [1, 0]])
    plain = layer(x, edge_index)
    out, info = layer(x, edge_index, return_info=True)
    assert plain.shape == out.shape == (2, 2)
    assert torch.equal(plain, out)
    assert info["choice"] == "baseline"
    native_out, native_info = autosage.AutoSAGEConv(3, 2, mode="native")(x, edge_index, return_info=True)
    assert native_out.shape == (2, 2)
    assert native_info == {"operation": "spmm", "choice": "baseline", "from_cache": False}
    with pytest.raises(ValueError, match="'auto' or 'native'"):
        autosage.AutoSAGEConv(3, 2, mode="fused")


def test_convolution_weights_follow_their_edges():
    # edges 2->0 (w 10), 0->1 (w 20), 1->0 (w 30): node 0 gets 10·x2 + 30·x1 = 90,
    # node 1 gets 20·x0 = 20, node 2 nothing
    edge_index = torch.tensor([[2, 0, 1], [0, 1, 0]])
    weights = torch.tensor([10.0, 20.0, 30.0])
    x = torch.tensor([[1.0], [2.0], [3.0]])
    layer = autosage.AutoSAGEConv(1, 1, mode="native", bias=False)
    with torch.no_grad():
        layer.linear.weight.fill_(1.0)
    assert torch.equal(layer(x, edge_index, weights), torch.tensor([[90.0], [20.0], [0.0]]))
    with pytest.raises(ValueError, match="one value per edge"):
        layer(x, edge_index, weights[:2])


def test_convolution_builds_each_graph_once():
    from autosage_amd.conv import _graph_csr

    edge_index = torch.tensor([[2, 0, 1, 2], [0, 1, 0, 1]])
    first = _graph_csr(edge_index, 3)
    again = _graph_csr(edge_index, 3)
    assert all(a is b for a, b in zip(first, again))
    crow, col, order = first
    assert torch.equal(crow, torch.tensor([0, 2, 4, 4]))
    assert torch.equal(col, torch.tensor([2, 1, 0, 2]))
    assert torch.equal(order, torch.tensor([0, 2, 1, 3]))
    # an in-place edit of edge_index is a new graph
    edge_index[1, 3] = 2
    crow2, _, _ = _graph_csr(edge_index, 3)
    assert torch.equal(crow2, torch.tensor([0, 2, 3, 4]))


def test_fractional_indices_are_rejected():
    with pytest.raises(TypeError, match="integer indices"):
        autosage.spmm_csr(torch.tensor([0.0, 1.0]), torch.tensor([0.0]), None, torch.ones(1, 1))


@pytest.mark.parametrize(
    "crow, col, val, x, exc, message",
    [
        (torch.tensor([[0, 1]]), torch.tensor([0]), None, torch.ones(1, 1), ValueError, "one-dimensional"),
        (torch.tensor([0, 1]), torch.tensor([0]), None, torch.ones(1), ValueError, r"shape \[N, F\]"),
        (torch.tensor([0, 1]), torch.tensor([0]), None, torch.ones(1, 1, dtype=torch.long), TypeError,
         "floating-point"),
        (torch.tensor([0, 1, 1]), torch.tensor([0]), None, torch.ones(1, 1), ValueError, "N \\+ 1"),
        (torch.tensor([0, 1]), torch.tensor([0]), torch.ones(2), torch.ones(1, 1), ValueError, "one weight"),
    ],
)
def test_validation_messages_match_reference(crow, col, val, x, exc, message):
    with pytest.raises(exc, match=message):
        autosage.spmm_csr(crow, col, val, x)


def test_int32_indices_are_promoted():
    crow = torch.tensor([0, 1, 2], dtype=torch.int32)
    col = torch.tensor([1, 0], dtype=torch.int32)
    x = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
    assert torch.equal(autosage.spmm_csr(crow, col, None, x), torch.tensor([[3.0, 4.0], [1.0, 2.0]]))


def test_cpu_attention_composes_sddmm_softmax_spmm():
    crow = torch.tensor([0, 2, 3], dtype=torch.long)
    col = torch.tensor([0, 1, 0], dtype=torch.long)
    q = torch.tensor([[1.0, 0.0], [0.0, 1.0]])
    k = torch.tensor([[1.0, 0.0], [0.0, 1.0]])
    v = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
    out, info = autosage.csr_attention_forward(crow, col, q, k, v)
    p = torch.softmax(torch.tensor([1.0, 0.0]), 0)
    assert torch.allclose(out[0], p[0] * v[0] + p[1] * v[1])
    assert torch.allclose(out[1], v[0])
    assert set(info) == {"sddmm", "spmm"}
