"""Graph convolution layer on the scheduled SpMM (``autosage/conv.py:13-56``).

``AutoSAGEConv(in, out)`` sums the (optionally weighted) features of every
node's in-neighbours — CSR rows are destinations, ``edge_index[1]`` — and
applies a ``nn.Linear``.  Constructor arguments, error messages and the info
dictionary of ``mode="native"`` are the reference's interface.

Per-graph work is done once: the CSR of an ``edge_index`` and the edge
permutation of its stable sort are memoised per live, unmodified
``edge_index`` tensor.  Edge weights follow their edges through that same
permutation (one ``index_select``, no second sort), and because the same
``crow`` / ``col`` tensors come back on every forward over a graph, the
per-graph memos behind the scheduler (schedule key, slice counts, row-sorted
copy, transposed CSR of the backward) hit from the second call on.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from ._auto import spmm_csr_auto
from ._memo import GraphMemo
from .ops import spmm_csr
from .utils.csr import csr_with_edge_order

_CSR_MEMO = GraphMemo("edge_index_csr", max_entries=32, max_bytes=4 << 30)


def _graph_csr(edge_index: torch.Tensor, num_nodes: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _CSR_MEMO.get(
        (edge_index,), int(num_nodes), lambda: csr_with_edge_order(edge_index, num_nodes, rows_by="dst")
    )


def _weights_in_csr_order(edge_weight: torch.Tensor, edge_index: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    if edge_weight.ndim != 1 or edge_weight.numel() != edge_index.size(1):
        raise ValueError("edge_weight must contain one value per edge")
    if edge_weight.device != edge_index.device:
        raise ValueError("edge_weight and edge_index must be on the same device")
    return edge_weight.index_select(0, order)


class AutoSAGEConv(nn.Module):
    """Neighbour-sum aggregation on the native SpMM followed by a linear map.

    ``mode="auto"`` runs ``spmm_csr_auto`` (scheduled, cached per graph) and
    returns its info dictionary; ``mode="native"`` calls ``spmm_csr``
    directly.
    """

    def __init__(self, in_channels: int, out_channels: int, *, mode: str = "auto", bias: bool = True) -> None:
        super().__init__()
        if mode not in ("auto", "native"):
            raise ValueError("mode must be 'auto' or 'native'")
        self.mode = mode
        self.linear = nn.Linear(in_channels, out_channels, bias=bias)

    def forward(
        self,
        x: torch.Tensor,
        edge_index: torch.Tensor,
        edge_weight: Optional[torch.Tensor] = None,
        *,
        return_info: bool = False,
    ):
        crow, col, order = _graph_csr(edge_index, x.size(0))
        weights = None if edge_weight is None else _weights_in_csr_order(edge_weight, edge_index, order)
        if self.mode == "native":
            summed = spmm_csr(crow, col, weights, x)
            info = {"operation": "spmm", "choice": "native" if x.is_cuda else "baseline", "from_cache": False}
        else:
            summed, info = spmm_csr_auto(crow, col, weights, x)
        out = self.linear(summed)
        if return_info:
            return out, info
        return out
