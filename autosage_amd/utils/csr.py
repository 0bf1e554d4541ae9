"""edge_index -> CSR with destination rows (``autosage/utils/csr.py:6-26``).

Rows are ``edge_index[1]`` (destinations) by default.  Edges are ordered by a
stable sort of the row ids, so within a row the columns keep their edge_index
order; ``crow`` is the cumulative count of edges per row.  Integer-only and
identical on CPU and GPU.  The steps (stable argsort, ``index_add_`` of ones
at row + 1, ``cumsum``) are the reference's, because the output must be
bit-identical to it.
"""

from __future__ import annotations

import torch


def csr_with_edge_order(
    edge_index: torch.Tensor,
    num_nodes: int,
    *,
    rows_by: str = "dst",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(crow, col, order): the CSR of ``edge_index_to_csr`` and the edge
    permutation that produced it — CSR position k holds edge ``order[k]`` of
    ``edge_index`` — so per-edge data (weights) follows with one
    ``index_select``."""
    if edge_index.ndim != 2 or edge_index.size(0) != 2:
        raise ValueError("edge_index must have shape [2, E]")
    if rows_by not in ("dst", "src"):
        raise ValueError("rows_by must be 'dst' or 'src'")
    src = edge_index[0].to(dtype=torch.long)
    dst = edge_index[1].to(dtype=torch.long)
    rows, cols = (dst, src) if rows_by == "dst" else (src, dst)
    order = rows.argsort(stable=True)
    counts = torch.zeros(num_nodes + 1, dtype=torch.long, device=rows.device)
    # integer counts: the order of the additions does not matter
    counts.index_add_(0, rows + 1, torch.ones_like(rows))
    return counts.cumsum(0).contiguous(), cols.index_select(0, order).contiguous(), order


def edge_index_to_csr(
    edge_index: torch.Tensor,
    num_nodes: int,
    *,
    rows_by: str = "dst",
) -> tuple[torch.Tensor, torch.Tensor]:
    crow, col, _ = csr_with_edge_order(edge_index, num_nodes, rows_by=rows_by)
    return crow, col


__all__ = ["csr_with_edge_order", "edge_index_to_csr"]
