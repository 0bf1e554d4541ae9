"""edge_index -> CSR with destination rows (``autosage/utils/csr.py:6-26``).

Rows are ``edge_index[1]`` (destinations) by default.  Edges are ordered by a
stable sort of the row ids, so within a row the columns keep their edge_index
order; ``crow`` is the cumulative count of edges per row.  Integer-only and
identical on CPU and GPU.
"""

from __future__ import annotations

import torch


def edge_index_to_csr(
    edge_index: torch.Tensor,
    num_nodes: int,
    *,
    rows_by: str = "dst",
) -> tuple[torch.Tensor, torch.Tensor]:
    if edge_index.ndim != 2 or edge_index.size(0) != 2:
        raise ValueError("edge_index must have shape [2, E]")
    if rows_by not in ("dst", "src"):
        raise ValueError("rows_by must be 'dst' or 'src'")
    src = edge_index[0].to(dtype=torch.long)
    dst = edge_index[1].to(dtype=torch.long)
    rows, cols = (dst, src) if rows_by == "dst" else (src, dst)
    order = rows.argsort(stable=True)
    rows = rows[order]
    counts = torch.zeros(num_nodes + 1, dtype=torch.long, device=rows.device)
    counts.index_add_(0, rows + 1, torch.ones_like(rows))
    return counts.cumsum(0).contiguous(), cols[order].contiguous()


__all__ = ["edge_index_to_csr"]
