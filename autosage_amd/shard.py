"""Row shards: one GPU's share of a graph split by rows over several GPUs.

SpMM, SDDMM, the CSR row softmax and attention compute every output row
from that row's own edges and gathered rows of the dense operands, so a
graph splits over P GPUs by rows and no sum crosses GPUs:

* cut points: shard k holds rows [r_k, r_{k+1}), where r_k is the first
  row r with crow[r] >= ceil(k·nnz / P) (r_0 = 0, r_P = N).  These are
  nnz-balanced prefixes of crow: a run of hub rows spreads over the GPUs and
  every shard holds nnz / P edges give or take one row's degree;
* a shard's graph is the CSR of its rows with crow rebased to start at 0
  and the columns unchanged, an (r_{k+1} - r_k) × N matrix; each GPU needs
  the whole of X (one all-gather of the N × F features over the GPUs'
  links before the product);
* its product is rows [r_k, r_{k+1}) of the whole graph's product.

This module runs one shard on one GPU at its real shape, for the SpMM, the
SDDMM and the attention (the shard's rows of Q, the whole K and V).  The
exchange of X (or K and V) between GPUs is not part of it.  The reference
runs a graph on one GPU and has no counterpart (its ops are
``autosage/ops.py:146-164`` and ``autosage/_auto.py:544-780``).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _native
from .ops import load_native, native_load_error


def cut_rows(crow: torch.Tensor, parts: int) -> list[int]:
    """Row cut points [r_0 = 0, r_1, ..., r_parts = N] of an nnz-balanced
    split into ``parts`` shards (see the module docstring).  ``crow`` starts
    at 0 and does not decrease; it may live on any device (one host sync)."""
    if not isinstance(parts, int) or parts < 1:
        raise ValueError("parts must be a positive integer")
    if crow.dim() != 1 or crow.numel() < 1:
        raise ValueError("crow must be one-dimensional with N + 1 entries")
    if crow.dtype not in (torch.int32, torch.int64):
        raise TypeError("crow must use integer indices")
    n = crow.numel() - 1
    crow = crow.to(torch.long).contiguous()
    nnz = int(crow[-1].item())
    if parts == 1:
        return [0, n]
    # ceil(k·nnz / parts) for k = 1 .. parts - 1, in exact integer arithmetic
    targets = torch.tensor([(k * nnz + parts - 1) // parts for k in range(1, parts)], dtype=torch.long,
                           device=crow.device)
    inner = torch.searchsorted(crow, targets, right=False).clamp_(max=n)
    return [0, *(int(r) for r in inner.tolist()), n]


def shard_csr(crow: torch.Tensor, col: torch.Tensor, val: Optional[torch.Tensor], r0: int, r1: int):
    """(crow_k, col_k, val_k): the CSR of rows [r0, r1), crow rebased to 0,
    col_k and val_k views into the whole graph's arrays (no copy)."""
    n = crow.numel() - 1
    if not 0 <= r0 <= r1 <= n:
        raise ValueError(f"row range [{r0}, {r1}) is outside [0, {n}]")
    bounds = crow[[r0, r1]].tolist()
    e0, e1 = int(bounds[0]), int(bounds[1])
    crow_k = crow[r0:r1 + 1] - e0
    col_k = col[e0:e1]
    val_k = None if val is None else val[e0:e1]
    return crow_k, col_k, val_k


def spmm_csr_shard(crow: torch.Tensor, col: torch.Tensor, val: Optional[torch.Tensor], x: torch.Tensor, *,
                   exact: bool = False) -> torch.Tensor:
    """Y_k = A_k·X for a shard's CSR A_k (n_k × N, n_k = crow.numel() - 1)
    and the whole X [N, F]; Y_k is [n_k, F].

    On a GPU the native kernels run: by default the column-sliced SpMM
    (fp32 summed in fp64 per column slice and rounded once; bf16 / fp16
    rounded once), whose column slices cut the whole column space, so every
    row is summed as in the whole graph; ``exact=True`` (fp32) keeps the
    sequential fp32 order of ``spmm_csr``, bit-identical to the same rows of
    the whole graph's product.  On the CPU: ``torch.sparse.mm`` on the
    rectangular CSR tensor, the reference's CPU product
    (``autosage/ops.py:124-143``)."""
    if x.dim() != 2:
        raise ValueError("x must have shape [N, F]")
    if crow.dtype not in (torch.int32, torch.int64) or col.dtype not in (torch.int32, torch.int64):
        raise TypeError("crow and col must use integer indices")
    crow = crow.to(torch.long).contiguous()
    col = col.to(torch.long).contiguous()
    if val is not None:
        val = val.to(x.dtype).contiguous()
    if not x.is_cuda:
        n = crow.numel() - 1
        weights = val if val is not None else torch.ones(col.numel(), dtype=x.dtype)
        a = torch.sparse_csr_tensor(crow, col, weights, size=(n, x.size(0)), dtype=x.dtype)
        return torch.sparse.mm(a, x.contiguous())
    if not load_native():
        raise RuntimeError(f"AutoSAGE HIP library is not loaded: {native_load_error()}")
    if crow.device != x.device or col.device != x.device or (val is not None and val.device != x.device):
        raise ValueError("crow, col, val and x must be on the same device")
    return _native.spmm_csr_rect_impl(crow, col, val, x.contiguous(), exact=exact)


def _shard_edge_rows(crow: torch.Tensor) -> torch.Tensor:
    counts = (crow[1:] - crow[:-1]).to(torch.long)
    return torch.repeat_interleave(torch.arange(crow.numel() - 1, device=crow.device, dtype=torch.long), counts)


def sddmm_csr_shard(crow: torch.Tensor, col: torch.Tensor, query: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
    """out[e] = <query[r], key[col_e]> over a shard's edges: ``query`` holds
    the shard's rows of the whole query (n_k × F), ``key`` the whole key
    (N × F); the result is the whole graph's SDDMM output on the shard's
    edges, in CSR order.  On a GPU the native kernels (fp32 in the
    reference kernel's dot order, bf16 / fp16 rounded once); on the CPU the
    reference's gather-dot (``autosage/_auto.py:79-92``)."""
    if crow.dtype not in (torch.int32, torch.int64) or col.dtype not in (torch.int32, torch.int64):
        raise TypeError("crow and col must use integer indices")
    if query.dim() != 2 or key.dim() != 2 or query.size(1) != key.size(1):
        raise ValueError("query and key must have shapes [n_k, F] and [N, F]")
    if query.size(0) != crow.numel() - 1:
        raise ValueError("query must hold one row per row of the shard")
    crow = crow.to(torch.long).contiguous()
    col = col.to(torch.long).contiguous()
    if not query.is_cuda:
        rows = _shard_edge_rows(crow)
        return (query.index_select(0, rows) * key.index_select(0, col)).sum(dim=1)
    if not load_native():
        raise RuntimeError(f"AutoSAGE HIP library is not loaded: {native_load_error()}")
    return _native.sddmm_csr_rect_impl(crow, col, query.contiguous(), key.contiguous())


def csr_attention_shard(crow: torch.Tensor, col: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                        value: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """softmax_r(scale·<query[r], key[c]>)·value over a shard's rows:
    ``query`` holds the shard's rows (n_k × F_qk), ``key`` and ``value`` the
    whole graph's (N × F_qk, N × F_v); the result is the shard's rows of the
    attention output.  On a GPU the column-sliced attention (fp32, or bf16 /
    fp16 computed in fp32 and rounded once) with the column slices over the
    whole column space; on the CPU the reference's composition of
    gather-dot, row softmax and CSR product (``autosage/_auto.py:762-780``)."""
    if crow.dtype not in (torch.int32, torch.int64) or col.dtype not in (torch.int32, torch.int64):
        raise TypeError("crow and col must use integer indices")
    if value.dim() != 2 or value.size(0) != key.size(0):
        raise ValueError("value must have one row per row of key")
    crow = crow.to(torch.long).contiguous()
    col = col.to(torch.long).contiguous()
    if not query.is_cuda:
        scores = sddmm_csr_shard(crow, col, query * scale, key)
        rows = _shard_edge_rows(crow)
        n = crow.numel() - 1
        maxima = torch.full((n,), -torch.inf, dtype=scores.dtype)
        maxima.scatter_reduce_(0, rows, scores, reduce="amax", include_self=True)
        exps = (scores - maxima.index_select(0, rows)).exp()
        sums = torch.zeros_like(maxima).scatter_add_(0, rows, exps)
        probs = exps / sums.index_select(0, rows)
        a = torch.sparse_csr_tensor(crow, col, probs, size=(n, key.size(0)), dtype=value.dtype)
        return torch.sparse.mm(a, value.contiguous())
    if not load_native():
        raise RuntimeError(f"AutoSAGE HIP library is not loaded: {native_load_error()}")
    if query.dim() != 2 or query.size(0) != crow.numel() - 1:
        raise ValueError("query must hold one row per row of the shard")
    return _native.csr_attention_rect_impl(crow, col, query.contiguous(), key.contiguous(), value.contiguous(),
                                           scale)
