"""Backward formulas for the ``autosage::*`` SpMM and SDDMM operators.

The reference registers no autograd for its operators, so ``AutoSAGEConv``
trains only through the PyTorch baseline there.  Here the SpMM and SDDMM operators get
backward formulas built from the same native kernels:

* ``Y = A·X`` (A: CSR, weights ``val`` or ones):
  ``dX = Aᵀ·dY`` — a native SpMM over the transposed CSR — and
  ``dval[e] = <dY[row(e)], X[col(e)]>`` — a native SDDMM;
  both on the degree-split schedules (same bits as the whole-graph kernels);
  the column-sliced operators take dX on the column-sliced SpMM instead
  (same fp64-partial contract as their forward).
  With bf16 / fp16 features both come from the rounded 16-bit kernels
  (SpMM and SDDMM: fp64 sums of exact products, rounded to fp32 and then to
  the 16-bit type).
* ``s[e] = <Q[row(e)], K[col(e)]>``:
  ``dQ = A_ds·K`` (SpMM with weights ``ds``) and ``dK = A_dsᵀ·Q``.
* ``p = softmax_row(s)``: ``ds = p·(dp − Σ_row dp·p)`` (native kernel).
* the fused attention ``out = softmax_row(scale·s)·V``: the scores and
  probabilities are recomputed with the native ops and the three formulas
  above are chained (``dV = Pᵀ·dOut``); the column-sliced attention takes two
  native gather passes instead (``as_csr_attention_backward_f32`` / ``_16``:
  float32, bf16 or fp16, fp32 sums), with no nnz-sized intermediate.

The transposed CSR (rows of Aᵀ list the source rows in ascending order, a
stable sort of the edges by column) is built with torch ops and memoised per
live (crow, col) tensor pair, like the schedule keys.  Every product is
deterministic: the same inputs give the same bits.
"""

from __future__ import annotations

from typing import Optional

import torch

from ._memo import GraphMemo

# The transposed CSR of a cfg3-sized graph holds about 16·nnz bytes (1.8 GB);
# entries go when their graph's tensors die, and at most 4 GiB stay cached.
_TRANSPOSE_MEMO = GraphMemo("csr_transpose", max_entries=16, max_bytes=4 << 30)


def csr_transpose(crow: torch.Tensor, col: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(crow_t, col_t, perm) of Aᵀ for a square CSR A; ``perm[k]`` is the
    edge of A that becomes edge k of Aᵀ, so ``val_t = val[perm]``."""
    return _TRANSPOSE_MEMO.get((crow, col), None, lambda: _build_transpose(crow, col))


def _build_transpose(crow: torch.Tensor, col: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    n = crow.numel() - 1
    counts = (crow[1:] - crow[:-1]).to(torch.long)
    rows = torch.repeat_interleave(torch.arange(n, device=crow.device, dtype=torch.long), counts)
    perm = col.argsort(stable=True)
    crow_t = torch.zeros(n + 1, dtype=torch.long, device=crow.device)
    crow_t[1:] = torch.bincount(col, minlength=n).cumsum(0)
    return crow_t, rows.index_select(0, perm).contiguous(), perm


# The backward products run on the degree-split schedules when the graph has
# hub rows: bit-identical to the whole-graph kernels (the SpMM keeps CSR
# order per output, the SDDMM the reference's dot order), but hub rows are
# split across waves, which matters on skewed graphs (one wave per 200k-edge
# row is several times slower).  Without hub rows the whole-graph SpMM runs
# (memoised per-graph row count, one launch).
_HUB_THRESHOLD = 1024


def _spmm(crow, col, val, x, sliced: bool = False):
    if x.dtype != torch.float32:
        # bf16 / fp16: the rounded SpMM, the same bits on any schedule
        return torch.ops.autosage.spmm_csr(crow, col, val, x)
    if sliced and _column_slices_allowed():
        # the column-sliced operators' gradients keep their forward's contract
        # (fp64 partials, within 1e-6 of fp64); the transposed CSR lists its
        # columns in ascending order, so it needs no row-sorted copy
        return torch.ops.autosage.spmm_csr_colslice(crow, col, val, x)
    if _feature_slices_pay(crow, col, x):
        # the same bits as the schedules below, XCD-local on large graphs
        return torch.ops.autosage.spmm_csr_fslice(crow, col, val, x)
    from ._native import row_counts

    if row_counts(crow, _HUB_THRESHOLD, 0)[0] == 0:
        # no hub row: the whole-graph kernel, one launch without binning
        return torch.ops.autosage.spmm_csr(crow, col, val, x)
    tile = 64 if x.size(1) <= 64 else 128
    return torch.ops.autosage.spmm_csr_split(crow, col, val, x, tile, 2, _HUB_THRESHOLD)


def _feature_slices_pay(crow, col, x) -> bool:
    """The feature-sliced SpMM for a backward product when the forward
    scheduler would time it (``auto``: X beyond the L2s with long rows, or a
    hub row) or it is forced on."""
    from ._auto import fslice_suits
    from .config import SchedulerConfig

    return fslice_suits(crow, col, x, SchedulerConfig.from_env().feature_slices)


def _column_slices_allowed() -> bool:
    from .config import SchedulerConfig

    return SchedulerConfig.from_env().column_slices != "off"


def _sddmm(crow, col, query, key):
    return torch.ops.autosage.sddmm_csr_split(crow, col, query, key, 4, _HUB_THRESHOLD)


def _spmm_setup(ctx, inputs, output) -> None:
    crow, col, val, x = inputs[:4]
    ctx.save_for_backward(crow, col, val, x)
    ctx.has_val = val is not None
    ctx.sliced = False


def _spmm_sliced_setup(ctx, inputs, output) -> None:
    _spmm_setup(ctx, inputs, output)
    ctx.sliced = True


def _spmm_backward(ctx, grad_y: torch.Tensor):
    crow, col, val, x = ctx.saved_tensors
    if not ctx.has_val:
        val = None
    grad_x: Optional[torch.Tensor] = None
    grad_val: Optional[torch.Tensor] = None
    grad_y = grad_y.contiguous()
    if ctx.needs_input_grad[3]:
        crow_t, col_t, perm = csr_transpose(crow, col)
        val_t = None if val is None else val.index_select(0, perm).contiguous()
        grad_x = _spmm(crow_t, col_t, val_t, grad_y, ctx.sliced)
    if val is not None and ctx.needs_input_grad[2]:
        grad_val = _sddmm(crow, col, grad_y, x)
    # one gradient per schema argument (the split op has three int arguments more)
    extra = (None,) * (len(ctx.needs_input_grad) - 4)
    return (None, None, grad_val, grad_x, *extra)


def _sddmm_setup(ctx, inputs, output) -> None:
    crow, col, query, key = inputs[:4]
    ctx.save_for_backward(crow, col, query, key)


def _sddmm_backward(ctx, grad_s: torch.Tensor):
    crow, col, query, key = ctx.saved_tensors
    grad_s = grad_s.contiguous()
    grad_q = grad_k = None
    if ctx.needs_input_grad[2]:
        grad_q = _spmm(crow, col, grad_s, key)
    if ctx.needs_input_grad[3]:
        crow_t, col_t, perm = csr_transpose(crow, col)
        grad_k = _spmm(crow_t, col_t, grad_s.index_select(0, perm).contiguous(), query)
    extra = (None,) * (len(ctx.needs_input_grad) - 4)
    return (None, None, grad_q, grad_k, *extra)


def _softmax_setup(ctx, inputs, output) -> None:
    ctx.save_for_backward(inputs[0], output)


def _softmax_backward(ctx, grad_p: torch.Tensor):
    from ._native import csr_row_softmax_backward_impl

    crow, probs = ctx.saved_tensors
    return None, csr_row_softmax_backward_impl(crow, probs, grad_p.contiguous())


def _attention_setup(ctx, inputs, output) -> None:
    crow, col, query, key, value = inputs[:5]
    ctx.save_for_backward(crow, col, query, key, value, output)
    ctx.scale = float(inputs[5])
    ctx.sliced = False


def _attention_sliced_setup(ctx, inputs, output) -> None:
    _attention_setup(ctx, inputs, output)
    ctx.sliced = True


def _attention_backward(ctx, grad_out: torch.Tensor):
    """out = P·V with P = softmax_row(scale·SDDMM(Q, K)).

    The column-sliced op (column slices allowed; float32, bf16 or fp16) takes
    the two-pass native backward: pass 1 over the rows of A recomputes the
    scores with an online maximum and sum and writes dQ and the row
    log-sum-exp; pass 2 over the rows of Aᵀ writes dK and dV; t_r =
    <dOut[r], out[r]> comes from the saved output (float32) or is summed in
    pass 1 (16-bit, whose output is rounded).  Otherwise (the exact fused op,
    column slices off) the scores and P are recomputed with the native ops, then
    dV = Pᵀ·dOut, dP[e] = <dOut[row(e)], V[col(e)]>, dS = softmax'(P, dP)·scale,
    dQ = A_dS·K, dK = A_dSᵀ·Q (native SpMM / SDDMM / softmax backward)."""
    from ._native import (
        attention_backward_supported,
        csr_attention_backward_impl,
        csr_row_softmax_backward_impl,
        row_sorted,
    )

    crow, col, query, key, value, out = ctx.saved_tensors
    grad_out = grad_out.contiguous()
    if ctx.sliced and _column_slices_allowed() and attention_backward_supported(query, key, value, out, grad_out):
        # the column-sliced op: two gather passes (over A, then over Aᵀ) with
        # the row log-sum-exp of the first feeding the second; no scores,
        # probabilities or their gradients in memory
        col_s = row_sorted(crow, col)[0]
        crow_t, col_t, _ = csr_transpose(crow, col_s)
        grad_q, grad_k, grad_v = csr_attention_backward_impl(crow, col_s, crow_t, col_t, query, key, value, out,
                                                             grad_out, ctx.scale)
        needs = ctx.needs_input_grad
        return (None, None, grad_q if needs[2] else None, grad_k if needs[3] else None,
                grad_v if needs[4] else None, None)
    scores = _sddmm(crow, col, query, key)
    if ctx.scale != 1.0:
        scores = scores * ctx.scale
    probs = torch.ops.autosage.csr_row_softmax(crow, scores)
    grad_q = grad_k = grad_v = None
    crow_t, col_t, perm = csr_transpose(crow, col)
    if ctx.needs_input_grad[4]:
        grad_v = _spmm(crow_t, col_t, probs.index_select(0, perm).contiguous(), grad_out, ctx.sliced)
    if ctx.needs_input_grad[2] or ctx.needs_input_grad[3]:
        grad_s = csr_row_softmax_backward_impl(crow, probs, _sddmm(crow, col, grad_out, value))
        if ctx.scale != 1.0:
            grad_s = grad_s * ctx.scale
        if ctx.needs_input_grad[2]:
            grad_q = _spmm(crow, col, grad_s, key, ctx.sliced)
        if ctx.needs_input_grad[3]:
            grad_k = _spmm(crow_t, col_t, grad_s.index_select(0, perm).contiguous(), query, ctx.sliced)
    return None, None, grad_q, grad_k, grad_v, None


def register() -> None:
    """Attaches the backward formulas to the registered operators."""
    for name in ("spmm_csr", "spmm_csr_split", "spmm_csr_fslice"):
        torch.library.register_autograd(f"autosage::{name}", _spmm_backward, setup_context=_spmm_setup)
    torch.library.register_autograd("autosage::spmm_csr_colslice", _spmm_backward, setup_context=_spmm_sliced_setup)
    for name in ("sddmm_csr", "sddmm_csr_split"):
        torch.library.register_autograd(f"autosage::{name}", _sddmm_backward, setup_context=_sddmm_setup)
    torch.library.register_autograd("autosage::csr_row_softmax", _softmax_backward, setup_context=_softmax_setup)
    torch.library.register_autograd("autosage::csr_attention", _attention_backward, setup_context=_attention_setup)
    torch.library.register_autograd(
        "autosage::csr_attention_colslice", _attention_backward, setup_context=_attention_sliced_setup
    )
