"""CPU oracle for the sparse hot path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for
``cpu_baseline``, as the timed CPU reference path).  The product package
``autosage_amd`` never imports it and has no CPU fallback.

Contents:
* ``csr_oracle.c`` (ctypes, built by ``oracle/build.py``): sequential-fmaf
  SpMM, fp64 SpMM, degree binning, SDDMM in the reference kernel order, fp64
  SDDMM, row softmax in fp32 and fp64 — each citing the reference lines it
  restates;
* torch CPU restatements of the reference's own CPU/baseline compositions:
  ``torch_cpu_spmm`` (autosage/ops.py:124-143), ``torch_gather_dot``
  (autosage/_auto.py:79-92), ``torch_row_softmax`` (autosage/_auto.py:744-759),
  ``numpy_edge_index_to_csr`` (autosage/utils/csr.py:6-26);
* ``attention_ref`` = composition of the above (autosage/_auto.py:762-780);
* ``spmm_rounded_16`` / ``sddmm_rounded_16``: the bf16 / fp16 SpMM and
  SDDMM rule (fp64 sum of exact products, rounded to fp32, then to the 16-bit
  type); ``row_softmax_rounded_16``: the fp32 row softmax of 16-bit scores,
  rounded once (a composition of or_row_softmax_f32 and torch's rounding,
  pinned through them).

How each function is pinned (independent checks in tests/test_oracle.py):
* or_spmm_seq_f32: bit-identical to torch.sparse.mm on CPU (MKL) on random
  weighted/unweighted graphs; fp64 bound; reference KATs (tests/test_cpu.py
  of the reference, lines 16-32, 70-78).
* or_spmm_f64: brute-force dense A @ X in float64 on tiny graphs.
* or_bin_rows: numpy flatnonzero restatement + hand-built KAT.
* or_sddmm_ref_f32: KAT [4, 7, 10] (reference test_cpu.py:45-53), fp64
  bound, torch gather-dot within tolerance, and a tree-order check where the
  reference order and sequential order give different bits.
* or_row_softmax_backward_f32: a Python restatement of the lane order on
  values whose products and sums are exact in fp64 (so every fmaf is one
  rounding), with a row where that order and a sequential sum differ; fp64
  closed forms (uniform probabilities with constant grad -> 0, one-entry rows
  -> 0, torch autograd of the fp64 softmax within 1e-6).
* or_row_softmax_f32: KAT (rows sum to 1, single-entry rows = 1.0), torch
  scatter composition within 1e-6 relative, fp64 bound.
* or_attention_f64: a dense brute force (masked fp64 softmax of Q·Kᵀ·scale
  times V) on small graphs, and closed forms (zero scores give the mean of
  the row's V rows; a one-edge row returns that V row).
* spmm_rounded_16: exact rational sums (fractions.Fraction) rounded the same
  way on random graphs; hand-computed ties (round to even, and the fp32 step
  that decides a tie the exact sum would not), fp16 overflow to inf.
* sddmm_rounded_16: exact rational dot products (fractions.Fraction) on
  random graphs; hand-computed cases: a product that rounding to the 16-bit
  type first would change (1 + 2^-7)(1 + 2^-5) - 1, a tie decided to even,
  fp16 overflow to inf.  (or_sddmm_f64 itself is pinned by a dense
  brute-force product.)
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"

_lib: Optional[ctypes.CDLL] = None


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            from .build import build

            build()
        lib = ctypes.CDLL(str(LIBRARY))
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.or_spmm_seq_f32.argtypes = [p, p, p, p, p, i64, i64, p]
        lib.or_spmm_f64.argtypes = [p, p, p, p, p, i64, i64, p]
        lib.or_bin_rows.argtypes = [p, i64, i64, p, p, p]
        lib.or_sddmm_ref_f32.argtypes = [p, p, p, p, i64, i64, p]
        lib.or_sddmm_f64.argtypes = [p, p, p, p, i64, i64, p]
        lib.or_row_softmax_f32.argtypes = [p, p, i64, p]
        lib.or_row_softmax_f64.argtypes = [p, p, i64, p]
        lib.or_row_softmax_backward_f32.argtypes = [p, p, p, i64, p]
        lib.or_attention_f64.argtypes = [p, p, p, p, p, i64, i64, i64, ctypes.c_double, p]
        for name in ("or_spmm_seq_f32", "or_spmm_f64", "or_bin_rows", "or_sddmm_ref_f32", "or_sddmm_f64",
                     "or_row_softmax_f32", "or_row_softmax_f64", "or_row_softmax_backward_f32", "or_attention_f64"):
            getattr(lib, name).restype = None
        _lib = lib
    return _lib


def _np(a, dtype) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def spmm_seq(crow, col, val, x, rows=None) -> np.ndarray:
    """fp32 sequential-fmaf SpMM; ``rows`` selects output rows (default all)."""
    crow, col, x = _np(crow, np.int64), _np(col, np.int64), _np(x, np.float32)
    val = None if val is None else _np(val, np.float32)
    f = x.shape[1]
    rows_a = None if rows is None else _np(rows, np.int64)
    nrows = crow.size - 1 if rows_a is None else rows_a.size
    y = np.empty((nrows, f), dtype=np.float32)
    _load().or_spmm_seq_f32(_p(crow), _p(col), _p(val), _p(x), _p(rows_a), nrows, f, _p(y))
    return y


def spmm_f64(crow, col, val, x, rows=None) -> np.ndarray:
    crow, col, x = _np(crow, np.int64), _np(col, np.int64), _np(x, np.float32)
    val = None if val is None else _np(val, np.float32)
    f = x.shape[1]
    rows_a = None if rows is None else _np(rows, np.int64)
    nrows = crow.size - 1 if rows_a is None else rows_a.size
    y = np.empty((nrows, f), dtype=np.float64)
    _load().or_spmm_f64(_p(crow), _p(col), _p(val), _p(x), _p(rows_a), nrows, f, _p(y))
    return y


def spmm_rounded_16(crow, col, val, x, dtype: torch.dtype, rows=None) -> torch.Tensor:
    """SpMM on bf16 / fp16 features, the rule of as_spmm_csr_rounded_16 (the
    reference has no kernel for these types, autosage/ops.py:156-157, and no
    CPU path: torch's CPU CSR product rejects them): weights cast to ``dtype``
    (as the reference's torch path does, autosage/_auto.py:68-76), the exact
    products summed in fp64, the sum rounded to fp32 and then to ``dtype``,
    round to nearest even both times.  ``x`` / ``val``: tensors of ``dtype``
    or arrays of values it represents exactly."""
    xt = torch.as_tensor(x).to(dtype)
    x32 = xt.float().numpy()
    v32 = None if val is None else torch.as_tensor(val).to(dtype).float().numpy()
    y64 = spmm_f64(crow, col, v32, x32, rows=rows)
    return torch.from_numpy(y64).to(torch.float32).to(dtype)


def bin_rows(crow, threshold: int) -> tuple[np.ndarray, np.ndarray]:
    crow = _np(crow, np.int64)
    n = crow.size - 1
    heavy = np.empty(max(n, 1), dtype=np.int32)
    light = np.empty(max(n, 1), dtype=np.int32)
    counts = np.zeros(2, dtype=np.int64)
    _load().or_bin_rows(_p(crow), n, int(threshold), _p(heavy), _p(light), _p(counts))
    return heavy[: counts[0]].copy(), light[: counts[1]].copy()


def sddmm_ref(crow, col, query, key) -> np.ndarray:
    crow, col = _np(crow, np.int64), _np(col, np.int64)
    q, k = _np(query, np.float32), _np(key, np.float32)
    out = np.empty(col.size, dtype=np.float32)
    _load().or_sddmm_ref_f32(_p(crow), _p(col), _p(q), _p(k), crow.size - 1, q.shape[1], _p(out))
    return out


def sddmm_f64(crow, col, query, key) -> np.ndarray:
    crow, col = _np(crow, np.int64), _np(col, np.int64)
    q, k = _np(query, np.float32), _np(key, np.float32)
    out = np.empty(col.size, dtype=np.float64)
    _load().or_sddmm_f64(_p(crow), _p(col), _p(q), _p(k), crow.size - 1, q.shape[1], _p(out))
    return out


def sddmm_rounded_16(crow, col, query, key, dtype: torch.dtype) -> torch.Tensor:
    """SDDMM on bf16 / fp16 query and key, the rule of as_sddmm_csr_rounded_16
    (the reference's op takes float32 only, csrc/sddmm_csr_op.cu:94-95, and
    its scheduler runs the gather-dot baseline for other types,
    autosage/_auto.py:575-581): the exact products summed in fp64 (in feature
    order), the sum rounded to fp32 and then to ``dtype``, round to nearest
    even both times."""
    q32 = torch.as_tensor(query).to(dtype).float().numpy()
    k32 = torch.as_tensor(key).to(dtype).float().numpy()
    out64 = sddmm_f64(crow, col, q32, k32)
    return torch.from_numpy(out64).to(torch.float32).to(dtype)


def row_softmax(crow, scores) -> np.ndarray:
    crow, s = _np(crow, np.int64), _np(scores, np.float32)
    out = np.zeros_like(s)
    _load().or_row_softmax_f32(_p(crow), _p(s), crow.size - 1, _p(out))
    return out


def row_softmax_backward(crow, probs, grad) -> np.ndarray:
    """dL/dscores of the row softmax from its output and dL/dprobs, fp32 in
    the GPU kernel's order (64 lane partials of grad·p, butterfly)."""
    crow = _np(crow, np.int64)
    p, g = _np(probs, np.float32), _np(grad, np.float32)
    out = np.zeros(p.size, dtype=np.float32)
    _load().or_row_softmax_backward_f32(_p(crow), _p(p), _p(g), crow.size - 1, _p(out))
    return out


def row_softmax_backward_rounded_16(crow, probs, grad, dtype: torch.dtype) -> torch.Tensor:
    """The same on 16-bit values: exact conversions to fp32, each result
    rounded once to ``dtype``."""
    p32 = torch.as_tensor(probs).to(dtype).float().numpy()
    g32 = torch.as_tensor(grad).to(dtype).float().numpy()
    return torch.from_numpy(row_softmax_backward(crow, p32, g32)).to(dtype)


def row_softmax_rounded_16(crow, scores, dtype: torch.dtype) -> torch.Tensor:
    """The row softmax of 16-bit scores as as_csr_row_softmax_16 defines it:
    the fp32 softmax (``row_softmax``) of the exactly converted scores, each
    probability rounded once to ``dtype``."""
    s32 = torch.as_tensor(scores).to(dtype).float().numpy()
    return torch.from_numpy(row_softmax(crow, s32)).to(dtype)


def row_softmax_f64(crow, scores) -> np.ndarray:
    crow, s = _np(crow, np.int64), _np(scores, np.float64)
    out = np.zeros_like(s)
    _load().or_row_softmax_f64(_p(crow), _p(s), crow.size - 1, _p(out))
    return out


def attention_ref(crow, col, query, key, value, scale: float = 1.0) -> np.ndarray:
    """scores = SDDMM (reference order) · scale -> row softmax -> sequential SpMM."""
    scores = sddmm_ref(crow, col, query, key) * np.float32(scale)
    probs = row_softmax(crow, scores)
    return spmm_seq(crow, col, probs, value)


def attention_f64(crow, col, query, key, value, scale: float = 1.0) -> np.ndarray:
    """CSR attention in fp64 (``or_attention_f64``): scaled fp64 dot products,
    fp64 row softmax, fp64 weighted sums of V rows in CSR order."""
    crow_a, col_a = _np(crow, np.int64), _np(col, np.int64)
    q, k, v = _np(query, np.float32), _np(key, np.float32), _np(value, np.float32)
    n = crow_a.size - 1
    out = np.empty((n, v.shape[1]), dtype=np.float64)
    _load().or_attention_f64(_p(crow_a), _p(col_a), _p(q), _p(k), _p(v), n, q.shape[1], v.shape[1],
                             float(scale), _p(out))
    return out


# --- torch CPU restatements of the reference compositions -------------------


def torch_cpu_spmm(crow, col, val, x) -> torch.Tensor:
    """The reference CPU SpMM path (autosage/ops.py:124-143)."""
    n = x.size(0)
    weights = torch.ones(col.numel(), dtype=x.dtype) if val is None else val.to(x.dtype)
    matrix = torch.sparse_csr_tensor(crow, col, weights, size=(n, n), dtype=x.dtype)
    return torch.sparse.mm(matrix, x)


def torch_gather_dot(crow, col, query, key) -> torch.Tensor:
    """The reference SDDMM baseline (autosage/_auto.py:79-92)."""
    counts = (crow[1:] - crow[:-1]).to(torch.long)
    rows = torch.repeat_interleave(torch.arange(crow.numel() - 1, dtype=torch.long), counts)
    return (query.index_select(0, rows) * key.index_select(0, col)).sum(dim=1)


def torch_row_softmax(crow, scores) -> torch.Tensor:
    """The reference row softmax composition (autosage/_auto.py:744-759)."""
    counts = (crow[1:] - crow[:-1]).to(torch.long)
    rows = torch.repeat_interleave(torch.arange(crow.numel() - 1, dtype=torch.long), counts)
    if scores.numel() == 0:
        return scores.clone()
    maxima = torch.full((crow.numel() - 1,), -torch.inf, dtype=scores.dtype)
    maxima.scatter_reduce_(0, rows, scores, reduce="amax", include_self=True)
    exps = (scores - maxima.index_select(0, rows)).exp()
    sums = torch.zeros_like(maxima)
    sums.scatter_add_(0, rows, exps)
    return exps / sums.index_select(0, rows)


def numpy_edge_index_to_csr(edge_index: np.ndarray, num_nodes: int) -> tuple[np.ndarray, np.ndarray]:
    """Destination-row CSR by stable sort (autosage/utils/csr.py:6-26)."""
    src = np.asarray(edge_index[0], dtype=np.int64)
    dst = np.asarray(edge_index[1], dtype=np.int64)
    order = np.argsort(dst, kind="stable")
    crow = np.zeros(num_nodes + 1, dtype=np.int64)
    np.add.at(crow, dst + 1, 1)
    return np.cumsum(crow), src[order]
