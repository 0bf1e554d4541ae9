"""Operator front-end: input normalisation, the CPU path and the native loader.

Mirrors ``autosage/ops.py`` of the reference: the same public functions
(``spmm_csr``, ``load_native``, ``native_available``, ``native_op``,
``native_load_error``), the same validation messages and exception types
(``ops.py:82-121``), the CPU path through ``torch.sparse.mm`` on a CSR tensor
(``ops.py:124-143``) and the GPU path through ``torch.ops.autosage.spmm_csr``
(``ops.py:146-164``).  The native library is the gfx950 HIP build
``libautosage_hip.so`` instead of ``libautosage_cuda.so``; there is no silent
fallback: a GPU call without the library raises ``RuntimeError``.
"""

from __future__ import annotations

import os
from pathlib import Path
from typing import Optional

import torch

from . import _env
from . import _native

_LOAD_ATTEMPTED = False
_LOAD_ERROR: Optional[BaseException] = None


def _candidate_libraries() -> list[Path]:
    """Search order of ``ops.py:14-28``: explicit path, then ``build/`` at the
    repository root, then the package's ``lib/``."""
    found: list[Path] = []
    explicit = os.getenv("AUTOSAGE_NATIVE_PATH")
    if explicit:
        found.append(Path(explicit).expanduser())
    package = Path(__file__).resolve().parent
    for directory in (package.parent / "build", package / "lib"):
        found.append(directory / _native.LIBRARY_NAME)
    return found


def load_native() -> bool:
    """Loads the HIP library once per process (``ops.py:31-61``)."""
    global _LOAD_ATTEMPTED, _LOAD_ERROR
    if native_available():
        return True
    if _LOAD_ATTEMPTED:
        return False
    _LOAD_ATTEMPTED = True
    failures: list[BaseException] = []
    for candidate in _candidate_libraries():
        if not candidate.is_file():
            continue
        try:
            _native.load(candidate)
            return native_available()
        except (OSError, RuntimeError, AttributeError) as exc:
            failures.append(exc)
    _LOAD_ERROR = (
        failures[-1]
        if failures
        else FileNotFoundError(
            "AutoSAGE native library was not found. Build it with python -m autosage_amd._build."
        )
    )
    return False


def native_op(name: str):
    namespace = getattr(torch.ops, "autosage", None)
    if namespace is None:
        return None
    try:
        return getattr(namespace, name)
    except (AttributeError, RuntimeError):
        return None


def native_available() -> bool:
    return native_op("spmm_csr") is not None


def native_load_error() -> Optional[BaseException]:
    return _LOAD_ERROR


def _validate_csr(crow, col, val, x) -> None:
    if crow.ndim != 1 or col.ndim != 1:
        raise ValueError("crow and col must be one-dimensional")
    if crow.dtype != torch.long or col.dtype != torch.long:
        raise TypeError("crow and col must use torch.long indices")
    if x.ndim != 2:
        raise ValueError("x must have shape [N, F]")
    if not x.is_floating_point():
        raise TypeError("x must use a floating-point dtype")
    if crow.numel() != x.size(0) + 1:
        raise ValueError("crow must contain N + 1 entries")
    if val is not None and (val.ndim != 1 or val.numel() != col.numel()):
        raise ValueError("val must contain one weight per nonzero")
    if not (crow.device == col.device == x.device):
        raise ValueError("crow, col, and x must be on the same device")
    if val is not None and val.device != x.device:
        raise ValueError("val and x must be on the same device")


def _normalize_csr(crow, col, val, x):
    """Promotes int32/int64 indices to contiguous int64, makes ``x``
    contiguous, casts ``val`` to ``x.dtype`` and validates (``ops.py:106-121``)."""
    if crow.dtype not in (torch.int32, torch.int64) or col.dtype not in (torch.int32, torch.int64):
        raise TypeError("crow and col must use integer indices")
    # tensors already in shape are passed through as they are (no new tensor)
    if crow.dtype != torch.long or not crow.is_contiguous():
        crow = crow.to(dtype=torch.long).contiguous()
    if col.dtype != torch.long or not col.is_contiguous():
        col = col.to(dtype=torch.long).contiguous()
    if not x.is_contiguous():
        x = x.contiguous()
    if val is not None and (val.dtype != x.dtype or not val.is_contiguous()):
        val = val.to(dtype=x.dtype).contiguous()
    _validate_csr(crow, col, val, x)
    validate_if_requested(crow, col)
    return crow, col, val, x


def validate_if_requested(crow, col) -> None:
    """Runs ``validate_csr`` on CUDA graphs when ``AUTOSAGE_VALIDATE=1``,
    before any baseline or native gather touches them."""
    if _env.get("AUTOSAGE_VALIDATE") == "1" and crow.is_cuda:
        validate_csr(crow, col)


def _cpu_spmm(crow, col, val, x) -> torch.Tensor:
    """The reference CPU path: ``torch.sparse.mm`` on an N×N CSR tensor with
    unit values when unweighted (``ops.py:124-143``)."""
    weights = torch.ones(col.numel(), dtype=x.dtype, device=x.device) if val is None else val.to(x.dtype)
    n = x.size(0)
    matrix = torch.sparse_csr_tensor(crow, col, weights, size=(n, n), dtype=x.dtype, device=x.device)
    return torch.sparse.mm(matrix, x)


def spmm_csr(crow, col, val, x) -> torch.Tensor:
    crow, col, val, x = _normalize_csr(crow, col, val, x)
    if not x.is_cuda:
        return _cpu_spmm(crow, col, val, x)
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError("AutoSAGE CUDA kernels currently support float32 features only (and bf16/fp16 for SpMM)")
    if not load_native():
        detail = f": {_LOAD_ERROR}" if _LOAD_ERROR else ""
        raise RuntimeError(f"AutoSAGE CUDA extension is unavailable{detail}")
    op = native_op("spmm_csr")
    if op is None:
        raise RuntimeError("native operator autosage::spmm_csr is not registered")
    return op(crow, col, val, x)


def validate_csr(crow, col, n_cols: Optional[int] = None) -> None:
    """Checks a CUDA CSR graph with one native pass: ``crow[0] == 0``,
    ``crow`` non-decreasing, ``crow[-1] == col.numel()`` and every column in
    ``[0, n_cols)`` (``n_cols`` defaults to N, the square graphs of the
    operators).  Raises ``ValueError`` naming each violated rule.  The
    operators themselves run it first when ``AUTOSAGE_VALIDATE=1``."""
    if crow.dtype not in (torch.int32, torch.int64) or col.dtype not in (torch.int32, torch.int64):
        raise TypeError("crow and col must use integer indices")
    if crow.ndim != 1 or col.ndim != 1:
        raise ValueError("crow and col must be one-dimensional")
    if not (crow.is_cuda and col.is_cuda):
        raise ValueError("validate_csr checks CUDA tensors")
    if not load_native():
        detail = f": {_LOAD_ERROR}" if _LOAD_ERROR else ""
        raise RuntimeError(f"AutoSAGE CUDA extension is unavailable{detail}")
    _native.validate_csr(crow.to(torch.long), col.to(torch.long), n_cols)


def spmm_csr_auto(*args, **kwargs):
    from ._auto import spmm_csr_auto as implementation

    return implementation(*args, **kwargs)


__all__ = [
    "load_native",
    "native_available",
    "native_load_error",
    "native_op",
    "spmm_csr",
    "spmm_csr_auto",
    "validate_csr",
]
