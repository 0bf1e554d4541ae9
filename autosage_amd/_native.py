"""ctypes binding of ``libautosage_hip.so`` and the ``autosage::*`` operators.

The reference registers its CUDA kernels as torch operators from C++
(``csrc/spmm_binding.cpp:65-75``, ``csrc/sddmm_csr_op.cu:191-201``).  Here the
kernels live behind the plain C ABI of ``include/autosage_hip.h`` and this
module registers the same operator schemas under the same ``autosage``
namespace with ``torch.library``, implemented for the CUDA dispatch key (HIP
devices on PyTorch-ROCm).  Callers that use ``torch.ops.autosage.spmm_csr``,
``spmm_csr_split``, ``sddmm_csr`` or ``sddmm_csr_split`` keep working.  Two
operators are new: ``csr_row_softmax`` and ``csr_attention``.

Input checks and their messages follow ``check_inputs``
(``csrc/spmm_binding.cpp:9-29``) and ``check_sddmm_inputs``
(``csrc/sddmm_csr_op.cu:85-106``); a failing check raises ``RuntimeError``
as ``TORCH_CHECK`` does.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

from . import _env
from ._memo import GraphMemo

LIBRARY_NAME = "libautosage_hip.so"
ABI_VERSION = 9
HUB_EXACT = 0
HUB_SPLIT64 = 1
# 16-bit feature types of as_spmm_csr_rounded_16 (AS_DTYPE_BF16 / AS_DTYPE_F16)
DTYPES_16 = {torch.bfloat16: 1, torch.float16: 2}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_ptr = ctypes.c_void_p
_c_size = ctypes.c_size_t

_SIGNATURES = {
    "as_last_error": (ctypes.c_char_p, []),
    "as_abi_version": (_c_int, []),
    "as_spmm_csr_f32": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr]),
    "as_bin_workspace_bytes": (_c_size, [_c_i64]),
    "as_bin_rows_by_degree": (_c_int, [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "as_spmm_split_workspace_bytes": (_c_size, [_c_i64]),
    "as_spmm_csr_split_f32": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_i64, _c_int, _c_int,
         _c_ptr, _c_size, _c_ptr],
    ),
    "as_spmm_fslice_plan_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "as_spmm_fslice_plan_workspace_bytes": (_c_size, [_c_i64]),
    "as_spmm_fslice_plan": (
        _c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_size, _c_ptr, _c_size,
         ctypes.POINTER(ctypes.c_int64), _c_ptr],
    ),
    "as_spmm_fslice_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "as_spmm_csr_fslice_f32": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_size, _c_i64, _c_ptr, _c_size,
         _c_ptr],
    ),
    "as_spmm_fslice_relayout_f32": (_c_int, [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_size, _c_ptr]),
    "as_spmm_csr_fslice_sliced_f32": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_size, _c_i64, _c_ptr],
    ),
    "as_spmm_csr_split_f32_static": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_i64, _c_int, _c_int,
         _c_ptr],
    ),
    "as_sddmm_csr_f32": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr]),
    "as_sddmm_split_workspace_bytes": (_c_size, [_c_i64]),
    "as_sddmm_csr_split_f32": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_i64, _c_ptr, _c_size, _c_ptr],
    ),
    "as_csr_row_softmax_f32": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr]),
    "as_spmm_colslice_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "as_spmm_csr_colslice_f32": (
        _c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_size, _c_i64, _c_ptr]
    ),
    "as_spmm_colslice_min_degree": (_c_i64, [_c_int, _c_i64, _c_int]),
    "as_spmm_colslice_plan_bytes": (_c_size, [_c_i64]),
    "as_spmm_colslice_plan": (
        _c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr, _c_size, ctypes.POINTER(ctypes.c_int64),
         _c_ptr],
    ),
    "as_spmm_colslice_plan_rect": (
        _c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr, _c_size,
         ctypes.POINTER(ctypes.c_int64), _c_ptr],
    ),
    "as_spmm_csr_colslice_planned_rect": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr, _c_size,
         _c_i64, _c_ptr, _c_size, _c_i64, _c_i64, _c_ptr],
    ),
    "as_spmm_colslice_planned_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int, _c_i64]),
    "as_spmm_colslice_row_blocks": (_c_i64, [_c_i64, _c_int, ctypes.POINTER(ctypes.c_int64), _c_i64]),
    "as_spmm_csr_colslice_planned": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr, _c_size, _c_i64,
         _c_ptr, _c_size, _c_i64, _c_i64, _c_ptr],
    ),
    "as_spmm_csr_rounded_16": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr, _c_size, _c_i64,
         _c_i64, _c_ptr],
    ),
    "as_spmm_rounded_16_group_degree": (_c_i64, [_c_i64]),
    "as_spmm_colslice_group_degree": (_c_i64, [_c_i64, _c_int]),
    "as_spmm_rounded_16_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "as_spmm_csr_rows_16": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr]),
    "as_csr_row_softmax_16": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_int, _c_ptr]),
    "as_csr_row_softmax_backward": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_int, _c_ptr]),
    "as_sddmm_csr_rounded_16": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_i64, _c_ptr, _c_size,
         _c_ptr],
    ),
    "as_sddmm_edges_16_workspace_bytes": (_c_size, [_c_i64]),
    "as_sddmm_csr_edges_16_rect": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_size, _c_ptr],
    ),
    "as_csr_attention_plan_rect": (
        _c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_size, ctypes.POINTER(ctypes.c_int64), _c_ptr],
    ),
    "as_sddmm_csr_edges_16": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_size, _c_ptr],
    ),
    "as_csr_attention_colslice_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "as_csr_attention_plan_bytes": (_c_size, [_c_i64]),
    "as_csr_attention_plan": (
        _c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_int, _c_ptr, _c_size, ctypes.POINTER(ctypes.c_int64), _c_ptr]
    ),
    "as_csr_attention_colslice_f32": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_ptr,
         _c_i64, _c_ptr, _c_size, _c_ptr],
    ),
    "as_csr_attention_colslice_16": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_int,
         _c_ptr, _c_i64, _c_ptr, _c_size, _c_ptr],
    ),
    "as_csr_attention_backward_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "as_csr_attention_backward_f32": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64,
         _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_size, _c_ptr],
    ),
    "as_csr_attention_backward_16": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64,
         _c_i64, _c_i64, ctypes.c_float, _c_int, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_size, _c_ptr],
    ),
    "as_csr_validate": (_c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr]),
    "as_induced_sample_workspace_bytes": (_c_size, [_c_i64]),
    "as_induced_sample_count": (_c_int, [_c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "as_induced_sample_fill": (
        _c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr]
    ),
    "as_csr_attention_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "as_csr_attention_f32": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_ptr,
         _c_size, _c_ptr],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_LIB: Optional[ctypes.CDLL] = None
_LIB_PATH: Optional[Path] = None
_OPS_LIBRARY: Optional[torch.library.Library] = None


def package_library_path() -> Path:
    return Path(__file__).resolve().parent / "lib" / LIBRARY_NAME


def open_library(path: os.PathLike[str] | str) -> ctypes.CDLL:
    """dlopens the C-ABI library and declares every exported signature.

    torch is imported first so that its HIP runtime is the one the library
    binds to (both use the soname ``libamdhip64.so.7``)."""
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.as_abi_version()
    if version != ABI_VERSION:
        raise OSError(f"{path}: ABI version {version}, expected {ABI_VERSION}")
    return lib


def library() -> ctypes.CDLL:
    if _LIB is None:
        raise RuntimeError("AutoSAGE HIP library is not loaded")
    return _LIB


def loaded_path() -> Optional[Path]:
    return _LIB_PATH


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


_NO_GUARD = contextlib.nullcontext()


def _on(device: torch.device):
    """``torch.cuda.device(device)``, or nothing when that device is already
    the current one (the common case; entering the guard costs microseconds
    on every call)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NO_GUARD
    return torch.cuda.device(device)


# torch's accessor of a device's current stream as a raw handle (what
# torch.cuda.current_stream(device).cuda_stream returns, without building a
# Stream object: ~0.3 against ~4.5 us a call)
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    if _RAW_STREAM is not None:
        index = device.index
        return _RAW_STREAM(torch.cuda.current_device() if index is None else index)
    return torch.cuda.current_stream(device).cuda_stream


def _raise(status: int, what: str) -> None:
    if status != 0:
        message = library().as_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{what}: {message} (status {status})")


def _env_vec4() -> bool:
    value = _env.get("AUTOSAGE_VEC4")
    if value is None:
        return True
    return value.strip().lower() not in {"0", "false", "no", "off"}


def _env_hub_mode() -> int:
    value = (_env.get("AUTOSAGE_HUB_MODE") or "exact").strip().lower()
    if value in {"exact", "0"}:
        return HUB_EXACT
    if value in {"split64", "1"}:
        return HUB_SPLIT64
    raise ValueError("AUTOSAGE_HUB_MODE must be 'exact' or 'split64'")


def _check(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def check_spmm_inputs(crow, col, val, x, allow_16: bool = False, rect: bool = False) -> None:
    """Raises ``RuntimeError`` unless the inputs suit the native SpMM.
    ``rect``: crow may have any number of rows (a row shard against the
    whole X), else it has x.size(0) + 1 entries."""
    # every condition at once (device indices as ints, no device objects);
    # on a failure the checks below name the first one that fails
    xd = x.dtype
    if (crow.is_cuda and col.is_cuda and x.is_cuda and crow.dtype is torch.long and col.dtype is torch.long
            and crow.dim() == 1 and col.dim() == 1 and x.dim() == 2 and x.is_contiguous()
            and crow.is_contiguous() and col.is_contiguous()
            and crow.get_device() == x.get_device() == col.get_device()
            and (crow.numel() == x.size(0) + 1 or (rect and crow.numel() >= 1))
            and (xd is torch.float32 or (allow_16 and xd in DTYPES_16))
            and (val is None or (val.is_cuda and val.get_device() == x.get_device() and val.dtype is xd
                                 and val.is_contiguous() and val.numel() == col.numel()))):
        return
    _check(crow.is_cuda and col.is_cuda and x.is_cuda, "crow, col, and x must be CUDA tensors")
    _check(crow.dtype == torch.long and col.dtype == torch.long, "crow and col must use torch.long indices")
    _check(crow.dim() == 1 and col.dim() == 1, "crow and col must be one-dimensional")
    _check(x.dim() == 2 and x.is_contiguous(), "x must be contiguous with shape [N, F]")
    _check(crow.is_contiguous() and col.is_contiguous(), "crow and col must be contiguous")
    _check(crow.device == x.device and col.device == x.device, "crow, col, and x must be on the same CUDA device")
    if rect:
        _check(crow.numel() >= 1, "crow must contain at least one entry")
    else:
        _check(crow.numel() == x.size(0) + 1, "crow must contain N + 1 entries")
    if allow_16:
        _check(x.dtype == torch.float32 or x.dtype in DTYPES_16, "x must be float32, bfloat16 or float16")
    else:
        _check(x.dtype == torch.float32, "x must be float32")
    if val is not None:
        _check(val.is_cuda and val.device == x.device, "val must be on the same CUDA device as x")
        _check(val.dtype == x.dtype and val.is_contiguous(), "val must be contiguous and of x's dtype")
        _check(val.numel() == col.numel(), "val must contain one weight per nonzero")


def check_sddmm_inputs(crow, col, query, key, allow_16: bool = False) -> None:
    _check(crow.is_cuda and col.is_cuda and query.is_cuda and key.is_cuda, "all SDDMM inputs must be CUDA tensors")
    _check(crow.dtype == torch.long and col.dtype == torch.long, "crow and col must use torch.long indices")
    if allow_16 and query.dtype in DTYPES_16:
        _check(key.dtype == query.dtype, "query and key must use the same dtype")
    else:
        _check(query.dtype == torch.float32 and key.dtype == torch.float32, "query and key must be float32")
    _check(query.dim() == 2 and query.shape == key.shape, "query and key must have the same [N, F] shape")
    _check(crow.numel() == query.size(0) + 1, "crow must contain N + 1 entries")
    _check(
        crow.device == query.device and col.device == query.device and key.device == query.device,
        "all SDDMM inputs must be on the same CUDA device",
    )
    _check(
        crow.is_contiguous() and col.is_contiguous() and query.is_contiguous() and key.is_contiguous(),
        "all SDDMM inputs must be contiguous",
    )
    _check(query.size(0) <= 2**31 - 1 and query.size(1) <= 2**31 - 1, "SDDMM dimensions exceed the kernel index range")


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# Operator implementations (CUDA dispatch key)


def spmm_csr_impl(crow, col, val, x):
    check_spmm_inputs(crow, col, val, x, allow_16=True)
    _maybe_validate(crow, col)
    if x.dtype in DTYPES_16:
        # the same bits on every schedule: rows whole on small graphs and on
        # graphs without a row to slice (one launch), else edge slices (any
        # column order; column slices, which need ascending columns, are
        # within 1-5 % of them on the skewed graph at F >= 128 and slower at
        # F = 64; spmm_csr_auto times both)
        if col.numel() <= ROWS_16_MAX_NNZ or sliced_rows(crow, False, x.size(1), x.dtype) == 0:
            return spmm_rows_16_impl(crow, col, val, x)
        return spmm_rounded_16_impl(crow, col, val, x, column_slices=False)
    y = torch.empty_like(x)
    n, f = x.shape
    if n == 0 or f == 0:
        return y
    with _on(x.device):
        status = library().as_spmm_csr_f32(
            _ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(), f, int(_env_vec4()), _stream(x.device)
        )
    _raise(status, "autosage::spmm_csr")
    return y


def spmm_csr_split_impl(crow, col, val, x, feature_tile, warps_per_block, hub_threshold):
    check_spmm_inputs(crow, col, val, x)
    _maybe_validate(crow, col)
    _check(feature_tile in (64, 128), "feature_tile must be 64 or 128")
    _check(warps_per_block in (2, 4, 8), "warps_per_block must be 2, 4, or 8")
    _check(hub_threshold > 0, "hub_threshold must be positive")
    y = torch.empty_like(x)
    n, f = x.shape
    if n == 0 or f == 0:
        return y
    lib = library()
    ws = _workspace(lib.as_spmm_split_workspace_bytes(n), x.device)
    with _on(x.device):
        status = lib.as_spmm_csr_split_f32(
            _ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(), f, int(feature_tile),
            int(warps_per_block), int(hub_threshold), int(_env_vec4()), _env_hub_mode(), _ptr(ws), ws.numel(),
            _stream(x.device),
        )
    _raise(status, "autosage::spmm_csr_split")
    return y


# A plan holds 4 bytes per edge and per row (460 MB for a 115M-edge graph).
_FSLICE_PLAN_MEMO = GraphMemo("fslice_plan", max_entries=8, max_bytes=4 << 30)
FSLICE_FLAG_BAD_COLUMN = 1
FSLICE_FLAG_LONG_ROW = 2


# Column phases of the feature-sliced SpMM (the same bits for any count):
# two where one slice of X (n_cols x 128 bytes) is well beyond an XCD's 4 MB
# L2, the rows are long enough to cut, and the columns ascend in every row
# (otherwise a cut narrows no gather window).  On the 233k-row skewed graph
# two phases take F = 128 from 3.15 to 2.82 ms; three or more cost more than
# they save.  AUTOSAGE_FSLICE_PHASES = 1 .. 8 forces a count.
FSLICE_MAX_PHASES = 8
_FSLICE_PHASE_MIN_COLS = 1 << 16
_FSLICE_PHASE_MIN_MEAN_DEGREE = 32


def fslice_phases(crow: torch.Tensor, col: torch.Tensor, n_cols: int) -> int:
    """The column-phase count the feature-sliced SpMM uses for this graph."""
    forced = _env.get("AUTOSAGE_FSLICE_PHASES", "auto").strip().lower()
    if forced != "auto":
        try:
            phases = int(forced)
        except ValueError:
            phases = 0
        if not 1 <= phases <= FSLICE_MAX_PHASES:
            raise ValueError(f"AUTOSAGE_FSLICE_PHASES must be auto or an integer in [1, {FSLICE_MAX_PHASES}]")
        return phases
    n = crow.numel() - 1
    if n_cols < _FSLICE_PHASE_MIN_COLS or col.numel() < _FSLICE_PHASE_MIN_MEAN_DEGREE * max(n, 1):
        return 1
    if not columns_ascending(crow, col, None if n_cols == n else int(n_cols)):
        return 1
    return 2


def fslice_plan(crow: torch.Tensor, col: torch.Tensor, n_cols: int,
                phases: Optional[int] = None) -> tuple[torch.Tensor, int]:
    """(plan, tag) of the feature-sliced SpMM for this graph: the rows sorted
    by degree, the columns as int32 and each column phase's row tasks, built
    on the device once per live, unmodified (crow, col) pair, column count and
    phase count (``fslice_phases`` when None), then reused whatever X, F and
    the weights.  The build synchronises the stream once and raises on a
    column outside [0, n_cols) or a row of 2^31 or more edges."""
    lib = library()
    if phases is None:
        phases = fslice_phases(crow, col, n_cols)

    def compute() -> tuple[torch.Tensor, int]:
        n = crow.numel() - 1
        nnz = col.numel()
        plan = _workspace(lib.as_spmm_fslice_plan_bytes(n, nnz, phases), crow.device)
        scratch = _workspace(lib.as_spmm_fslice_plan_workspace_bytes(n), crow.device)
        tag = ctypes.c_int64(0)
        with _on(crow.device):
            status = lib.as_spmm_fslice_plan(_ptr(crow), _ptr(col), n, int(n_cols), nnz, int(phases), _ptr(plan),
                                             plan.numel(), _ptr(scratch), scratch.numel(), ctypes.byref(tag),
                                             _stream(crow.device))
            _raise(status, "autosage feature-sliced plan")
            flags = int(plan[:4].view(torch.int32).item())  # synchronises the stream
        del scratch
        _check(not flags & FSLICE_FLAG_BAD_COLUMN, f"col values must be in [0, {int(n_cols)})")
        _check(not flags & FSLICE_FLAG_LONG_ROW, "rows of 2^31 or more edges are not supported")
        return plan, int(tag.value)

    return _FSLICE_PLAN_MEMO.get((crow, col), (int(n_cols), int(phases)), compute)


def _spmm_fslice(crow, col, val, x, n_rows: int) -> torch.Tensor:
    """Feature-sliced exact SpMM of an n_rows × x.size(0) CSR (the bits of
    spmm_csr: CSR-order fp32 chains)."""
    f = x.size(1)
    y = torch.empty((n_rows, f), dtype=x.dtype, device=x.device)
    if n_rows == 0 or f == 0:
        return y
    lib = library()
    n_cols = x.size(0)
    plan, tag = fslice_plan(crow, col, n_cols)
    ws = _workspace(lib.as_spmm_fslice_workspace_bytes(n_cols, f), x.device)
    with _on(x.device):
        status = lib.as_spmm_csr_fslice_f32(
            _ptr(crow), _ptr(val), _ptr(x), _ptr(y), n_rows, n_cols, col.numel(), f, _ptr(plan), plan.numel(), tag,
            _ptr(ws), ws.numel(), _stream(x.device),
        )
    _raise(status, "autosage::spmm_csr_fslice")
    return y


def spmm_csr_fslice_impl(crow, col, val, x):
    """Feature-sliced SpMM: bit-identical to ``spmm_csr`` (per output element
    an fp32 chain over the row's edges in CSR order), with 32-feature slices
    of X spread over the XCDs (any column order, any F)."""
    check_spmm_inputs(crow, col, val, x)
    _maybe_validate(crow, col)
    return _spmm_fslice(crow, col, val, x, crow.numel() - 1)


def _colslice_workspace_cap() -> int:
    return int(float(_env.get("AUTOSAGE_COLSLICE_WORKSPACE_MB", "4096")) * 2**20)


def spmm_csr_colslice_impl(crow, col, val, x):
    """Column-sliced SpMM (fp64 accumulation, one column slice per XCD).
    The kernels cut rows along ascending columns: a graph whose columns do
    not ascend runs on its row-sorted copy (``row_sorted``, built once per
    graph), which has the same products in every row."""
    check_spmm_inputs(crow, col, val, x, allow_16=True)
    _maybe_validate(crow, col)
    sorted_col, perm = row_sorted(crow, col)
    val = _row_sorted_weights(col, val, perm)
    col = sorted_col
    if x.dtype in DTYPES_16:
        return spmm_rounded_16_impl(crow, col, val, x, column_slices=True)
    y = torch.empty_like(x)
    n, f = x.shape
    if n == 0 or f == 0:
        return y
    lib = library()
    if colslice_plans_enabled():
        sliced, grouped = colslice_row_counts(crow, f, x.dtype)
        return _spmm_colslice_planned(crow, col, val, x, y, column_slices=True, sliced=sliced, grouped=grouped)
    # the preferred size (two partial buffers of a quarter of the rows); a
    # smaller cap runs the pipeline in more, smaller chunks
    full = lib.as_spmm_colslice_workspace_bytes(n, f)
    ws = _workspace(min(full, _colslice_workspace_cap()), x.device)
    with _on(x.device):
        status = lib.as_spmm_csr_colslice_f32(
            _ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(), f, _ptr(ws), ws.numel(),
            sliced_rows(crow, True, f, x.dtype), _stream(x.device),
        )
    _raise(status, "autosage::spmm_csr_colslice")
    return y


def block_sliced_rows(crow: torch.Tensor, f: int, dtype: torch.dtype, column_slices: bool) -> int:
    """The most rows of slicing degree in one row block of the column-sliced
    plan: what its partial buffers are sized for.  One device reduction and
    host sync per live, unmodified crow and settings (memoised)."""
    lib = library()
    code = 0 if dtype == torch.float32 else DTYPES_16[dtype]
    degree = int(lib.as_spmm_colslice_min_degree(int(bool(column_slices)), f, code))
    n = crow.numel() - 1

    def compute() -> int:
        begins = (ctypes.c_int64 * 65)()
        blocks = int(lib.as_spmm_colslice_row_blocks(n, code, begins, 65))
        if blocks < 1 or blocks > 64:
            return -1
        deg = crow[1:] - crow[:-1]
        long = (deg >= degree).to(torch.int64).cumsum(0)
        ends = torch.tensor([begins[b] for b in range(blocks + 1)], device=crow.device)
        at = torch.cat([torch.zeros(1, dtype=torch.int64, device=crow.device), long])[ends]
        return int((at[1:] - at[:-1]).max().item())

    return _ROW_COUNT_MEMO.get((crow,), ("block_sliced", degree, code), compute)


def colslice_plans_enabled() -> bool:
    """Whether the column-sliced SpMM reuses a per-graph plan (slice points
    and binned row order) across calls; ``AUTOSAGE_COLSLICE_PLAN=off`` builds
    them on every call instead (same bits)."""
    return _env.get("AUTOSAGE_COLSLICE_PLAN", "on").lower() != "off"


# A plan holds about 28 bytes per row (6.5 MB for a 233k-row graph).
_PLAN_MEMO = GraphMemo("colslice_plan", max_entries=32, max_bytes=1 << 30)


def colslice_plan(crow: torch.Tensor, col: torch.Tensor, f: int, dtype: torch.dtype,
                  column_slices: bool, n_cols: Optional[int] = None) -> tuple[torch.Tensor, int]:
    """(plan, tag) of the column-sliced SpMM for this graph (columns ascending
    within rows for column slices), F and element type: the slice points and
    the degree-binned row order, built on the device once per live,
    unmodified (crow, col) pair and settings, then reused by every call
    whatever X.  ``n_cols``: the column space of a row shard (the rows of
    the whole X); None for a square graph.  The build synchronises the
    stream once, so that a later call on another stream finds the plan
    complete."""
    lib = library()
    code = 0 if dtype == torch.float32 else DTYPES_16[dtype]
    degree = int(lib.as_spmm_colslice_min_degree(int(bool(column_slices)), f, code))

    def compute() -> tuple[torch.Tensor, int]:
        n = crow.numel() - 1
        plan = _workspace(lib.as_spmm_colslice_plan_bytes(n), crow.device)
        tag = ctypes.c_int64(0)
        with _on(crow.device):
            if n_cols is None:
                status = lib.as_spmm_colslice_plan(_ptr(crow), _ptr(col), n, col.numel(), f, code,
                                                   int(bool(column_slices)), _ptr(plan), plan.numel(),
                                                   ctypes.byref(tag), _stream(crow.device))
            else:
                status = lib.as_spmm_colslice_plan_rect(_ptr(crow), _ptr(col), n, int(n_cols), col.numel(), f, code,
                                                        int(bool(column_slices)), _ptr(plan), plan.numel(),
                                                        ctypes.byref(tag), _stream(crow.device))
            _raise(status, "autosage column-sliced plan")
            torch.cuda.current_stream(crow.device).synchronize()
        return plan, int(tag.value)

    # the plan depends on the slicing degree and on fp32 against 16-bit (the
    # number of light buckets), not on F itself
    return _PLAN_MEMO.get((crow, col), (degree, code != 0, bool(column_slices), n_cols), compute)


def _spmm_colslice_planned(crow, col, val, x, y, column_slices: bool, sliced: int, grouped: int,
                           n_cols: Optional[int] = None):
    """The column-sliced SpMM on its per-graph plan: the workspace holds the
    partial buffers only (the workspace cap counts the plan, as in the
    unplanned call).  ``n_cols``: as for ``colslice_plan``."""
    n = crow.numel() - 1
    f = x.size(1)
    code = 0 if x.dtype == torch.float32 else DTYPES_16[x.dtype]
    lib = library()
    plan, tag = colslice_plan(crow, col, f, x.dtype, column_slices, n_cols)
    needed = lib.as_spmm_colslice_planned_workspace_bytes(n, col.numel(), f, code,
                                                          block_sliced_rows(crow, f, x.dtype, column_slices))
    ws = _workspace(max(min(needed, _colslice_workspace_cap() - plan.numel()), 0), x.device)
    with _on(x.device):
        if n_cols is None:
            status = lib.as_spmm_csr_colslice_planned(
                _ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(), f, code, int(column_slices),
                _ptr(plan), plan.numel(), tag, _ptr(ws), ws.numel(), sliced, grouped, _stream(x.device),
            )
        else:
            status = lib.as_spmm_csr_colslice_planned_rect(
                _ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, int(n_cols), col.numel(), f, code,
                int(column_slices), _ptr(plan), plan.numel(), tag, _ptr(ws), ws.numel(), sliced, grouped,
                _stream(x.device),
            )
    _raise(status, "autosage::spmm_csr_colslice" if code == 0 else "autosage::spmm_csr (16-bit)")
    return y


def spmm_csr_rect_impl(crow, col, val, x, exact: bool = False):
    """Y = A·X for an n × n_cols CSR A (n = crow.numel() - 1 rows, n_cols =
    x.size(0)); Y has n rows.  This is the product of one row shard of a
    larger graph (its rows, crow rebased to 0, the columns unchanged) with
    the whole X.

    ``exact``: fp32 only, one wave per row in CSR order (the sequential
    fp32 product of ``spmm_csr``, bit-identical to the same rows of the whole
    graph's product).  Otherwise the column-sliced schedule: fp32 with fp64
    partials per column slice, 16-bit rounded once; the slices cut the
    whole column space [0, n_cols), so every row is summed as in the whole
    graph (a graph whose columns do not ascend runs on its row-sorted copy)."""
    check_spmm_inputs(crow, col, val, x, allow_16=not exact, rect=True)
    n = crow.numel() - 1
    n_cols, f = x.shape
    _check(n <= 2**31 - 1 and n_cols <= 2**31 - 1, "crow and x must have fewer than 2^31 rows")
    y = torch.empty((n, f), dtype=x.dtype, device=x.device)
    if n == 0 or f == 0:
        return y
    if _env.get("AUTOSAGE_VALIDATE") == "1":
        validate_csr(crow, col, n_cols)
    if exact:
        with _on(x.device):
            status = library().as_spmm_csr_f32(
                _ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(), f, int(_env_vec4()),
                _stream(x.device),
            )
        _raise(status, "autosage row-shard SpMM")
        return y
    sorted_col, perm = row_sorted(crow, col, n_cols)
    val = _row_sorted_weights(col, val, perm)
    col = sorted_col
    sliced, grouped = colslice_row_counts(crow, f, x.dtype)
    return _spmm_colslice_planned(crow, col, val, x, y, True, sliced, grouped, n_cols=n_cols)


# 16-bit spmm_csr on graphs of at most this many edges, or without a row of
# slicing degree, sums every row whole in one launch (the sliced schedule's
# set-up costs more there: 0.012 against 0.060 ms on a 131k-edge graph,
# 0.637 against 0.705 ms on 16.8M edges in rows of 16).
ROWS_16_MAX_NNZ = 1 << 18


def spmm_rows_16_impl(crow, col, val, x):
    """The 16-bit SpMM of ``spmm_rounded_16_impl`` (same bits) with every
    row summed whole by one wavefront: one launch, no workspace."""
    y = torch.empty_like(x)
    n, f = x.shape
    if n == 0 or f == 0:
        return y
    with _on(x.device):
        status = library().as_spmm_csr_rows_16(
            _ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(), f, DTYPES_16[x.dtype],
            _stream(x.device),
        )
    _raise(status, "autosage::spmm_csr (16-bit rows)")
    return y


def spmm_rounded_16_impl(crow, col, val, x, column_slices: bool):
    """SpMM on bf16/fp16 features (weights of the same type): every output is
    the fp64 sum of the exact products rounded to fp32 and then to x's dtype,
    the same bits whatever the schedule when that sum is exact.  Short rows
    of degree below ``as_spmm_rounded_16_group_degree(F)`` run several to a
    wavefront.  ``column_slices``: one column slice
    per XCD (columns must ascend within rows); otherwise rows of degree >= 1024
    are cut into 8 equal runs of edges."""
    y = torch.empty_like(x)
    n, f = x.shape
    if n == 0 or f == 0:
        return y
    lib = library()
    threshold = int(lib.as_spmm_colslice_min_degree(int(bool(column_slices)), f, DTYPES_16[x.dtype]))
    sliced, grouped = row_counts(crow, threshold, int(lib.as_spmm_rounded_16_group_degree(f)))
    if colslice_plans_enabled():
        return _spmm_colslice_planned(crow, col, val, x, y, bool(column_slices), sliced, grouped)
    # partial rows for the sliced rows only (a short workspace sums the rest
    # whole, with the same bits)
    needed = lib.as_spmm_rounded_16_workspace_bytes(n, f, sliced)
    ws = _workspace(min(needed, _colslice_workspace_cap()), x.device)
    with _on(x.device):
        status = lib.as_spmm_csr_rounded_16(
            _ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(), f, DTYPES_16[x.dtype],
            int(bool(column_slices)), _ptr(ws), ws.numel(), sliced, grouped, _stream(x.device),
        )
    _raise(status, "autosage::spmm_csr (16-bit)")
    return y


# Schedule of sddmm_csr on 16-bit inputs: any schedule gives the same bits,
# so the whole-graph op takes blocks of 64 edges in CSR order, faster than
# the split schedule (rows by degree, hub rows in 2048-edge chunks) on every
# graph measured: 14 % on the 50M-edge hub graph (bf16, F = 64), 28 % on
# the 124M-edge attention graph, 11 % on the skewed 115M-edge graph.


# fp32 sddmm_csr: every output keeps the reference kernel's dot order on any
# schedule, so graphs that can hold a row of this many edges take the split
# schedule (such rows cut into 2048-edge chunks over a workgroup's waves)
# instead of one wave per row; the bits are the same.
SDDMM_HUB_THRESHOLD = 1024
SDDMM_WAVES = 4


def sddmm_csr_impl(crow, col, query, key):
    check_sddmm_inputs(crow, col, query, key, allow_16=True)
    if query.dtype in DTYPES_16:
        return sddmm_edges_16_impl(crow, col, query, key)
    if col.numel() >= SDDMM_HUB_THRESHOLD:
        return sddmm_csr_split_impl(crow, col, query, key, SDDMM_WAVES, SDDMM_HUB_THRESHOLD)
    _maybe_validate(crow, col)
    nnz = col.numel()
    n, f = query.shape
    if f == 0:
        return torch.zeros(nnz, dtype=query.dtype, device=query.device)
    out = torch.empty(nnz, dtype=query.dtype, device=query.device)
    if n == 0 or nnz == 0:
        return out
    with _on(query.device):
        status = library().as_sddmm_csr_f32(
            _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(out), n, nnz, f, _stream(query.device)
        )
    _raise(status, "autosage::sddmm_csr")
    return out


def sddmm_csr_split_impl(crow, col, query, key, warps_per_block, hub_threshold):
    check_sddmm_inputs(crow, col, query, key, allow_16=True)
    if query.dtype in DTYPES_16:
        return sddmm_rounded_16_impl(crow, col, query, key, warps_per_block, hub_threshold)
    _maybe_validate(crow, col)
    _check(warps_per_block in (2, 4, 8), "warps_per_block must be 2, 4, or 8")
    _check(0 < hub_threshold <= 2**31 - 1, "hub_threshold must be a positive 32-bit integer")
    nnz = col.numel()
    n, f = query.shape
    if f == 0:
        return torch.zeros(nnz, dtype=query.dtype, device=query.device)
    out = torch.empty(nnz, dtype=query.dtype, device=query.device)
    if n == 0 or nnz == 0:
        return out
    lib = library()
    ws = _workspace(lib.as_sddmm_split_workspace_bytes(n), query.device)
    with _on(query.device):
        status = lib.as_sddmm_csr_split_f32(
            _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(out), n, nnz, f, int(warps_per_block),
            int(hub_threshold), _ptr(ws), ws.numel(), _stream(query.device),
        )
    _raise(status, "autosage::sddmm_csr_split")
    return out


def sddmm_rounded_16_impl(crow, col, query, key, warps_per_block: int, hub_threshold: int):
    """SDDMM on bf16/fp16 query and key: out[e] is the fp64 sum of the exact
    products rounded to fp32 and then to the input dtype; the same bits for
    any schedule when that sum is exact.  The split schedule of
    ``sddmm_csr_split`` (rows of degree >= ``hub_threshold`` in 2048-edge
    chunks)."""
    check_sddmm_inputs(crow, col, query, key, allow_16=True)
    _check(query.dtype in DTYPES_16, "query and key must be bfloat16 or float16")
    _maybe_validate(crow, col)
    _check(warps_per_block in (2, 4, 8), "warps_per_block must be 2, 4, or 8")
    _check(0 < hub_threshold <= 2**31 - 1, "hub_threshold must be a positive 32-bit integer")
    nnz = col.numel()
    n, f = query.shape
    if f == 0:
        return torch.zeros(nnz, dtype=query.dtype, device=query.device)
    out = torch.empty(nnz, dtype=query.dtype, device=query.device)
    if n == 0 or nnz == 0:
        return out
    lib = library()
    ws = _workspace(lib.as_sddmm_split_workspace_bytes(n), query.device)
    with _on(query.device):
        status = lib.as_sddmm_csr_rounded_16(
            _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(out), n, nnz, f, DTYPES_16[query.dtype],
            int(warps_per_block), int(hub_threshold), _ptr(ws), ws.numel(), _stream(query.device),
        )
    _raise(status, "autosage::sddmm_csr (16-bit)")
    return out


def sddmm_edges_16_impl(crow, col, query, key):
    """SDDMM on bf16/fp16 query and key over blocks of 64 edges in CSR order
    (no degree split): the same bits as ``sddmm_rounded_16_impl``."""
    check_sddmm_inputs(crow, col, query, key, allow_16=True)
    _check(query.dtype in DTYPES_16, "query and key must be bfloat16 or float16")
    _maybe_validate(crow, col)
    nnz = col.numel()
    n, f = query.shape
    if f == 0:
        return torch.zeros(nnz, dtype=query.dtype, device=query.device)
    out = torch.empty(nnz, dtype=query.dtype, device=query.device)
    if n == 0 or nnz == 0:
        return out
    lib = library()
    ws = _workspace(lib.as_sddmm_edges_16_workspace_bytes(nnz), query.device)
    with _on(query.device):
        status = lib.as_sddmm_csr_edges_16(
            _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(out), n, nnz, f, DTYPES_16[query.dtype],
            _ptr(ws), ws.numel(), _stream(query.device),
        )
    _raise(status, "autosage::sddmm_csr (16-bit, edge blocks)")
    return out


def csr_row_softmax_impl(crow, scores):
    _check(crow.is_cuda and scores.is_cuda, "crow and scores must be CUDA tensors")
    _check(crow.dtype == torch.long and crow.dim() == 1 and crow.is_contiguous(), "crow must be contiguous torch.long")
    _check((scores.dtype == torch.float32 or scores.dtype in DTYPES_16) and scores.dim() == 1,
           "scores must be one-dimensional float32 (or bfloat16 / float16)")
    _check(crow.device == scores.device, "crow and scores must be on the same CUDA device")
    scores = scores.contiguous()
    probs = torch.empty_like(scores)
    n = crow.numel() - 1
    if n <= 0 or scores.numel() == 0:
        return probs
    with _on(scores.device):
        if scores.dtype in DTYPES_16:
            # fp32 softmax of the exactly converted scores, rounded once
            status = library().as_csr_row_softmax_16(
                _ptr(crow), _ptr(scores), _ptr(probs), n, scores.numel(), DTYPES_16[scores.dtype],
                _stream(scores.device)
            )
        else:
            status = library().as_csr_row_softmax_f32(
                _ptr(crow), _ptr(scores), _ptr(probs), n, scores.numel(), _stream(scores.device)
            )
    _raise(status, "autosage::csr_row_softmax")
    return probs


def csr_row_softmax_backward_impl(crow, probs, grad):
    """dL/dscores of ``csr_row_softmax`` from its output ``probs`` and
    dL/dprobs (fp32 arithmetic; 16-bit values convert exactly and each result
    is rounded once)."""
    _check(crow.is_cuda and probs.is_cuda and grad.is_cuda, "crow, probs and grad must be CUDA tensors")
    _check(crow.dtype == torch.long and crow.dim() == 1 and crow.is_contiguous(), "crow must be contiguous torch.long")
    _check(probs.dtype == grad.dtype and probs.shape == grad.shape and probs.dim() == 1,
           "probs and grad must be one-dimensional, of one dtype and shape")
    _check(probs.dtype == torch.float32 or probs.dtype in DTYPES_16, "probs must be float32, bfloat16 or float16")
    probs, grad = probs.contiguous(), grad.contiguous()
    out = torch.empty_like(probs)
    n = crow.numel() - 1
    if n <= 0 or probs.numel() == 0:
        return out.zero_()
    dtype = 0 if probs.dtype == torch.float32 else DTYPES_16[probs.dtype]
    with _on(probs.device):
        status = library().as_csr_row_softmax_backward(
            _ptr(crow), _ptr(probs), _ptr(grad), _ptr(out), n, probs.numel(), dtype, _stream(probs.device)
        )
    _raise(status, "autosage::csr_row_softmax (backward)")
    return out


def csr_attention_impl(crow, col, query, key, value, scale=1.0):
    check_sddmm_inputs(crow, col, query, key)
    _maybe_validate(crow, col)
    _check(value.is_cuda and value.device == query.device, "value must be on the same CUDA device as query")
    _check(value.dtype == torch.float32 and value.dim() == 2 and value.is_contiguous(),
           "value must be contiguous float32 with shape [N, F_v]")
    _check(value.size(0) == query.size(0), "value must have one row per node")
    n, fqk = query.shape
    fv = value.size(1)
    nnz = col.numel()
    out = torch.empty((n, fv), dtype=value.dtype, device=value.device)
    if n == 0 or fv == 0:
        return out
    if fqk == 0 and nnz > 0:
        # all scores are zero: the softmax of each row is uniform
        scores = torch.zeros(nnz, dtype=query.dtype, device=query.device)
        return spmm_csr_impl(crow, col, csr_row_softmax_impl(crow, scores), value)
    lib = library()
    ws = _workspace(lib.as_csr_attention_workspace_bytes(n, nnz), query.device)
    with _on(query.device):
        status = lib.as_csr_attention_f32(
            _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(value), _ptr(out), n, nnz, fqk, fv, float(scale),
            _ptr(ws), ws.numel(), _stream(query.device),
        )
    _raise(status, "autosage::csr_attention")
    return out


def attention_colslice_supported(query: torch.Tensor, value: torch.Tensor) -> bool:
    """Feature widths the column-sliced attention handles (16-byte lanes):
    fp32 multiples of 4 in [4, 256], bf16 / fp16 multiples of 8 in [8, 512];
    rows 16-byte aligned."""
    fqk, fv = query.size(1), value.size(1)
    if query.dtype in DTYPES_16:
        widths = fqk % 8 == 0 and 8 <= fqk <= 512 and fv % 8 == 0 and 8 <= fv <= 512
    else:
        widths = fqk % 4 == 0 and 4 <= fqk <= 256 and fv % 4 == 0 and 4 <= fv <= 256
    return widths and all(t.data_ptr() % 16 == 0 for t in (query, value))


def csr_attention_colslice_impl(crow, col, query, key, value, scale=1.0):
    """Column-sliced attention (one column slice per XCD, online softmax per
    (row, slice)).  A graph whose columns do not ascend runs on its row-sorted
    copy (``row_sorted``, built once per graph).  float32 inputs, or bf16 /
    fp16 (computed in fp32, each output rounded once)."""
    check_sddmm_inputs(crow, col, query, key, allow_16=True)
    _maybe_validate(crow, col)
    _check(value.is_cuda and value.device == query.device, "value must be on the same CUDA device as query")
    _check(value.dtype == query.dtype and value.dim() == 2 and value.is_contiguous(),
           "value must be contiguous with shape [N, F_v] and query's dtype")
    _check(value.size(0) == query.size(0), "value must have one row per node")
    # the slices are cut along ascending columns: other graphs run on their
    # row-sorted copy (the same edges per row; the row softmax and the sum
    # over a row do not depend on the edge order beyond rounding)
    col = row_sorted(crow, col)[0]
    n, fqk = query.shape
    fv = value.size(1)
    nnz = col.numel()
    half = query.dtype in DTYPES_16
    if not attention_colslice_supported(query, value) or key.data_ptr() % 16 != 0:
        raise ValueError("csr_attention_colslice needs F_qk and F_v multiples of 4 in [4, 256] (float32) or of 8 "
                         "in [8, 512] (bfloat16 / float16) and 16-byte aligned rows")
    out = torch.empty((n, fv), dtype=value.dtype, device=value.device)
    if n == 0:
        return out
    lib = library()
    plan, tag = attention_plan(crow, col, query.dtype) if colslice_plans_enabled() else (None, 0)
    # the workspace cap counts the plan, as in a call that builds it
    size = min(lib.as_csr_attention_colslice_workspace_bytes(n, nnz, fv), _colslice_workspace_cap())
    ws = _workspace(size - (plan.numel() if plan is not None else 0), query.device)
    with _on(query.device):
        if half:
            status = lib.as_csr_attention_colslice_16(
                _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(value), _ptr(out), n, nnz, fqk, fv,
                float(scale), DTYPES_16[query.dtype], _ptr(plan), tag, _ptr(ws), ws.numel(), _stream(query.device),
            )
        else:
            status = lib.as_csr_attention_colslice_f32(
                _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(value), _ptr(out), n, nnz, fqk, fv,
                float(scale), _ptr(plan), tag, _ptr(ws), ws.numel(), _stream(query.device),
            )
    _raise(status, "autosage::csr_attention_colslice")
    return out


def attention_plan(crow: torch.Tensor, col: torch.Tensor, dtype: torch.dtype,
                   n_cols: Optional[int] = None) -> tuple[torch.Tensor, int]:
    """(plan, tag) of the column-sliced attention on this graph (columns
    ascending within rows) for ``dtype``: slice points and the binned row
    order, built once per live, unmodified (crow, col) pair and element type
    (fp32 or 16-bit), then reused whatever Q, K and V; it also serves the
    backward's passes of the same element type.  ``n_cols``: the column
    space of a row shard (the rows of the whole K and V); None for a square
    graph.  The build synchronises the stream once."""
    lib = library()
    code = 0 if dtype == torch.float32 else DTYPES_16[dtype]

    def compute() -> tuple[torch.Tensor, int]:
        n = crow.numel() - 1
        plan = _workspace(lib.as_csr_attention_plan_bytes(n), crow.device)
        tag = ctypes.c_int64(0)
        with _on(crow.device):
            if n_cols is None:
                status = lib.as_csr_attention_plan(_ptr(crow), _ptr(col), n, col.numel(), code, _ptr(plan),
                                                   plan.numel(), ctypes.byref(tag), _stream(crow.device))
            else:
                status = lib.as_csr_attention_plan_rect(_ptr(crow), _ptr(col), n, int(n_cols), col.numel(), code,
                                                        _ptr(plan), plan.numel(), ctypes.byref(tag),
                                                        _stream(crow.device))
            _raise(status, "autosage attention plan")
            torch.cuda.current_stream(crow.device).synchronize()
        return plan, int(tag.value)

    return _PLAN_MEMO.get((crow, col), ("attention", code != 0, n_cols), compute)


def _check_rect_pair(crow, col, rows: torch.Tensor, whole: torch.Tensor, what: str) -> None:
    """Inputs of a row shard's SDDMM or attention: ``rows`` holds the shard's
    rows of the query (crow.numel() - 1 of them), ``whole`` the whole key."""
    _check(crow.is_cuda and col.is_cuda and rows.is_cuda and whole.is_cuda, f"{what}: inputs must be CUDA tensors")
    _check(crow.dtype == torch.long and col.dtype == torch.long, "crow and col must use torch.long indices")
    _check(crow.dim() == 1 and col.dim() == 1 and crow.numel() >= 1, "crow and col must be one-dimensional")
    _check(rows.dim() == 2 and whole.dim() == 2 and rows.size(1) == whole.size(1),
           f"{what}: query and key must have the same feature width")
    _check(rows.size(0) == crow.numel() - 1, f"{what}: query must hold one row per row of the shard")
    _check(rows.dtype == whole.dtype and (rows.dtype == torch.float32 or rows.dtype in DTYPES_16),
           f"{what}: query and key must share float32, bfloat16 or float16")
    _check(crow.device == rows.device and col.device == rows.device and whole.device == rows.device,
           f"{what}: inputs must be on one CUDA device")
    _check(crow.is_contiguous() and col.is_contiguous() and rows.is_contiguous() and whole.is_contiguous(),
           f"{what}: inputs must be contiguous")
    _check(crow.numel() - 1 <= 2**31 - 1 and whole.size(0) <= 2**31 - 1, f"{what}: too many rows")


def sddmm_csr_rect_impl(crow, col, query, key):
    """out[e] = <query[r], key[col_e]> for the edges of a row shard: ``query``
    holds the shard's rows, ``key`` the whole key (any number of rows).  fp32
    keeps the reference kernel's dot order (``sddmm_csr``'s bits); bf16 /
    fp16 the fp64 sum of the exact products, rounded once to fp32 and then to
    the element type."""
    _check_rect_pair(crow, col, query, key, "row-shard SDDMM")
    if _env.get("AUTOSAGE_VALIDATE") == "1":
        validate_csr(crow, col, key.size(0))
    n, f = query.shape
    nnz = col.numel()
    if f == 0:
        return torch.zeros(nnz, dtype=query.dtype, device=query.device)
    out = torch.empty(nnz, dtype=query.dtype, device=query.device)
    if n == 0 or nnz == 0:
        return out
    lib = library()
    with _on(query.device):
        if query.dtype in DTYPES_16:
            ws = _workspace(lib.as_sddmm_edges_16_workspace_bytes(nnz), query.device)
            status = lib.as_sddmm_csr_edges_16_rect(
                _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(out), n, key.size(0), nnz, f,
                DTYPES_16[query.dtype], _ptr(ws), ws.numel(), _stream(query.device),
            )
        elif nnz >= SDDMM_HUB_THRESHOLD:
            # fp32 kernels address the key through the column indices only
            ws = _workspace(lib.as_sddmm_split_workspace_bytes(n), query.device)
            status = lib.as_sddmm_csr_split_f32(
                _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(out), n, nnz, f, SDDMM_WAVES,
                SDDMM_HUB_THRESHOLD, _ptr(ws), ws.numel(), _stream(query.device),
            )
        else:
            status = lib.as_sddmm_csr_f32(_ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(out), n, nnz, f,
                                          _stream(query.device))
    _raise(status, "autosage row-shard SDDMM")
    return out


def csr_attention_rect_impl(crow, col, query, key, value, scale=1.0):
    """The column-sliced attention of a row shard: ``query`` holds the
    shard's rows, ``key`` and ``value`` the whole graph's rows; the slices cut
    the whole column space, so every row is computed as in the whole graph
    (a graph whose columns do not ascend runs on its row-sorted copy)."""
    _check_rect_pair(crow, col, query, key, "row-shard attention")
    _check(value.is_cuda and value.device == query.device and value.dtype == query.dtype and value.dim() == 2
           and value.is_contiguous() and value.size(0) == key.size(0),
           "row-shard attention: value must be contiguous with key's rows and query's dtype")
    if not attention_colslice_supported(query, value) or key.data_ptr() % 16 != 0:
        raise ValueError("row-shard attention needs F_qk and F_v multiples of 4 in [4, 256] (float32) or of 8 "
                         "in [8, 512] (bfloat16 / float16) and 16-byte aligned rows")
    n_cols = key.size(0)
    col = row_sorted(crow, col, n_cols)[0]
    n, fqk = query.shape
    fv = value.size(1)
    nnz = col.numel()
    out = torch.empty((n, fv), dtype=value.dtype, device=value.device)
    if n == 0:
        return out
    lib = library()
    # a shard always runs on a plan: a call without one would cut the
    # slices over its own row count
    plan, tag = attention_plan(crow, col, query.dtype, n_cols)
    size = min(lib.as_csr_attention_colslice_workspace_bytes(n, nnz, fv), _colslice_workspace_cap())
    ws = _workspace(max(size - plan.numel(), 1), query.device)
    with _on(query.device):
        if query.dtype in DTYPES_16:
            status = lib.as_csr_attention_colslice_16(
                _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(value), _ptr(out), n, nnz, fqk, fv,
                float(scale), DTYPES_16[query.dtype], _ptr(plan), tag, _ptr(ws), ws.numel(), _stream(query.device),
            )
        else:
            status = lib.as_csr_attention_colslice_f32(
                _ptr(crow), _ptr(col), _ptr(query), _ptr(key), _ptr(value), _ptr(out), n, nnz, fqk, fv,
                float(scale), _ptr(plan), tag, _ptr(ws), ws.numel(), _stream(query.device),
            )
    _raise(status, "autosage row-shard attention")
    return out


def attention_backward_supported(query, key, value, out, grad_out) -> bool:
    """Shapes the two-pass attention backward handles: one element type for
    all five tensors, float32 with F_qk and F_v multiples of 4 in [4, 256] or
    bf16 / fp16 with multiples of 8 in [8, 512], 16-byte aligned dense
    tensors."""
    fqk, fv = query.size(1), value.size(1)
    tensors = (query, key, value, out, grad_out)
    dtype = query.dtype
    if dtype == torch.float32:
        step, top = 4, 256
    elif dtype in DTYPES_16:
        step, top = 8, 512
    else:
        return False
    return (all(t.dtype == dtype and t.is_contiguous() and t.data_ptr() % 16 == 0 for t in tensors)
            and fqk % step == 0 and step <= fqk <= top and fv % step == 0 and step <= fv <= top)


def csr_attention_backward_impl(crow, col, crow_t, col_t, query, key, value, out, grad_out, scale):
    """(grad_q, grad_k, grad_v) of the attention from its saved inputs, its
    output and dL/dout, in two native gather passes (over A and over its
    transpose (crow_t, col_t)); float32, or bf16 / fp16 (fp32 sums, each
    gradient rounded once)."""
    n, fqk = query.shape
    fv = value.size(1)
    nnz = col.numel()
    grad_q = torch.empty_like(query)
    grad_k = torch.empty_like(key)
    grad_v = torch.empty_like(value)
    if n == 0:
        return grad_q, grad_k, grad_v
    lib = library()
    code = 0 if query.dtype == torch.float32 else DTYPES_16[query.dtype]
    size = min(lib.as_csr_attention_backward_workspace_bytes(n, nnz, fqk, fv, code), _colslice_workspace_cap())
    plan = plan_t = None
    tag = tag_t = 0
    if colslice_plans_enabled():
        # plans of A and of Aᵀ for this element type (the forward's plan
        # serves pass 1); the workspace then needs no plan region
        plan, tag = attention_plan(crow, col, query.dtype)
        plan_t, tag_t = attention_plan(crow_t, col_t, query.dtype)
        size -= plan.numel()
    ws = _workspace(size, query.device)
    with _on(query.device):
        if code == 0:
            status = lib.as_csr_attention_backward_f32(
                _ptr(crow), _ptr(col), _ptr(crow_t), _ptr(col_t), _ptr(query), _ptr(key), _ptr(value), _ptr(out),
                _ptr(grad_out), _ptr(grad_q), _ptr(grad_k), _ptr(grad_v), n, nnz, fqk, fv, float(scale), _ptr(plan),
                tag, _ptr(plan_t), tag_t, _ptr(ws), ws.numel(), _stream(query.device),
            )
        else:
            # 16-bit: pass 1 sums t itself, the output is not read
            status = lib.as_csr_attention_backward_16(
                _ptr(crow), _ptr(col), _ptr(crow_t), _ptr(col_t), _ptr(query), _ptr(key), _ptr(value),
                _ptr(grad_out), _ptr(grad_q), _ptr(grad_k), _ptr(grad_v), n, nnz, fqk, fv, float(scale), code,
                _ptr(plan), tag, _ptr(plan_t), tag_t, _ptr(ws), ws.numel(), _stream(query.device),
            )
    _raise(status, "autosage::csr_attention (backward)")
    return grad_q, grad_k, grad_v


_VALIDATION_RULES = (
    (1, "crow[0] must be 0"),
    (2, "crow must be non-decreasing"),
    (4, "crow[-1] must equal the number of nonzeros"),
    (8, "column indices must lie in [0, N)"),
)


_UNSORTED_FLAG = 16
_ASCENDING_MEMO = GraphMemo("columns_ascending", max_entries=64)
_ROW_COUNT_MEMO = GraphMemo("row_counts", max_entries=64)
# A row-sorted copy of a cfg3-sized graph holds 16·nnz bytes (1.8 GB); it goes
# with its graph, and at most 4 GiB stay cached.
_ROW_SORTED_MEMO = GraphMemo("row_sorted", max_entries=16, max_bytes=4 << 30)
_SORTED_WEIGHTS_MEMO = GraphMemo("row_sorted_weights", max_entries=16, max_bytes=2 << 30)


def csr_flags(crow: torch.Tensor, col: torch.Tensor, n_cols: Optional[int] = None) -> int:
    """Bit mask of ``as_csr_validate`` (one device pass, one host sync)."""
    _check(crow.is_cuda and col.is_cuda, "crow and col must be CUDA tensors")
    _check(crow.dtype == torch.long and col.dtype == torch.long, "crow and col must use torch.long indices")
    crow = crow.contiguous()
    col = col.contiguous()
    n = crow.numel() - 1
    if n < 0:
        raise ValueError("crow must contain N + 1 entries")
    flags = torch.zeros(1, dtype=torch.int32, device=crow.device)
    with _on(crow.device):
        status = library().as_csr_validate(_ptr(crow), _ptr(col), n, col.numel(), n if n_cols is None else n_cols,
                                           _ptr(flags), _stream(crow.device))
    _raise(status, "csr_validate")
    return int(flags.item())


def _raise_for_flags(bad: int) -> None:
    problems = [text for bit, text in _VALIDATION_RULES if bad & bit]
    if problems:
        raise ValueError("invalid CSR graph: " + "; ".join(problems))


def validate_csr(crow: torch.Tensor, col: torch.Tensor, n_cols: Optional[int] = None) -> None:
    """Checks a device CSR graph on the GPU (one pass, one host sync) and
    raises ``ValueError`` naming every violated rule."""
    _raise_for_flags(csr_flags(crow, col, n_cols))


def columns_ascending(crow: torch.Tensor, col: torch.Tensor, n_cols: Optional[int] = None) -> bool:
    """Whether the columns of every row are in non-decreasing order (what
    the column slices of the sliced kernels are cut along).  Memoised per
    live, unmodified (crow, col) tensor pair; raises ``ValueError`` for a
    malformed graph.  ``n_cols``: the column count of a row shard (None: a
    square graph)."""

    def compute() -> bool:
        bad = csr_flags(crow, col, n_cols)
        _raise_for_flags(bad)
        return not bad & _UNSORTED_FLAG

    return _ASCENDING_MEMO.get((crow, col), n_cols, compute)


def row_sorted(crow: torch.Tensor, col: torch.Tensor,
               n_cols: Optional[int] = None) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    """(col', perm) with the columns of every row in ascending order:
    ``col'[k] = col[perm[k]]`` and ``perm`` permutes edges only inside their
    row (stable, so equal columns keep their order).  ``perm`` is None and
    ``col'`` is ``col`` when the columns already ascend.  The row-sorted
    graph has the same rows and the same multiset of (column, weight) pairs
    per row, so the column-sliced products over it are products of the
    original graph.  Built on the device once per live, unmodified graph
    (one sort of the nnz (row, column) keys) and memoised."""
    if columns_ascending(crow, col, n_cols):
        return col, None

    def compute():
        n = crow.numel() - 1
        width = n if n_cols is None else int(n_cols)
        counts = (crow[1:] - crow[:-1]).to(torch.long)
        rows = torch.repeat_interleave(torch.arange(n, device=crow.device, dtype=torch.long), counts,
                                       output_size=col.numel())
        # rows ascend already, so (row, column) keys sort each row's columns
        # in place; rows and columns below 2^31 keep row·width + column
        # inside int64
        keys = rows.mul_(width).add_(col)
        sorted_keys, perm = torch.sort(keys, stable=True)
        del keys
        col_sorted = sorted_keys.remainder_(width) if width > 0 else sorted_keys
        return col_sorted.contiguous(), perm

    return _ROW_SORTED_MEMO.get((crow, col), n_cols, compute)


def _row_sorted_weights(col: torch.Tensor, val: Optional[torch.Tensor], perm: Optional[torch.Tensor]):
    """``val`` in the order of ``row_sorted``'s permutation, memoised per live,
    unmodified (col, val, perm) triple (edge weights usually stay fixed per
    graph)."""
    if val is None or perm is None:
        return val
    # keyed on the permutation too: a new one (crow changed in place while
    # col and val did not) must miss
    return _SORTED_WEIGHTS_MEMO.get((col, val, perm), None, lambda: val.index_select(0, perm))


def row_counts(crow: torch.Tensor, long_from: int, short_below: int) -> tuple[int, int]:
    """(rows of degree >= ``long_from``, rows of degree < ``short_below``):
    per-graph constants that size the column-sliced SpMM's launches,
    computed once per live, unmodified ``crow`` (one host sync) and
    memoised."""

    def compute() -> tuple[int, int]:
        deg = crow[1:] - crow[:-1]
        counts = torch.stack([(deg >= long_from).sum(), (deg < short_below).sum()]).tolist()
        return int(counts[0]), int(counts[1])

    return _ROW_COUNT_MEMO.get((crow,), (long_from, short_below), compute)


def colslice_row_counts(crow: torch.Tensor, f: int, dtype: torch.dtype) -> tuple[int, int]:
    """(sliced rows, grouped short rows) of the column-sliced SpMM with column
    slices for F features of ``dtype``: its launch-sizing hints."""
    lib = library()
    code = 0 if dtype == torch.float32 else DTYPES_16[dtype]
    return row_counts(crow, int(lib.as_spmm_colslice_min_degree(1, f, code)),
                      int(lib.as_spmm_colslice_group_degree(f, code)))


def sliced_rows(crow: torch.Tensor, column_slices: bool, f: int, dtype: torch.dtype) -> int:
    """Rows the column-sliced SpMM slices for F features of ``dtype``
    (degree >= its threshold)."""
    code = 0 if dtype == torch.float32 else DTYPES_16[dtype]
    return row_counts(crow, int(library().as_spmm_colslice_min_degree(int(bool(column_slices)), f, code)), 0)[0]


def _maybe_validate(crow: torch.Tensor, col: torch.Tensor) -> None:
    if _env.get("AUTOSAGE_VALIDATE") == "1":
        validate_csr(crow, col)


def induced_sample(crow: torch.Tensor, col: torch.Tensor, val: Optional[torch.Tensor], selected: torch.Tensor):
    """(new_crow, new_col, new_val) of the sub-graph induced by the sorted
    row sample ``selected`` (``autosage/_auto.py:95-154``), on the device in
    two native passes and one host sync (the size of the kept edge list)."""
    _check(crow.is_cuda and col.is_cuda and selected.is_cuda, "induced_sample needs CUDA tensors")
    _check(crow.dtype == torch.long and col.dtype == torch.long and selected.dtype == torch.long,
           "crow, col and selected must use torch.long indices")
    _check(val is None or (val.is_cuda and val.dtype == torch.float32), "val must be a float32 CUDA tensor")
    crow, col, selected = crow.contiguous(), col.contiguous(), selected.contiguous()
    val = None if val is None else val.contiguous()
    n = crow.numel() - 1
    s = selected.numel()
    lib = library()
    ws = _workspace(lib.as_induced_sample_workspace_bytes(n), crow.device)
    new_crow = torch.empty(s + 1, dtype=torch.long, device=crow.device)
    with _on(crow.device):
        stream = _stream(crow.device)
        _raise(lib.as_induced_sample_count(_ptr(crow), _ptr(col), n, _ptr(selected), s, _ptr(new_crow), _ptr(ws),
                                           ws.numel(), stream), "induced_sample")
        kept = int(new_crow[s].item())
        new_col = torch.empty(kept, dtype=torch.long, device=crow.device)
        new_val = None if val is None else torch.empty(kept, dtype=val.dtype, device=val.device)
        _raise(lib.as_induced_sample_fill(_ptr(crow), _ptr(col), _ptr(val), n, _ptr(selected), s, _ptr(new_crow),
                                          _ptr(new_col), _ptr(new_val), _ptr(ws), ws.numel(), stream),
               "induced_sample")
    return new_crow, new_col, new_val


def bin_rows_by_degree(crow: torch.Tensor, threshold: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(heavy rows ascending, light rows ascending) as int32, computed on the
    device (``csrc/launcher_spmm.cu:49-59``).  Synchronises to split the lists."""
    _check(crow.is_cuda and crow.dtype == torch.long and crow.dim() == 1, "crow must be a CUDA torch.long vector")
    _check(threshold > 0, "hub_threshold must be positive")
    crow = crow.contiguous()
    n = crow.numel() - 1
    order = torch.empty(max(n, 1), dtype=torch.int32, device=crow.device)
    counts = torch.zeros(4, dtype=torch.int32, device=crow.device)
    lib = library()
    ws = _workspace(lib.as_bin_workspace_bytes(n), crow.device)
    with _on(crow.device):
        status = lib.as_bin_rows_by_degree(
            _ptr(crow), n, int(threshold), _ptr(order), _ptr(counts), _ptr(ws), ws.numel(), _stream(crow.device)
        )
    _raise(status, "bin_rows_by_degree")
    heavy = int(counts[0].item())
    return order[:heavy].clone(), order[heavy:n].clone()


_SCHEMAS = {
    "spmm_csr": ("spmm_csr(Tensor crow, Tensor col, Tensor? val, Tensor x) -> Tensor", spmm_csr_impl),
    "spmm_csr_split": (
        "spmm_csr_split(Tensor crow, Tensor col, Tensor? val, Tensor x, int feature_tile, int warps_per_block, "
        "int hub_threshold) -> Tensor",
        spmm_csr_split_impl,
    ),
    "spmm_csr_colslice": (
        "spmm_csr_colslice(Tensor crow, Tensor col, Tensor? val, Tensor x) -> Tensor",
        spmm_csr_colslice_impl,
    ),
    "spmm_csr_fslice": (
        "spmm_csr_fslice(Tensor crow, Tensor col, Tensor? val, Tensor x) -> Tensor",
        spmm_csr_fslice_impl,
    ),
    "sddmm_csr": ("sddmm_csr(Tensor crow, Tensor col, Tensor query, Tensor key) -> Tensor", sddmm_csr_impl),
    "sddmm_csr_split": (
        "sddmm_csr_split(Tensor crow, Tensor col, Tensor query, Tensor key, int warps_per_block, "
        "int hub_threshold) -> Tensor",
        sddmm_csr_split_impl,
    ),
    "csr_row_softmax": ("csr_row_softmax(Tensor crow, Tensor scores) -> Tensor", csr_row_softmax_impl),
    "csr_attention": (
        "csr_attention(Tensor crow, Tensor col, Tensor query, Tensor key, Tensor value, float scale=1.0) -> Tensor",
        csr_attention_impl,
    ),
    "csr_attention_colslice": (
        "csr_attention_colslice(Tensor crow, Tensor col, Tensor query, Tensor key, Tensor value, float scale=1.0) "
        "-> Tensor",
        csr_attention_colslice_impl,
    ),
}

OPERATOR_NAMES = tuple(_SCHEMAS)


def implementation(name: str):
    """The CUDA implementation registered for ``autosage::<name>``."""
    return _SCHEMAS[name][1]


def _register_operators() -> None:
    global _OPS_LIBRARY
    if _OPS_LIBRARY is not None:
        return
    lib = torch.library.Library("autosage", "DEF")
    for name, (schema, impl) in _SCHEMAS.items():
        lib.define(schema)
        lib.impl(name, impl, "CUDA")
    _OPS_LIBRARY = lib
    from . import _autograd

    _autograd.register()


def load(path: os.PathLike[str] | str) -> None:
    """Loads the library at ``path`` and registers the ``autosage::*`` ops."""
    global _LIB, _LIB_PATH
    if _LIB is None:
        _LIB = open_library(path)
        _LIB_PATH = Path(path)
    _register_operators()
