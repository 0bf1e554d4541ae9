"""The allocation-free split SpMM (``as_spmm_csr_split_f32_static``) through
the C ABI: bit for bit the output of ``as_spmm_csr_split_f32`` (the same
kernels, with the workspace in a static device array instead of a caller
buffer), on two calls in a row — the second on a smaller graph, so the
static scratch holds the first call's larger tables — and the size limit is
enforced on the host."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from autosage_amd import _native
from tests.gpu_common import case_graph, require_gpu

pytestmark = pytest.mark.gpu

MAX_ROWS = 1 << 22  # AS_STATIC_MAX_ROWS


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _graph(rows, features, seed, weighted):
    crow, col = case_graph(rows, 12, seed=seed, hubs=6, hub_degree=min(3000, rows), empty=0.05)
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((rows, features)).astype(np.float32)).cuda()
    val = torch.from_numpy(rng.standard_normal(col.size).astype(np.float32)).cuda() if weighted else None
    return torch.from_numpy(crow).cuda(), torch.from_numpy(col).cuda(), val, x


def _ptr(t):
    return None if t is None else t.data_ptr()


def _allocating(lib, crow, col, val, x, tile, waves, threshold):
    n, f = x.shape
    y = torch.full_like(x, float("nan"))
    ws = torch.empty(lib.as_spmm_split_workspace_bytes(n), dtype=torch.uint8, device=x.device)
    status = lib.as_spmm_csr_split_f32(_ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(), f, tile,
                                       waves, threshold, 1, 0, _ptr(ws), ws.numel(),
                                       torch.cuda.current_stream().cuda_stream)
    assert status == 0, lib.as_last_error()
    return y


def _static(lib, crow, col, val, x, tile, waves, threshold):
    n, f = x.shape
    y = torch.full_like(x, float("nan"))
    status = lib.as_spmm_csr_split_f32_static(_ptr(crow), _ptr(col), _ptr(val), _ptr(x), _ptr(y), n, col.numel(),
                                              f, tile, waves, threshold, 1, 0,
                                              torch.cuda.current_stream().cuda_stream)
    assert status == 0, lib.as_last_error()
    return y


@pytest.mark.parametrize("weighted", [False, True])
def test_static_split_equals_the_allocating_entry_point(weighted):
    lib = _native.library()
    # first call: 20,000 rows; second: 3,000 rows (smaller tables, the static
    # scratch still holds the first call's), other split parameters
    first = _graph(20_000, 128, seed=1, weighted=weighted)
    second = _graph(3_000, 64, seed=2, weighted=weighted)
    got1 = _static(lib, *first, 128, 4, 512)
    got2 = _static(lib, *second, 64, 2, 1024)
    want1 = _allocating(lib, *first, 128, 4, 512)
    want2 = _allocating(lib, *second, 64, 2, 1024)
    torch.cuda.synchronize()
    assert torch.equal(got1, want1)
    assert torch.equal(got2, want2)
    assert not torch.isnan(got2).any()


def test_static_split_limits_are_checked_on_the_host():
    lib = _native.library()
    stream = torch.cuda.current_stream().cuda_stream
    # too many rows: refused before any pointer is used or kernel launched
    status = lib.as_spmm_csr_split_f32_static(None, None, None, None, None, MAX_ROWS + 1, 0, 8, 64, 2, 1, 1, 0,
                                              stream)
    assert status == 4
    assert b"at most 4194304 rows" in lib.as_last_error()
    # the argument checks of the allocating entry point apply
    status = lib.as_spmm_csr_split_f32_static(None, None, None, None, None, 4, 0, 8, 32, 2, 1, 1, 0, stream)
    assert status == 1 and lib.as_last_error() == b"feature_tile must be 64 or 128"
    # nothing to do: a no-op success
    assert lib.as_spmm_csr_split_f32_static(None, None, None, None, None, 0, 0, 8, 64, 2, 1, 1, 0, stream) == 0
    assert lib.as_spmm_split_workspace_bytes(MAX_ROWS) <= 18 << 20
    assert isinstance(lib.as_spmm_csr_split_f32_static, ctypes._CFuncPtr)
