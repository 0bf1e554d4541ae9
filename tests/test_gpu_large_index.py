"""GPU parity on a graph of 2^24 + 1000 rows: the 64-bit address forms of the
column-sliced and 16-bit kernels (and, on 2^25 + 1000 rows, of the
feature-sliced SpMM).

Below 2^24 rows (and 4 GiB of features) the gather offsets of these kernels
are 32-bit (``off32`` / ``OFF32``); this graph is past that limit, so the
other forms run.  Most rows are empty; 2,000 rows hold short, column-sliced
and edge-sliced edges whose columns spread over the whole range, above 2^24
included.  The features and weights are small multiples of 2^-6 and 2^-3, so
every sum is exact in fp32 and the checks are bit-exact against the oracle on
the compacted sub-graph.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_common import require_gpu

pytestmark = pytest.mark.gpu

N = (1 << 24) + 1000
F = 64


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _values(rows: np.ndarray, features: int) -> np.ndarray:
    """x[r, f] = ((37 r + 11 f) mod 255 - 127) / 64 (exact in bf16, fp16, fp32)."""
    f = np.arange(features, dtype=np.int64)
    return (((rows[:, None] * 37 + f[None, :] * 11) % 255) - 127).astype(np.float32) / 64.0


def _device_values(n: int, features: int, dtype: torch.dtype) -> torch.Tensor:
    out = torch.empty(n, features, dtype=dtype, device="cuda")
    f = torch.arange(features, device="cuda", dtype=torch.int64)
    step = 1 << 20
    for r0 in range(0, n, step):
        r = torch.arange(r0, min(r0 + step, n), device="cuda", dtype=torch.int64)
        out[r0:r0 + r.numel()] = ((((r[:, None] * 37 + f[None, :] * 11) % 255) - 127).float() / 64.0).to(dtype)
    return out


@pytest.fixture(scope="module")
def graph():
    rng = np.random.default_rng(2024)
    rows = np.sort(rng.choice(N, size=2000, replace=False))
    deg = np.concatenate([rng.integers(1, 128, 1500), rng.integers(128, 1024, 400), rng.integers(1024, 2500, 100)])
    rng.shuffle(deg)
    counts = np.zeros(N, dtype=np.int64)
    counts[rows] = deg
    crow = np.zeros(N + 1, dtype=np.int64)
    np.cumsum(counts, out=crow[1:])
    col = np.concatenate([np.sort(rng.choice(N, size=d, replace=False)) for d in deg]).astype(np.int64)
    assert col.max() >= (1 << 24)
    val = (rng.integers(-16, 17, col.size).astype(np.float32) / 8.0)
    # the compacted sub-graph: the rows with edges, columns renumbered
    uniq, inv = np.unique(col, return_inverse=True)
    sub_crow = np.concatenate([[0], np.cumsum(counts[rows])]).astype(np.int64)
    return {"rows": rows, "crow": crow, "col": col, "val": val, "uniq": uniq, "sub_col": inv.astype(np.int64),
            "sub_crow": sub_crow}


def _empty_rows(g, count=500):
    rng = np.random.default_rng(7)
    cand = rng.integers(0, N, count * 2)
    return np.setdiff1d(cand, g["rows"])[:count]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rounded_spmm_past_32_bit_offsets(graph, dtype):
    from autosage_amd import _native

    d_crow = torch.from_numpy(graph["crow"]).cuda()
    d_col = torch.from_numpy(graph["col"]).cuda()
    d_val = torch.from_numpy(graph["val"]).to(dtype).cuda()
    x = _device_values(N, F, dtype)
    x_sub = torch.from_numpy(_values(graph["uniq"], F)).to(dtype)
    want = oracle.spmm_rounded_16(graph["sub_crow"], graph["sub_col"], torch.from_numpy(graph["val"]).to(dtype),
                                  x_sub, dtype)
    rows = torch.from_numpy(graph["rows"]).cuda()
    empty = torch.from_numpy(_empty_rows(graph)).cuda()
    for column_slices in (True, False):
        y = _native.spmm_rounded_16_impl(d_crow, d_col, d_val, x, column_slices=column_slices)
        got = y.index_select(0, rows).cpu()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), column_slices
        assert torch.count_nonzero(y.index_select(0, empty)).item() == 0
    del x


def test_colslice_fp32_past_32_bit_offsets(graph):
    d_crow = torch.from_numpy(graph["crow"]).cuda()
    d_col = torch.from_numpy(graph["col"]).cuda()
    d_val = torch.from_numpy(graph["val"]).cuda()
    x = _device_values(N, F, torch.float32)
    want = oracle.spmm_f64(graph["sub_crow"], graph["sub_col"], graph["val"], _values(graph["uniq"], F))
    y = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, x)
    got = y.index_select(0, torch.from_numpy(graph["rows"]).cuda()).cpu().numpy()
    assert np.array_equal(got, want.astype(np.float32))
    assert torch.count_nonzero(y.index_select(0, torch.from_numpy(_empty_rows(graph)).cuda())).item() == 0
    del x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rounded_sddmm_past_32_bit_offsets(graph, dtype):
    d_crow = torch.from_numpy(graph["crow"]).cuda()
    d_col = torch.from_numpy(graph["col"]).cuda()
    q = _device_values(N, F, dtype)
    k = q.flip(1).contiguous()
    q_sub = torch.from_numpy(_values(graph["rows"], F)).to(dtype)
    k_sub = torch.from_numpy(_values(graph["uniq"], F)[:, ::-1].copy()).to(dtype)
    want = oracle.sddmm_rounded_16(graph["sub_crow"], graph["sub_col"], q_sub, k_sub, dtype)
    for waves, threshold in ((4, 1024), (8, 2**31 - 1)):
        got = torch.ops.autosage.sddmm_csr_split(d_crow, d_col, q, k, waves, threshold).cpu()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (waves, threshold)
    del q, k


N_WIDE = (1 << 25) + 1000


def test_fslice_past_32_bit_offsets():
    """The feature-sliced SpMM on 2^25 + 1000 rows: the slice-major copy of X
    is then past 4 GiB (2^25 columns of 128 bytes per slice), so the kernel
    takes its 64-bit gather offsets.  1,000 rows hold edges (up to 2,500,
    columns over the whole range, above 2^25 included); exact values, so the
    rows with edges equal the sequential oracle on the compacted sub-graph bit
    for bit, weighted and not, and the other rows stay zero."""
    from autosage_amd import _native

    rng = np.random.default_rng(99)
    rows = np.sort(rng.choice(N_WIDE, size=1000, replace=False))
    deg = np.concatenate([rng.integers(1, 64, 700), rng.integers(64, 1024, 250), rng.integers(1024, 2500, 50)])
    rng.shuffle(deg)
    counts = np.zeros(N_WIDE, dtype=np.int64)
    counts[rows] = deg
    crow = np.zeros(N_WIDE + 1, dtype=np.int64)
    np.cumsum(counts, out=crow[1:])
    col = np.concatenate([np.sort(rng.choice(N_WIDE, size=d, replace=False)) for d in deg]).astype(np.int64)
    assert col.max() >= (1 << 25)
    val = rng.integers(-16, 17, col.size).astype(np.float32) / 8.0
    uniq, inv = np.unique(col, return_inverse=True)
    sub_crow = np.concatenate([[0], np.cumsum(counts[rows])]).astype(np.int64)
    features = 32
    lib = _native.library()
    assert lib.as_spmm_fslice_workspace_bytes(N_WIDE, features) > 0xFFFFFFFF
    d_crow, d_col, d_val = (torch.from_numpy(a).cuda() for a in (crow, col, val))
    del counts, crow
    x = _device_values(N_WIDE, features, torch.float32)
    x_sub = _values(uniq, features)
    d_rows = torch.from_numpy(rows).cuda()
    empty = torch.from_numpy(np.setdiff1d(rng.integers(0, N_WIDE, 1000), rows)).cuda()
    for weights, h_val in ((d_val, val), (None, None)):
        y = torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, weights, x)
        want = oracle.spmm_seq(sub_crow, inv.astype(np.int64), h_val, x_sub)
        got = y.index_select(0, d_rows).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), weights is None
        assert torch.count_nonzero(y.index_select(0, empty)).item() == 0
        del y
    del x
