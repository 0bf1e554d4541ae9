"""GPU parity of the column-sliced SpMM (``autosage::spmm_csr_colslice``).

The kernel accumulates each (row, column slice) partial in fp64 and adds the
partials in fp64 before one rounding, so it is checked against the CPU
oracle's fp64 product: |gpu - fp64| <= 1e-6·|fp64| + 1e-9 (tighter than the
1e-5 relative / 1e-6 absolute bar for fp32 results, which is asserted too).
It is deterministic: repeated and chunked calls give identical bits.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import _native, synth
from tests.gpu_common import case_graph, require_gpu, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _inputs(features, weighted, seed=0, rows=3000, degree=9, hubs=3, hub_degree=2500, empty=0.08):
    crow, col = case_graph(rows, degree, seed=seed, hubs=hubs, hub_degree=hub_degree, empty=empty)
    rng = np.random.default_rng(seed + 100)
    val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
    x = rng.standard_normal((rows, features)).astype(np.float32)
    return crow, col, val, x


def _assert_fp64_close(got: np.ndarray, exact: np.ndarray) -> None:
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= 1e-6 * np.abs(exact) + 1e-9), float(np.max(err - 1e-6 * np.abs(exact)))
    assert np.all(err <= 1e-5 * np.abs(exact) + 1e-6)


def _colslice(crow, col, val, x):
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    return torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x)


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [1, 3, 33, 64, 96, 128, 200, 256, 300])
def test_colslice_against_fp64(features, weighted):
    crow, col, val, x = _inputs(features, weighted, seed=features + 3 * weighted)
    got = _colslice(crow, col, val, x).cpu().numpy()
    _assert_fp64_close(got, oracle.spmm_f64(crow, col, val, x))
    # and against the reference's CPU result (torch.sparse.mm, restated
    # bit-exactly by the sequential oracle) at the reference's own GPU test
    # bar (tests/test_cuda.py:40 of the reference: rtol 1e-4, atol 3e-3)
    assert np.allclose(got, oracle.spmm_seq(crow, col, val, x), rtol=1e-4, atol=3e-3)


@pytest.mark.parametrize("features", [512, 1024, 1028])
def test_colslice_wide_features(features):
    # 4 / 8 / 9 feature tiles of 128 in one launch (1028: a partial last tile)
    crow, col, val, x = _inputs(features, True, seed=features, rows=1500, hub_degree=1200)
    got = _colslice(crow, col, val, x).cpu().numpy()
    _assert_fp64_close(got, oracle.spmm_f64(crow, col, val, x))


def test_colslice_long_slices_and_empty_rows():
    # hub rows of 20000 edges: about 2500 per slice, the U = 16 path
    crow, col, val, x = _inputs(128, True, seed=11, rows=24000, degree=4, hubs=4, hub_degree=20000, empty=0.3)
    assert np.diff(crow).max() == 20000 and (np.diff(crow) == 0).sum() > 1000
    got = _colslice(crow, col, val, x).cpu().numpy()
    _assert_fp64_close(got, oracle.spmm_f64(crow, col, val, x))
    assert np.all(got[np.diff(crow) == 0] == 0)


def test_colslice_edges_in_one_slice_and_tiny_graphs():
    # all columns of every row fall into the last slice
    rows = 64
    crow = np.arange(0, 3 * rows + 1, 3, dtype=np.int64)
    col = np.tile(np.array([61, 62, 63], dtype=np.int64), rows)
    x = np.random.default_rng(0).standard_normal((rows, 64)).astype(np.float32)
    got = _colslice(crow, col, None, x).cpu().numpy()
    _assert_fp64_close(got, oracle.spmm_f64(crow, col, None, x))
    # fewer rows than slices; and a graph without edges
    for n in (1, 2, 7):
        crow, col = case_graph(n, 2, seed=n)
        x = np.random.default_rng(n).standard_normal((n, 16)).astype(np.float32)
        _assert_fp64_close(_colslice(crow, col, None, x).cpu().numpy(), oracle.spmm_f64(crow, col, None, x))
    crow = np.zeros(11, dtype=np.int64)
    got = _colslice(crow, np.zeros(0, dtype=np.int64), None, np.ones((10, 8), np.float32))
    assert torch.count_nonzero(got).item() == 0


def test_colslice_deterministic_and_chunked(monkeypatch):
    crow, col, val, x = _inputs(128, True, seed=5)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    first = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x)
    again = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x)
    assert torch.equal(first, again)
    # a workspace for ~100 rows of partials (two buffers of ~50): about 55 chunks
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", str((100 * 128 * 64 + 200_000) / 2**20))
    chunked = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x)
    assert torch.equal(first, chunked)


@pytest.mark.parametrize("weighted", [False, True])
def test_colslice_unsorted_columns_run_row_sorted(weighted):
    """A graph whose columns do not ascend runs on its row-sorted copy: the
    same result as the op on the sorted graph (bit for bit: the same edges
    per row, sorted the same way) and the fp64 bar of the shuffled graph."""
    crow, col, val, x = _inputs(64, weighted, seed=9)
    rng = np.random.default_rng(90)
    perm = np.arange(col.size)
    for r in range(crow.size - 1):
        rng.shuffle(perm[crow[r]:crow[r + 1]])
    s_col = col[perm]
    s_val = None if val is None else val[perm]
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    d_scol = torch.from_numpy(s_col).cuda()
    d_sval = None if s_val is None else torch.from_numpy(s_val).cuda()
    assert _native.columns_ascending(d_crow, d_col)
    assert not _native.columns_ascending(d_crow, d_scol)
    # the row-sorted copy restores the sorted graph and its permutation
    sorted_col, p = _native.row_sorted(d_crow, d_scol)
    assert torch.equal(sorted_col, d_col)
    assert np.array_equal(s_col[p.cpu().numpy()], col)
    assert _native.row_sorted(d_crow, d_col)[1] is None
    got = torch.ops.autosage.spmm_csr_colslice(d_crow, d_scol, d_sval, d_x)
    assert torch.equal(got, torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x))
    _assert_fp64_close(got.cpu().numpy(), oracle.spmm_f64(crow, s_col, s_val, x))
    # memoised per graph: the second call reuses the sorted copy
    assert _native.row_sorted(d_crow, d_scol)[0] is sorted_col
    # new weights on the same graph are permuted afresh
    if d_sval is not None:
        d_sval.mul_(-2.0)
        again = torch.ops.autosage.spmm_csr_colslice(d_crow, d_scol, d_sval, d_x)
        _assert_fp64_close(again.cpu().numpy(), oracle.spmm_f64(crow, s_col, -2.0 * s_val, x))
    # equal neighbouring columns count as ascending
    crow2 = np.array([0, 3], dtype=np.int64)
    col2 = np.array([0, 0, 0], dtype=np.int64)
    assert _native.columns_ascending(*to_dev(crow2, col2))
    # the memo follows in-place changes of col
    d_col_copy = d_col.clone()
    assert _native.columns_ascending(d_crow, d_col_copy)
    row = int(np.argmax(np.diff(crow)))
    d_col_copy[crow[row]:crow[row + 1]] = d_col_copy[crow[row]:crow[row + 1]].flip(0)
    assert not _native.columns_ascending(d_crow, d_col_copy)


def test_row_sorted_memo_drops_dead_graphs():
    """Derived per-graph buffers go when the graph's tensors are collected."""
    import gc

    crow, col, _, x = _inputs(16, False, seed=4)
    d_crow = torch.from_numpy(crow).cuda()
    d_col = torch.from_numpy(np.concatenate([col[crow[r]:crow[r + 1]][::-1] for r in range(crow.size - 1)])).cuda()
    before = len(_native._ROW_SORTED_MEMO)
    _native.row_sorted(d_crow, d_col)
    assert len(_native._ROW_SORTED_MEMO) == before + 1
    del d_col
    gc.collect()
    assert len(_native._ROW_SORTED_MEMO) == before


def _grads(op, d_crow, d_col, d_val, d_x):
    v = d_val.clone().requires_grad_(True)
    xx = d_x.clone().requires_grad_(True)
    y = op(d_crow, d_col, v, xx)
    (y * torch.arange(d_x.size(1), device="cuda", dtype=torch.float32)).sum().backward()
    return v.grad, xx.grad


def test_colslice_backward(monkeypatch):
    """dX = Aᵀ·dY of the column-sliced op runs column-sliced over the
    transposed CSR (fp64 bound); dval is the bit-exact SDDMM; with column
    slices off both equal the exact op's gradients bit for bit."""
    from autosage_amd._autograd import csr_transpose

    crow, col, val, x = _inputs(64, True, seed=21)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    exact = _grads(torch.ops.autosage.spmm_csr, d_crow, d_col, d_val, d_x)
    sliced = _grads(torch.ops.autosage.spmm_csr_colslice, d_crow, d_col, d_val, d_x)
    assert torch.equal(sliced[0], exact[0])
    g = np.broadcast_to(np.arange(64, dtype=np.float32), x.shape)
    t_crow, t_col, perm = csr_transpose(torch.from_numpy(crow), torch.from_numpy(col))
    _assert_fp64_close(sliced[1].cpu().numpy(), oracle.spmm_f64(t_crow, t_col, val[perm.numpy()], g))
    assert torch.equal(sliced[1], _grads(torch.ops.autosage.spmm_csr_colslice, d_crow, d_col, d_val, d_x)[1])
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "off")
    off = _grads(torch.ops.autosage.spmm_csr_colslice, d_crow, d_col, d_val, d_x)
    assert torch.equal(off[0], exact[0]) and torch.equal(off[1], exact[1])


def test_colslice_skewed_config_rows():
    """A generated power-law graph (the structure of the benchmark graphs, at
    a smaller size): sampled rows against fp64 sums on the GPU."""
    crow, col = synth.random_csr(60000, 40, seed=3, hub_rows=20, hub_degree=30000)
    x = np.random.default_rng(3).standard_normal((60000, 128)).astype(np.float32)
    d_crow, d_col, d_x = to_dev(crow, col, x)
    got = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, d_x)
    rows = np.concatenate([np.argsort(-np.diff(crow))[:20], np.random.default_rng(4).choice(60000, 500, False)])
    x64 = d_x.double()
    for r in rows.tolist():
        exact = x64.index_select(0, d_col[crow[r]:crow[r + 1]]).sum(0).cpu().numpy()
        _assert_fp64_close(got[r].cpu().numpy(), exact)


def _timed(info) -> list:
    return [c["candidate"] for c in info.get("full_graph", {}).get("candidates", [])]


def test_scheduler_times_colslice_on_the_full_graph(monkeypatch, tmp_path):
    import autosage_amd

    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "on")
    crow, col, val, x = _inputs(64, False, seed=31, rows=6000, degree=30)
    d_crow, d_col, _, d_x = to_dev(crow, col, None, x)
    out, info = autosage_amd.spmm_csr_auto(d_crow, d_col, None, d_x)
    assert "colslice" in _timed(info) and None in _timed(info)
    assert all(c["best_ms"] > 0 for c in info["full_graph"]["candidates"])
    exact = oracle.spmm_f64(crow, col, None, x)
    if info["candidate"] == "colslice":
        _assert_fp64_close(out.cpu().numpy(), exact)
    elif info["choice"] == "autosage":
        assert np.array_equal(out.cpu().numpy(), oracle.spmm_seq(crow, col, None, x))
    again, cached = autosage_amd.spmm_csr_auto(d_crow, d_col, None, d_x)
    assert cached["from_cache"] and cached["candidate"] == info["candidate"]
    assert torch.equal(again, out)
    # a graph whose columns are not ascending: its schedule key equals the
    # sorted graph's (the key hashes only the ends of col) ...
    shuffled = col.copy()
    r = int(np.argmax(np.diff(crow)))
    assert 2048 < crow[r] and crow[r + 1] < col.size - 2048
    shuffled[crow[r]:crow[r + 1]] = shuffled[crow[r]:crow[r + 1]][::-1]
    d_shuffled = torch.from_numpy(shuffled).cuda()
    replayed, info_r = autosage_amd.spmm_csr_auto(d_crow, d_shuffled, None, d_x)
    assert info_r["from_cache"]
    if info_r["candidate"] == "colslice":
        # ... so a cached column-sliced choice runs on its row-sorted copy
        _assert_fp64_close(replayed.cpu().numpy(), oracle.spmm_f64(crow, shuffled, None, x))
    # ... and without a cache record it is timed with column slices too
    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path / "second"))
    out2, info2 = autosage_amd.spmm_csr_auto(d_crow, d_shuffled, None, d_x)
    assert "colslice" in _timed(info2)
    if info2["candidate"] == "colslice":
        _assert_fp64_close(out2.cpu().numpy(), oracle.spmm_f64(crow, shuffled, None, x))
    # off: never timed
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "off")
    _, info3 = autosage_amd.spmm_csr_auto(d_crow, d_col, None, d_x)
    assert "colslice" not in _timed(info3) and info3.get("candidate") != "colslice"


def test_sliced_rows_hint_only_sizes_the_launches():
    """The sliced-row count passed through the C ABI sizes the launches; any
    value (unknown, zero, too small, exact, too large) gives the same bits."""
    crow, col, val, x = _inputs(128, True, seed=21, rows=9000, degree=20, hubs=40, hub_degree=3000)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    n, f = x.shape
    lib = _native.library()
    exact = _native.sliced_rows(d_crow, True, f, torch.float32)
    assert exact == int((np.diff(crow) >= lib.as_spmm_colslice_min_degree(1, f, 0)).sum()) and exact >= 40
    ws = torch.empty(lib.as_spmm_colslice_workspace_bytes(n, f), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for hint in (-1, 0, 1, exact // 2, exact, exact * 1000):
        y = torch.empty_like(d_x)
        status = lib.as_spmm_csr_colslice_f32(d_crow.data_ptr(), d_col.data_ptr(), d_val.data_ptr(), d_x.data_ptr(),
                                              y.data_ptr(), n, col.size, f, ws.data_ptr(), ws.numel(), hint, stream)
        assert status == 0, lib.as_last_error()
        outs.append(y)
    torch.cuda.synchronize()
    for y in outs[1:]:
        assert torch.equal(y, outs[0])
    # 16-bit features, column and edge slices (thresholds 512 and 1024), with
    # the count of grouped short rows (degree below 64 for F = 128) too
    xb = d_x.to(torch.bfloat16)
    limit = lib.as_spmm_rounded_16_group_degree(f)
    assert limit == 64
    for column_slices in (1, 0):
        sliced, grouped = _native.row_counts(d_crow, lib.as_spmm_colslice_min_degree(column_slices, f, 1), limit)
        assert grouped == int((np.diff(crow) < limit).sum()) and 0 < grouped < n
        outs = []
        for hints in ((-1, -1), (0, 0), (sliced, grouped), (sliced + 500, n), (sliced, 0), (1, 3 * n), (-1, grouped)):
            y = torch.empty_like(xb)
            status = lib.as_spmm_csr_rounded_16(d_crow.data_ptr(), d_col.data_ptr(), 0, xb.data_ptr(), y.data_ptr(),
                                                n, col.size, f, 1, column_slices, ws.data_ptr(), ws.numel(), *hints,
                                                stream)
            assert status == 0, lib.as_last_error()
            outs.append(y)
        torch.cuda.synchronize()
        for y in outs[1:]:
            assert torch.equal(y, outs[0])
        # partial buffers for 1 row, half the sliced rows and all of them: the
        # sliced rows past the capacity are summed whole, with the same bits
        fixed = lib.as_spmm_rounded_16_workspace_bytes(n, f, 0) - 2 * 8 * f * 8
        for rows in (1, max(sliced // 2, 1), sliced):
            small = torch.empty(fixed + 2 * rows * 8 * f * 8, dtype=torch.uint8, device="cuda")
            assert lib.as_spmm_rounded_16_workspace_bytes(n, f, rows) == small.numel()
            y = torch.empty_like(xb)
            status = lib.as_spmm_csr_rounded_16(d_crow.data_ptr(), d_col.data_ptr(), 0, xb.data_ptr(), y.data_ptr(),
                                                n, col.size, f, 1, column_slices, small.data_ptr(), small.numel(),
                                                sliced, grouped, stream)
            assert status == 0, lib.as_last_error()
            torch.cuda.synchronize()
            assert torch.equal(y, outs[0]), rows


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_planned_calls_match_unplanned(dtype, monkeypatch):
    """A plan (slice points and binned row order, built once per graph)
    gives the bits of a call that builds them itself: fp32 and 16-bit, F of
    either fp32 slicing degree (256 at F = 64, 128 above), column and edge
    slices, a short partial workspace; a plan is built per (graph, settings),
    and it goes with the graph."""
    import gc

    crow, col, val, x = _inputs(128, True, seed=31, rows=9000, degree=20, hubs=40, hub_degree=3000)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    d_val, d_x = d_val.to(dtype), d_x.to(dtype)
    before = len(_native._PLAN_MEMO)
    for f in (64, 128):
        xf = d_x[:, :f].contiguous()
        modes = [True] if dtype == torch.float32 else [True, False]
        for column_slices in modes:
            if dtype == torch.float32:
                planned = _native.spmm_csr_colslice_impl(d_crow, d_col, d_val, xf)
            else:
                planned = _native.spmm_rounded_16_impl(d_crow, d_col, d_val, xf, column_slices)
            monkeypatch.setenv("AUTOSAGE_COLSLICE_PLAN", "off")
            if dtype == torch.float32:
                unplanned = _native.spmm_csr_colslice_impl(d_crow, d_col, d_val, xf)
            else:
                unplanned = _native.spmm_rounded_16_impl(d_crow, d_col, d_val, xf, column_slices)
            monkeypatch.delenv("AUTOSAGE_COLSLICE_PLAN")
            assert torch.equal(planned, unplanned), (f, column_slices)
            # a short workspace (partials for ~40 rows) with the same plan: more chunks, same bits
            plan_bytes = _native.library().as_spmm_colslice_plan_bytes(crow.size - 1)
            monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", str((plan_bytes + 40 * 8 * f * 8) / 2**20))
            if dtype == torch.float32:
                short = _native.spmm_csr_colslice_impl(d_crow, d_col, d_val, xf)
            else:
                short = _native.spmm_rounded_16_impl(d_crow, d_col, d_val, xf, column_slices)
            monkeypatch.delenv("AUTOSAGE_COLSLICE_WORKSPACE_MB")
            assert torch.equal(short, planned)
    if dtype == torch.float32:
        _assert_fp64_close(planned.cpu().numpy(), oracle.spmm_f64(crow, col, val, x[:, :128]))
    # fp32 slices from 256 at F = 64 and 128 at F = 128: two plans; 16-bit:
    # column slices from 128 at both F, edge slices from 1024: two plans
    assert len(_native._PLAN_MEMO) == before + 2
    del d_col
    gc.collect()
    assert len(_native._PLAN_MEMO) == before


def test_planned_call_rejects_a_plan_of_other_settings():
    crow, col, val, x = _inputs(64, False, seed=32, rows=2000)
    d_crow, d_col, d_x = to_dev(crow, col, x)
    lib = _native.library()
    n, f = x.shape
    plan64, tag64 = _native.colslice_plan(d_crow, d_col, 64, torch.float32, True)
    _, tag128 = _native.colslice_plan(d_crow, d_col, 128, torch.float32, True)
    assert tag64 != tag128
    y = torch.empty_like(d_x)
    ws = torch.empty(lib.as_spmm_colslice_planned_workspace_bytes(n, col.size, f, 0, -1), dtype=torch.uint8,
                     device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    args = (d_crow.data_ptr(), d_col.data_ptr(), 0, d_x.data_ptr(), y.data_ptr(), n, col.size, f, 0, 1,
            plan64.data_ptr(), plan64.numel())
    assert lib.as_spmm_csr_colslice_planned(*args, tag128, ws.data_ptr(), ws.numel(), -1, 0, stream) == 1
    assert lib.as_last_error().startswith(b"the plan was built for other settings")
    assert lib.as_spmm_csr_colslice_planned(*args, tag64, ws.data_ptr(), ws.numel(), -1, 0, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(y, _native.spmm_csr_colslice_impl(d_crow, d_col, None, d_x))


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [64, 128, 256, 33])
def test_colslice_cooperative_hub_rows(features, weighted, monkeypatch):
    """Rows of degree >= 2^6 times the slicing degree (8,192 edges at 128,
    16,384 at 256 for F <= 64) run each (row, slice) on all waves of a
    workgroup, their fp64 sums added in wave order: within the fp64 bound,
    deterministic, and the same bits with a short workspace (many chunks) and
    without the per-graph plan.  F = 33 (narrow lanes) keeps one wave per
    (row, slice)."""
    crow, col, val, x = _inputs(features, weighted, seed=features + 40, rows=30000, degree=3, hubs=6,
                                hub_degree=24000, empty=0.2)
    deg = np.diff(crow)
    assert (deg >= 16384).sum() == 6 and deg[deg < 24000].max() < 100
    d = to_dev(crow, col, val, x)
    first = torch.ops.autosage.spmm_csr_colslice(*d)
    _assert_fp64_close(first.cpu().numpy(), oracle.spmm_f64(crow, col, val, x))
    assert torch.equal(first, torch.ops.autosage.spmm_csr_colslice(*d))
    monkeypatch.setenv("AUTOSAGE_COLSLICE_PLAN", "off")
    assert torch.equal(first, torch.ops.autosage.spmm_csr_colslice(*d))
    monkeypatch.delenv("AUTOSAGE_COLSLICE_PLAN")
    # partial rows for two sliced rows at a time
    plan_bytes = _native.library().as_spmm_colslice_plan_bytes(crow.size - 1)
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", str((plan_bytes + 4 * 8 * features * 8) / 2**20))
    assert torch.equal(first, torch.ops.autosage.spmm_csr_colslice(*d))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rounded16_cooperative_hub_rows(dtype):
    """16-bit features with column slices (slicing degree 512, so rows of
    32,768 edges and more cooperate): the cooperative hub rows give the bits
    of the rounded fp64 oracle."""
    n = 50000
    crow, col = case_graph(n, 3, seed=41, hubs=4, hub_degree=40000, empty=0.2)
    assert np.diff(crow).max() >= 512 * 64
    rng = np.random.default_rng(42)
    x = torch.from_numpy(rng.standard_normal((n, 128)).astype(np.float32)).to(dtype)
    val = torch.from_numpy(rng.standard_normal(col.size).astype(np.float32)).to(dtype)
    want = oracle.spmm_rounded_16(crow, col, val, x, dtype)
    d_crow, d_col = to_dev(crow, col)
    got = _native.spmm_rounded_16_impl(d_crow, d_col, val.cuda(), x.cuda(), column_slices=True)
    assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [64, 128, 33])
def test_colslice_row_blocks(features, weighted, monkeypatch):
    """fp32 graphs of at least 65,536 rows run as row blocks (each with its
    own binned order): within the fp64 bound, and the same bits as the
    per-call plan, as row shards of one block each (``autosage_amd.shard``)
    and as a short workspace (several chunks per block).  Hub rows of 9,000
    edges take the cooperative form (graphs of at most 2^24 edges)."""
    from autosage_amd import shard

    rows = 140_000
    crow, col, val, x = _inputs(features, weighted, seed=features + 60, rows=rows, degree=6, hubs=5,
                                hub_degree=9000, empty=0.1)
    d = to_dev(crow, col, val, x)
    first = torch.ops.autosage.spmm_csr_colslice(*d)
    _assert_fp64_close(first.cpu().numpy(), oracle.spmm_f64(crow, col, val, x))
    pieces = []
    cuts = shard.cut_rows(d[0], 3)
    for r0, r1 in zip(cuts, cuts[1:]):
        s_crow, s_col, s_val = shard.shard_csr(d[0], d[1], d[2], r0, r1)
        pieces.append(shard.spmm_csr_shard(s_crow, s_col, s_val, d[3]))
    assert torch.equal(first, torch.cat(pieces))
    monkeypatch.setenv("AUTOSAGE_COLSLICE_PLAN", "off")
    assert torch.equal(first, torch.ops.autosage.spmm_csr_colslice(*d))
    monkeypatch.delenv("AUTOSAGE_COLSLICE_PLAN")
    plan_bytes = _native.library().as_spmm_colslice_plan_bytes(rows)
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", str((plan_bytes + 2 * 3000 * 8 * features * 8) / 2**20))
    assert torch.equal(first, torch.ops.autosage.spmm_csr_colslice(*d))


@pytest.mark.parametrize("features", [300, 128, 64])
def test_colslice_row_blocks_with_empty_blocks_and_feature_tiles(features):
    """Row blocks of a graph whose middle rows have no edges at all (two of
    its four blocks empty, the others holding hub rows and short rows), at a
    width of several feature tiles (F = 300: three tiles of 128) and at one
    (F = 128; F = 64, where the blocks run as one pipeline): within the fp64
    bound, the empty rows zero, and the same bits as the
    graph's row shards (one block each)."""
    from autosage_amd import shard

    rows = 140_000
    crow, col, val, x = _inputs(features, True, seed=features + 70, rows=rows, degree=7, hubs=4,
                                hub_degree=5000, empty=0.05)
    deg = np.diff(crow)
    deg[rows // 4: 3 * rows // 4] = 0  # blocks 1 and 2 of 4 hold no edge
    keep = np.concatenate([np.arange(crow[r], crow[r + 1]) for r in range(rows) if deg[r] > 0])
    new_crow = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    col, val = col[keep], val[keep]
    assert new_crow[-1] == col.size
    d = to_dev(new_crow, col, val, x)
    got = torch.ops.autosage.spmm_csr_colslice(*d)
    host = got.cpu().numpy()
    _assert_fp64_close(host, oracle.spmm_f64(new_crow, col, val, x))
    assert not host[rows // 4: 3 * rows // 4].any()
    cuts = [0, rows // 3, 2 * rows // 3, rows]
    pieces = []
    for r0, r1 in zip(cuts, cuts[1:]):
        s_crow, s_col, s_val = shard.shard_csr(d[0], d[1], d[2], r0, r1)
        pieces.append(shard.spmm_csr_shard(s_crow, s_col, s_val, d[3]))
    assert torch.equal(got, torch.cat(pieces))


def test_row_sorted_weights_follow_an_in_place_change_of_crow():
    """A weighted graph whose columns do not ascend runs on its row-sorted
    copy with the weights permuted the same way.  When crow changes in place
    (same col and val objects, new row boundaries) the permutation changes,
    and the permuted weights must follow it."""
    rng = np.random.default_rng(51)
    rows, f = 400, 32
    crow = np.concatenate([[0], np.cumsum(rng.integers(0, 30, size=rows))]).astype(np.int64)
    nnz = int(crow[-1])
    col = rng.integers(0, rows, size=nnz).astype(np.int64)  # unsorted, duplicates allowed
    val = rng.standard_normal(nnz).astype(np.float32)
    x = rng.standard_normal((rows, f)).astype(np.float32)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    first = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x).cpu().numpy()
    _assert_fp64_close(first, oracle.spmm_f64(crow, col, val, x))
    # new row boundaries over the same edges
    crow2 = np.concatenate([[0], np.sort(rng.integers(0, nnz + 1, size=rows - 1)), [nnz]]).astype(np.int64)
    d_crow.copy_(torch.from_numpy(crow2))
    second = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x).cpu().numpy()
    _assert_fp64_close(second, oracle.spmm_f64(crow2, col, val, x))


@pytest.mark.parametrize("features", [64, 128, 200])
def test_fp32_partial_buffers_smaller_than_the_sliced_rows(features):
    """fp32 with a workspace sized below a block's sliced rows (a graph of more
    than 2^24 edges, so no cooperative rows): the sliced rows past the
    capacity are summed one wave each with the sliced rows' own arithmetic,
    so every workspace size gives the bits of the full one, weighted or not."""
    rows = 120_000
    crow, col = case_graph(rows, 150, seed=features, hubs=30, hub_degree=20_000, empty=0.02)
    assert col.size > (1 << 24)
    rng = np.random.default_rng(features)
    val = rng.standard_normal(col.size).astype(np.float32)
    x = rng.standard_normal((rows, features)).astype(np.float32)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    n, f = x.shape
    lib = _native.library()
    stream = torch.cuda.current_stream().cuda_stream
    plan, tag = _native.colslice_plan(d_crow, d_col, f, torch.float32, True)
    most = _native.block_sliced_rows(d_crow, f, torch.float32, True)
    degree = lib.as_spmm_colslice_min_degree(1, f, 0)
    begins = (ctypes.c_int64 * 65)()
    blocks = lib.as_spmm_colslice_row_blocks(n, 0, begins, 65)
    want_most = max(int((np.diff(crow)[begins[b]:begins[b + 1]] >= degree).sum()) for b in range(blocks))
    assert blocks >= 2 and most == want_most
    row_bytes = lib.as_spmm_colslice_planned_workspace_bytes(n, col.size, f, 0, 1) // 2
    sliced, grouped = _native.colslice_row_counts(d_crow, f, torch.float32)
    for weights in (None, d_val):
        outs = []
        for rows_per_buffer in (-1, most, most // 3, 1):
            ws_bytes = (lib.as_spmm_colslice_planned_workspace_bytes(n, col.size, f, 0, -1) if rows_per_buffer < 0
                        else 2 * rows_per_buffer * row_bytes)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
            y = torch.empty_like(d_x)
            status = lib.as_spmm_csr_colslice_planned(
                d_crow.data_ptr(), d_col.data_ptr(), None if weights is None else weights.data_ptr(), d_x.data_ptr(),
                y.data_ptr(), n, col.size, f, 0, 1, plan.data_ptr(), plan.numel(), tag, ws.data_ptr(), ws.numel(),
                sliced, grouped, stream)
            assert status == 0, lib.as_last_error()
            outs.append(y)
        torch.cuda.synchronize()
        for y in outs[1:]:
            assert torch.equal(y, outs[0])
        picked = np.concatenate([np.argsort(-np.diff(crow))[:6], rng.choice(rows, 300, replace=False)])
        exact = oracle.spmm_f64(crow, col, None if weights is None else val, x, rows=picked)
        _assert_fp64_close(outs[-1][torch.from_numpy(picked).cuda()].cpu().numpy(), exact)
    # the op sizes its workspace for the sliced rows of the largest block (a
    # block's rows at most)
    block_rows = max(begins[b + 1] - begins[b] for b in range(blocks))
    assert lib.as_spmm_colslice_planned_workspace_bytes(n, col.size, f, 0, -1) >= 2 * block_rows * row_bytes
    capped = lib.as_spmm_colslice_planned_workspace_bytes(n, col.size, f, 0, most)
    if f % 4 == 0:
        assert capped == 2 * min(most, block_rows) * row_bytes
    else:
        # narrow lanes cut chunks to the buffers: a block's rows, not its sliced rows
        assert capped >= 2 * block_rows * row_bytes


def test_few_sliced_rows_keep_one_chunk():
    """The reference hub sweep's graph (20,000 rows, one of 12,000 edges, the
    rest of 32; 652k edges, so cooperative hub rows): the op sizes its fp32
    partial buffers for a chunk's rows, not for its one sliced row, so the
    graph runs as one chunk (buffers of one row would cut it into 20,000
    one-row launches, about 150 ms).  Within 1e-6 of fp64, and well under a
    millisecond per call."""
    from autosage_amd import synth

    d_crow, d_col = synth.hub_sweep_graph()
    rows = d_crow.numel() - 1
    x = torch.randn(rows, 128, device="cuda")
    y = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, x)
    h_crow, h_col = d_crow.cpu().numpy(), d_col.cpu().numpy()
    _assert_fp64_close(y.cpu().numpy(), oracle.spmm_f64(h_crow, h_col, None, x.cpu().numpy()))
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(5):
        torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, x)
    end.record()
    end.synchronize()
    per_call = start.elapsed_time(end) / 5
    print(f"[colslice] hub sweep graph: {per_call:.4f} ms per call", flush=True)
    assert per_call < 5.0, per_call
