"""GPU parity of the feature-sliced SpMM (``autosage::spmm_csr_fslice``).

Every output element is one fp32 chain over its row's edges in CSR order, so
the result must equal the sequential CPU oracle (``oracle.spmm_seq``, the
reference's CPU ``torch.sparse.mm`` restated bit for bit) in every bit, for
any F (slices of 32 features, a partial last slice, 1 to 1028 features), with
or without weights, for empty rows, hub rows longer than any unrolled batch,
misaligned X or Y, row shards (n × n_cols) and graphs without edges.
"""

from __future__ import annotations

import ctypes
import json

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import _native
from tests.gpu_common import bitwise_equal, case_graph, mismatch_report, require_gpu, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _inputs(features, weighted, seed=0, rows=3000, degree=9, hubs=3, hub_degree=2500, empty=0.08):
    crow, col = case_graph(rows, degree, seed=seed, hubs=hubs, hub_degree=hub_degree, empty=empty)
    rng = np.random.default_rng(seed + 7)
    val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
    x = rng.standard_normal((rows, features)).astype(np.float32)
    return crow, col, val, x


def _fslice(crow, col, val, x):
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    return torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, d_val, d_x)


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [1, 3, 4, 31, 32, 33, 64, 96, 100, 128, 160, 256, 300, 520])
def test_fslice_bitwise_equals_sequential_oracle(features, weighted):
    crow, col, val, x = _inputs(features, weighted, seed=features + 5 * weighted)
    print(f"[fslice] F={features} weighted={weighted}", flush=True)
    got = _fslice(crow, col, val, x)
    want = oracle.spmm_seq(crow, col, val, x)
    assert bitwise_equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("features", [1028, 1536])
def test_fslice_more_than_eight_slices(features):
    # 33 / 48 slices: each XCD works its slices one after the other
    crow, col, val, x = _inputs(features, True, seed=features, rows=1200, hub_degree=900)
    got = _fslice(crow, col, val, x)
    want = oracle.spmm_seq(crow, col, val, x)
    assert bitwise_equal(got, want), mismatch_report(got, want)


def test_fslice_long_rows_and_empty_rows():
    # rows of 20000 edges (500 unrolled batches of 40) next to a third of empty rows
    crow, col, val, x = _inputs(128, True, seed=11, rows=24000, degree=4, hubs=4, hub_degree=20000, empty=0.3)
    deg = np.diff(crow)
    assert deg.max() == 20000 and (deg == 0).sum() > 1000
    got = _fslice(crow, col, val, x)
    want = oracle.spmm_seq(crow, col, val, x)
    assert bitwise_equal(got, want), mismatch_report(got, want)
    assert np.all(got.cpu().numpy()[deg == 0] == 0)


def test_fslice_every_degree_from_zero_to_ninety():
    # one row of each degree 0..90 (twice, shuffled): every mask pattern of
    # the unmasked / masked / skipped batches of 40 and groups of 8
    rng = np.random.default_rng(3)
    deg = rng.permutation(np.concatenate([np.arange(91), np.arange(91)])).astype(np.int64)
    rows = deg.size
    crow = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(deg, out=crow[1:])
    col = np.concatenate([np.sort(rng.choice(rows, size=d, replace=False)) for d in deg]).astype(np.int64)
    for weighted in (False, True):
        val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
        x = rng.standard_normal((rows, 40)).astype(np.float32)
        got = _fslice(crow, col, val, x)
        want = oracle.spmm_seq(crow, col, val, x)
        assert bitwise_equal(got, want), mismatch_report(got, want)


def test_fslice_special_values_keep_their_bits():
    # inf, nan, signed zeros and subnormals go through the same fp32 chain
    crow, col, val, x = _inputs(64, True, seed=21, rows=500, hubs=1, hub_degree=400)
    x[::7, ::3] = np.inf
    x[::11, 1::5] = -0.0
    x[::13, 2::9] = np.float32(1e-42)
    val[::17] = -0.0
    got = _fslice(crow, col, val, x).cpu().numpy()
    want = oracle.spmm_seq(crow, col, val, x)
    nan_got, nan_want = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_got, nan_want)
    assert np.array_equal(got[~nan_got].view(np.uint32), want[~nan_want].view(np.uint32))


def test_fslice_misaligned_features_and_output():
    crow, col, val, x = _inputs(64, True, seed=5, rows=800)
    d_crow, d_col, d_val = to_dev(crow, col, val)
    flat = torch.empty(x.size + 1, device="cuda")
    d_x = flat[1:].view(x.shape)
    d_x.copy_(torch.from_numpy(x))
    assert d_x.data_ptr() % 16 != 0
    got = torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, d_val, d_x)
    want = oracle.spmm_seq(crow, col, val, x)
    assert bitwise_equal(got, want), mismatch_report(got, want)
    # the C entry with a misaligned Y
    n, f = x.shape
    plan, tag = _native.fslice_plan(d_crow, d_col, n)
    lib = _native.library()
    ws = torch.empty(lib.as_spmm_fslice_workspace_bytes(n, f), dtype=torch.uint8, device="cuda")
    y_flat = torch.empty(n * f + 1, device="cuda")
    y = y_flat[1:].view(n, f)
    status = lib.as_spmm_csr_fslice_f32(d_crow.data_ptr(), d_val.data_ptr(), d_x.data_ptr(), y.data_ptr(), n, n,
                                        col.size, f, plan.data_ptr(), plan.numel(), tag, ws.data_ptr(), ws.numel(),
                                        torch.cuda.current_stream().cuda_stream)
    assert status == 0, lib.as_last_error()
    assert bitwise_equal(y, want), mismatch_report(y, want)


def test_fslice_graph_without_edges_and_single_rows():
    for rows in (1, 2, 65):
        crow = np.zeros(rows + 1, dtype=np.int64)
        col = np.zeros(0, dtype=np.int64)
        x = np.random.default_rng(rows).standard_normal((rows, 48)).astype(np.float32)
        for val in (None, np.zeros(0, dtype=np.float32)):
            got = _fslice(crow, col, val, x)
            assert torch.equal(got, torch.zeros_like(got))
    crow = np.array([0, 3], dtype=np.int64)
    col = np.array([0, 0, 0], dtype=np.int64)
    x = np.array([[0.1, -2.5, 3.0]], dtype=np.float32)
    val = np.array([1.5, -0.25, 2.0], dtype=np.float32)
    got = _fslice(crow, col, val, x)
    assert bitwise_equal(got, oracle.spmm_seq(crow, col, val, x))


def test_fslice_row_shard_against_whole_x():
    # an n × n_cols CSR: the rows [r0, r1) of a graph with crow rebased, X whole
    crow, col, val, x = _inputs(128, True, seed=9, rows=4000, hubs=2, hub_degree=3000)
    r0, r1 = 1000, 2600
    s_crow = crow[r0:r1 + 1] - crow[r0]
    s_col = col[crow[r0]:crow[r1]]
    s_val = val[crow[r0]:crow[r1]]
    d_crow, d_col, d_val, d_x = to_dev(s_crow, s_col, s_val, x)
    got = _native._spmm_fslice(d_crow, d_col, d_val, d_x, r1 - r0)
    want = oracle.spmm_seq(crow, col, val, x)[r0:r1]
    assert bitwise_equal(got, want), mismatch_report(got, want)


def test_fslice_plan_is_reused_and_rebuilt_on_change():
    crow, col, val, x = _inputs(96, False, seed=13, rows=2000)
    d_crow, d_col, d_x = to_dev(crow, col, x)
    first = torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, None, d_x)
    plan_a, _ = _native.fslice_plan(d_crow, d_col, crow.size - 1)
    x2 = np.random.default_rng(1).standard_normal(x.shape).astype(np.float32)
    second = torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, None, torch.from_numpy(x2).cuda())
    plan_b, _ = _native.fslice_plan(d_crow, d_col, crow.size - 1)
    assert plan_a.data_ptr() == plan_b.data_ptr()
    assert bitwise_equal(first, oracle.spmm_seq(crow, col, None, x))
    assert bitwise_equal(second, oracle.spmm_seq(crow, col, None, x2))
    # an in-place change of the columns misses the memo and rebuilds the plan
    col2 = col.copy()
    col2[: col.size // 2] = (col2[: col.size // 2] * 7 + 1) % (crow.size - 1)
    d_col.copy_(torch.from_numpy(col2))
    third = torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, None, d_x)
    assert bitwise_equal(third, oracle.spmm_seq(crow, col2, None, x))


def test_fslice_plan_order_is_the_stable_degree_sort():
    crow, col, _, _ = _inputs(32, False, seed=17, rows=5000, empty=0.2)
    d_crow, d_col = to_dev(crow, col)
    n = crow.size - 1
    plan, _ = _native.fslice_plan(d_crow, d_col, n)
    order = plan[256:256 + 4 * n].view(torch.int32).cpu().numpy()
    deg = np.diff(crow)
    assert np.array_equal(order, np.argsort(-deg, kind="stable"))
    assert int(plan[:4].view(torch.int32).item()) == 0


def test_fslice_out_of_range_column_is_refused():
    crow, col, _, x = _inputs(32, False, seed=19, rows=600)
    bad = col.copy()
    bad[5] = crow.size - 1  # == n: out of range
    with pytest.raises(RuntimeError, match=r"col values must be in \[0, 600\)"):
        _fslice(crow, bad, None, x)
    bad[5] = -1
    with pytest.raises(RuntimeError, match="col values must be in"):
        _fslice(crow, bad, None, x)


def test_fslice_c_abi_checks():
    crow, col, val, x = _inputs(64, False, seed=23, rows=700)
    d_crow, d_col, d_x = to_dev(crow, col, x)
    n, f = x.shape
    lib = _native.library()
    plan, tag = _native.fslice_plan(d_crow, d_col, n)
    ws = torch.empty(lib.as_spmm_fslice_workspace_bytes(n, f), dtype=torch.uint8, device="cuda")
    y = torch.empty(n, f, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def call(plan_bytes=plan.numel(), plan_tag=tag, ws_bytes=ws.numel()):
        return lib.as_spmm_csr_fslice_f32(d_crow.data_ptr(), None, d_x.data_ptr(), y.data_ptr(), n, n, col.size, f,
                                          plan.data_ptr(), plan_bytes, plan_tag, ws.data_ptr(), ws_bytes, stream)

    assert call(plan_tag=tag + 1) == 1 and b"not a feature-sliced plan" in lib.as_last_error()
    assert call(plan_bytes=plan.numel() - 1) == 1 and b"too small" in lib.as_last_error()
    assert call(ws_bytes=ws.numel() - 1) == 4 and b"workspace" in lib.as_last_error()
    assert call() == 0
    assert bitwise_equal(y, oracle.spmm_seq(crow, col, None, x))
    # the plan builder refuses short buffers before launching anything
    tag_out = ctypes.c_int64(0)
    scratch = torch.empty(lib.as_spmm_fslice_plan_workspace_bytes(n), dtype=torch.uint8, device="cuda")
    status = lib.as_spmm_fslice_plan(d_crow.data_ptr(), d_col.data_ptr(), n, n, col.size, 1, plan.data_ptr(),
                                     plan.numel() - 1, scratch.data_ptr(), scratch.numel(), ctypes.byref(tag_out),
                                     stream)
    assert status == 4 and tag_out.value == 0
    for phases in (0, 9):
        status = lib.as_spmm_fslice_plan(d_crow.data_ptr(), d_col.data_ptr(), n, n, col.size, phases,
                                         plan.data_ptr(), plan.numel(), scratch.data_ptr(), scratch.numel(),
                                         ctypes.byref(tag_out), stream)
        assert status == 1 and b"phases must be in [1, 8]" in lib.as_last_error()
    assert lib.as_spmm_fslice_plan_bytes(n, col.size, 0) == 0
    # the tag carries the phase count: a one-phase plan under a two-phase tag is too small
    plan_bytes_2 = lib.as_spmm_fslice_plan_bytes(n, col.size, 2)
    assert plan_bytes_2 > lib.as_spmm_fslice_plan_bytes(n, col.size, 1)
    two_phase_tag = (tag & ~(0xFF << 8)) | (2 << 8)
    assert call(plan_tag=two_phase_tag) == 1 and b"too small" in lib.as_last_error()


def _timed(info) -> dict:
    return {json.dumps(c["candidate"]): c["best_ms"] for c in info.get("full_graph", {}).get("candidates", [])}


def test_scheduler_times_feature_slices_and_prefers_exact(monkeypatch, tmp_path):
    import autosage_amd
    from autosage_amd import _auto

    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    monkeypatch.setenv("AUTOSAGE_FEATURE_SLICES", "on")
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "on")
    crow, col, val, x = _inputs(128, True, seed=41, rows=8000, degree=40, hubs=6, hub_degree=4000)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    out, info = autosage_amd.spmm_csr_auto(d_crow, d_col, d_val, d_x)
    timed = _timed(info)
    assert '"fslice"' in timed and '"colslice"' in timed and "null" in timed, timed
    exact_best = min(t for k, t in timed.items() if k != '"colslice"')
    if info["candidate"] == "colslice":
        # the reassociating schedule only when it beats every exact one by the margin
        assert timed['"colslice"'] * (1.0 + _auto._INEXACT_MARGIN) < exact_best
    else:
        assert info["choice"] == "autosage"
        assert bitwise_equal(out, oracle.spmm_seq(crow, col, val, x))
    again, cached = autosage_amd.spmm_csr_auto(d_crow, d_col, d_val, d_x)
    assert cached["from_cache"] and cached["candidate"] == info["candidate"] and torch.equal(again, out)
    # off: never timed; column slices off keeps the feature slices (exact)
    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path / "b"))
    monkeypatch.setenv("AUTOSAGE_FEATURE_SLICES", "off")
    _, info_off = autosage_amd.spmm_csr_auto(d_crow, d_col, d_val, d_x)
    assert '"fslice"' not in _timed(info_off)
    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path / "c"))
    monkeypatch.setenv("AUTOSAGE_FEATURE_SLICES", "on")
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "off")
    out_exact, info_exact = autosage_amd.spmm_csr_auto(d_crow, d_col, d_val, d_x)
    assert '"fslice"' in _timed(info_exact) and '"colslice"' not in _timed(info_exact)
    if info_exact["choice"] == "autosage":
        assert bitwise_equal(out_exact, oracle.spmm_seq(crow, col, val, x))


def test_calibrate_full_keeps_exactness_margin(monkeypatch, tmp_path):
    import autosage_amd
    from autosage_amd import _auto

    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    monkeypatch.setenv("AUTOSAGE_FEATURE_SLICES", "on")
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "on")
    crow, col, _, x = _inputs(64, False, seed=43, rows=6000, degree=30, hubs=4, hub_degree=3000)
    d_crow, d_col, d_x = to_dev(crow, col, x)
    choice, result = autosage_amd.calibrate_full(d_crow, d_col, None, d_x)
    times = {json.dumps(c["candidate"]): c["best_ms"] for c in result["candidates"]}
    assert '"fslice"' in times and '"colslice"' in times
    if result["candidate"] == "colslice":
        assert times['"colslice"'] * (1.0 + _auto._INEXACT_MARGIN) < min(
            t for k, t in times.items() if k != '"colslice"')
    out, replay = autosage_amd.spmm_csr_auto(d_crow, d_col, None, d_x)
    assert replay["from_cache"] and replay["candidate"] == result["candidate"]
    if choice == "autosage" and result["candidate"] != "colslice":
        assert bitwise_equal(out, oracle.spmm_seq(crow, col, None, x))


def test_fslice_gradients_equal_the_exact_schedules():
    """Autograd through the feature-sliced op: dX = Aᵀ·dY and dval = SDDMM(dY, X)
    on the exact schedules, the same bits as spmm_csr's gradients."""
    crow, col, val, x = _inputs(64, True, seed=47, rows=1500)
    d_crow, d_col = to_dev(crow, col)
    grads = []
    for op in (torch.ops.autosage.spmm_csr, torch.ops.autosage.spmm_csr_fslice):
        d_val = torch.from_numpy(val).cuda().requires_grad_(True)
        d_x = torch.from_numpy(x).cuda().requires_grad_(True)
        y = op(d_crow, d_col, d_val, d_x)
        g = torch.linspace(-1.0, 1.0, y.numel(), device="cuda").view_as(y)
        y.backward(g)
        grads.append((y.detach(), d_val.grad, d_x.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def _shuffled_within_rows(crow, col, seed):
    rng = np.random.default_rng(seed)
    out = col.copy()
    for r in range(crow.size - 1):
        seg = out[crow[r]:crow[r + 1]]
        rng.shuffle(seg)
    return out


@pytest.mark.parametrize("phases", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("ascending", [True, False])
def test_fslice_column_phases_keep_the_bits(phases, ascending, monkeypatch):
    """Every phase count gives the sequential product's bits: a row's edges
    are cut into consecutive runs (at the phase's column bound when the
    columns ascend, at some point when they do not) and each launch continues
    the row's fp32 chain from Y.  Weighted and not, F = 96 (three slices, a
    chain read back through the float4 path) and F = 33 (a partial slice, the
    element path), hub rows, empty rows."""
    monkeypatch.setenv("AUTOSAGE_FSLICE_PHASES", str(phases))
    for features, weighted in ((96, True), (33, False)):
        crow, col, val, x = _inputs(features, weighted, seed=40 + phases, rows=2500, degree=14, hubs=4,
                                    hub_degree=2200, empty=0.1)
        if not ascending:
            col = _shuffled_within_rows(crow, col, seed=phases)
        d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
        assert _native.fslice_phases(d_crow, d_col, crow.size - 1) == phases
        got = torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, d_val, d_x)
        want = oracle.spmm_seq(crow, col, val, x)
        assert bitwise_equal(got, want), (features, weighted, mismatch_report(got, want))


def test_fslice_phase_tasks_cut_rows_at_the_column_bounds():
    """The plan's tasks: for position i of the order and phase p, the row's
    edges [first, first + count) are exactly those with a column in
    [p·N/P, (p+1)·N/P) when the columns ascend, and the phases of a row tile
    its edges in order."""
    crow, col, _, _ = _inputs(32, False, seed=61, rows=3000, degree=20, hubs=2, hub_degree=2900, empty=0.1)
    d_crow, d_col = to_dev(crow, col)
    n, nnz, phases = crow.size - 1, col.size, 3
    plan, tag = _native.fslice_plan(d_crow, d_col, n, phases=phases)
    assert (tag >> 8) & 0xFF == phases
    align = lambda b: (b + 255) // 256 * 256
    start = 256 + align(4 * n) + align(4 * (nnz + 64))
    tasks = plan[start:start + 16 * n * phases].view(torch.int32).view(phases, n, 4).cpu().numpy().astype(np.int64)
    order = plan[256:256 + 4 * n].view(torch.int32).cpu().numpy()
    for i in range(0, n, 7):
        row = order[i]
        edge = crow[row]
        for p in range(phases):
            r, count, lo, hi = tasks[p, i]
            first = lo & 0xFFFFFFFF | (hi << 32)
            assert r == row and first == edge, (i, p)
            cols = col[first:first + count]
            assert np.all(cols >= p * n // phases) and np.all(cols < (p + 1) * n // phases), (i, p)
            edge += count
        assert edge == crow[row + 1]


def test_fslice_phase_rule():
    """Two phases where a slice of X is well beyond an XCD's L2 (at least
    65,536 columns), rows average at least 32 edges and the columns ascend;
    one otherwise."""
    n, degree = 70_000, 40
    crow, col = case_graph(n, degree, seed=3)
    d_crow, d_col = to_dev(crow, col)
    assert _native.fslice_phases(d_crow, d_col, n) == 2
    d_shuffled = to_dev(_shuffled_within_rows(crow, col, seed=1))[0]
    assert _native.fslice_phases(d_crow, d_shuffled, n) == 1
    small_crow, small_col = case_graph(5000, degree, seed=4)
    assert _native.fslice_phases(*to_dev(small_crow, small_col), 5000) == 1
    sparse_crow, sparse_col = case_graph(n, 8, seed=5)
    assert _native.fslice_phases(*to_dev(sparse_crow, sparse_col), n) == 1
