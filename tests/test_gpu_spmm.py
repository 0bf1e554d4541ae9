"""GPU parity of the SpMM kernels against the CPU oracle.

Bar: the order-preserving kernels (whole graph, split with exact hub rows)
are bit-identical to the oracle's sequential fmaf product, which is itself
bit-identical to torch.sparse.mm on the CPU (tests/test_oracle.py).  The
reassociating split64 hub path is checked against the fp64 oracle:
|gpu - fp64| <= 1e-6·|fp64| + 1e-9.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import _native, synth
from tests.gpu_common import bitwise_equal, case_graph, mismatch_report, require_gpu, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _inputs(features, weighted, seed=0, rows=700, hubs=3, hub_degree=500):
    crow, col = case_graph(rows, 9, seed=seed, hubs=hubs, hub_degree=hub_degree, empty=0.08)
    rng = np.random.default_rng(seed + 100)
    val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
    x = rng.standard_normal((rows, features)).astype(np.float32)
    return crow, col, val, x


@pytest.mark.parametrize("vec4", ["1", "0"])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [1, 3, 32, 64, 100, 128, 200, 256, 300, 1024])
def test_spmm_csr_bitwise(features, weighted, vec4, monkeypatch):
    monkeypatch.setenv("AUTOSAGE_VEC4", vec4)
    crow, col, val, x = _inputs(features, weighted, seed=features)
    ref = oracle.spmm_seq(crow, col, val, x)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    got = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x)
    torch.cuda.synchronize()
    assert bitwise_equal(got, ref), mismatch_report(got, ref)


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [4, 16, 64, 68, 128, 132])
def test_spmm_csr_short_rows_bitwise(features, weighted):
    """Graphs of mean degree below 12 with float4 lanes take the sub-wave
    rows (16 or 32 lanes per row, several rows per wave; F > 128 one wave per
    row): the same sequential sums, so bitwise equal to the oracle, with empty
    rows, a hub row and rows of different lengths in one wave."""
    crow, col = case_graph(5000, 3, seed=features, hubs=1, hub_degree=900, empty=0.2)
    assert col.size < 12 * 5000
    rng = np.random.default_rng(features + 7)
    val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
    x = rng.standard_normal((5000, features)).astype(np.float32)
    ref = oracle.spmm_seq(crow, col, val, x)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    got = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x)
    torch.cuda.synchronize()
    assert bitwise_equal(got, ref), mismatch_report(got, ref)
    # the reference's Erdos-Renyi graph (200k rows, mean degree 4), sampled rows
    if features == 64 and not weighted:
        w = synth.erdos_renyi(seed=0, features=64)
        d = to_dev(w.crow, w.col, None, w.dense["x"])
        y = torch.ops.autosage.spmm_csr(*d).cpu().numpy()
        rows = np.random.default_rng(0).choice(w.rows, 2000, replace=False)
        for r in rows[:200]:
            cols = w.col[w.crow[r]:w.crow[r + 1]]
            want = np.zeros(64, dtype=np.float32)
            for c in cols:
                want = want + w.dense["x"][c]  # sequential fp32 adds in edge order
            assert np.array_equal(y[r].view(np.uint32), want.view(np.uint32)), r


@pytest.mark.parametrize("vec4", ["1", "0"])
@pytest.mark.parametrize("tile", [64, 128])
@pytest.mark.parametrize("waves", [2, 4, 8])
@pytest.mark.parametrize("threshold", [1, 10, 400, 10**6])
def test_spmm_split_exact_bitwise(tile, waves, threshold, vec4, monkeypatch):
    monkeypatch.setenv("AUTOSAGE_VEC4", vec4)
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", "exact")
    for features, weighted in ((64, False), (128, True), (256, False), (33, True)):
        crow, col, val, x = _inputs(features, weighted, seed=threshold + features)
        ref = oracle.spmm_seq(crow, col, val, x)
        d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
        got = torch.ops.autosage.spmm_csr_split(d_crow, d_col, d_val, d_x, tile, waves, threshold)
        torch.cuda.synchronize()
        assert bitwise_equal(got, ref), (features, weighted, mismatch_report(got, ref))


@pytest.mark.parametrize("waves", [2, 4, 8])
@pytest.mark.parametrize("features,weighted", [(64, False), (128, True), (256, False), (45, True)])
def test_spmm_split64_against_fp64(waves, features, weighted, monkeypatch):
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", "split64")
    crow, col, val, x = _inputs(features, weighted, seed=waves * 7 + features, hub_degree=650)
    exact = oracle.spmm_f64(crow, col, val, x)
    seq = oracle.spmm_seq(crow, col, val, x)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    got = torch.ops.autosage.spmm_csr_split(d_crow, d_col, d_val, d_x, 128, waves, 300).cpu().numpy()
    heavy = np.diff(crow) >= 300
    assert heavy.sum() >= 3
    # hub rows: fp64 partials rounded once, so within 1e-6 relative of fp64
    assert np.all(np.abs(got[heavy] - exact[heavy]) <= 1e-6 * np.abs(exact[heavy]) + 1e-9)
    # light rows: the exact kernel
    assert np.array_equal(got[~heavy], seq[~heavy])


@pytest.mark.parametrize("threshold", [1, 2, 9, 500, 10**9])
def test_bin_rows_bitwise(threshold):
    crow, _ = case_graph(5000, 8, seed=threshold % 97, hubs=20, hub_degree=600, empty=0.05)
    heavy_ref, light_ref = oracle.bin_rows(crow, threshold)
    (d_crow,) = to_dev(crow)
    heavy, light = _native.bin_rows_by_degree(d_crow, threshold)
    assert np.array_equal(heavy.cpu().numpy(), heavy_ref)
    assert np.array_equal(light.cpu().numpy(), light_ref)


def test_bin_rows_many_tiles():
    rng = np.random.default_rng(3)
    deg = rng.integers(0, 40, size=300_001)
    crow = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    heavy_ref, light_ref = oracle.bin_rows(crow, 20)
    (d_crow,) = to_dev(crow)
    heavy, light = _native.bin_rows_by_degree(d_crow, 20)
    assert np.array_equal(heavy.cpu().numpy(), heavy_ref)
    assert np.array_equal(light.cpu().numpy(), light_ref)


def test_config1_bitwise_against_oracle_and_torch_cpu():
    w = synth.config1(seed=0)
    x = w.dense["x"]
    ref = oracle.spmm_seq(w.crow, w.col, None, x)
    cpu = oracle.torch_cpu_spmm(torch.from_numpy(w.crow), torch.from_numpy(w.col), None, torch.from_numpy(x))
    assert np.array_equal(ref, cpu.numpy())
    d_crow, d_col, d_x = to_dev(w.crow, w.col, x)
    assert bitwise_equal(torch.ops.autosage.spmm_csr(d_crow, d_col, None, d_x), ref)
    for cand in ((64, 2, 9), (64, 8, 12), (128, 4, 10)):
        got = torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, *cand)
        assert bitwise_equal(got, ref), cand


def test_degenerate_shapes():
    # no nonzeros: zero output; single row; zero features
    crow = np.zeros(5, dtype=np.int64)
    col = np.zeros(0, dtype=np.int64)
    x = np.ones((4, 8), dtype=np.float32)
    d_crow, d_col, d_x = to_dev(crow, col, x)
    y = torch.ops.autosage.spmm_csr(d_crow, d_col, None, d_x)
    assert torch.count_nonzero(y).item() == 0
    y = torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, 64, 4, 1)
    assert torch.count_nonzero(y).item() == 0
    d_crow, d_col, d_x = to_dev(np.array([0, 1]), np.array([0]), np.array([[2.5, -1.0]], dtype=np.float32))
    assert torch.equal(torch.ops.autosage.spmm_csr(d_crow, d_col, None, d_x).cpu(), torch.tensor([[2.5, -1.0]]))
    empty_x = torch.empty((1, 0), device="cuda")
    assert torch.ops.autosage.spmm_csr(d_crow, d_col, None, empty_x).shape == (1, 0)


def test_input_checks_raise_runtime_error():
    d_crow, d_col, d_x = to_dev(np.array([0, 1]), np.array([0]), np.ones((1, 4), dtype=np.float32))
    with pytest.raises(RuntimeError, match="feature_tile must be 64 or 128"):
        torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, 32, 4, 1)
    with pytest.raises(RuntimeError, match="warps_per_block must be 2, 4, or 8"):
        torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, 64, 3, 1)
    with pytest.raises(RuntimeError, match="hub_threshold must be positive"):
        torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, 64, 4, 0)
    with pytest.raises(RuntimeError, match="crow must contain N \\+ 1 entries"):
        torch.ops.autosage.spmm_csr(d_crow[:1], d_col, None, d_x)
    with pytest.raises(RuntimeError, match="x must be contiguous"):
        torch.ops.autosage.spmm_csr(d_crow, d_col, None, torch.ones((4, 2), device="cuda").t())


def _duplicates_graph(rows: int, mean_degree: int, seed: int, hub_degree: int = 0):
    """Degrees U{0..2·mean}, columns drawn with replacement in no particular
    order (duplicates and unsorted rows allowed, as the reference's GPU test
    graphs have them); row 0 optionally a hub."""
    rng = np.random.default_rng(seed)
    degrees = rng.integers(0, 2 * mean_degree + 1, size=rows)
    if hub_degree:
        degrees[0] = hub_degree
    crow = np.concatenate([[0], np.cumsum(degrees)]).astype(np.int64)
    col = rng.integers(0, rows, size=int(crow[-1])).astype(np.int64)
    return crow, col


def _sparse_mm_gpu(crow, col, val, x):
    """PyTorch-ROCm's own CSR product on the GPU (rocSPARSE): another
    summation order, the comparison the reference's GPU tests make."""
    values = val if val is not None else torch.ones(col.numel(), device=x.device)
    n = crow.numel() - 1
    return torch.sparse.mm(torch.sparse_csr_tensor(crow, col, values, size=(n, x.size(0))), x)


# The reference compares its native SpMM with torch's CSR product at
# rtol 1e-4 / atol 3e-3 for F in {32, 64, 113, 128, 256}, and its split
# launcher (tile 128, 8 warps, threshold 128) on a 512-row graph with one
# 400-edge row (tests/test_cuda.py:32-57).  Here every exact schedule is
# held to that tolerance against PyTorch-ROCm's GPU product AND to the bits
# of the sequential oracle.
@pytest.mark.parametrize("features", [32, 64, 113, 128, 256])
def test_exact_schedules_on_duplicate_columns(features):
    crow, col = _duplicates_graph(320, 11, seed=features)
    rng = np.random.default_rng(features + 1)
    val = rng.random(col.size, dtype=np.float32)
    x = rng.standard_normal((320, features)).astype(np.float32)
    want = oracle.spmm_seq(crow, col, val, x)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    torch_gpu = _sparse_mm_gpu(d_crow, d_col, d_val, d_x)
    outputs = {
        "spmm_csr": torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x),
        "split": torch.ops.autosage.spmm_csr_split(d_crow, d_col, d_val, d_x, 64, 2, 16),
        "fslice": torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, d_val, d_x),
    }
    for name, out in outputs.items():
        assert bitwise_equal(out, want), (name, mismatch_report(out, want))
        assert torch.allclose(out, torch_gpu, rtol=1e-4, atol=3e-3), name


@pytest.mark.parametrize("tile, waves, threshold", [(128, 8, 128), (64, 2, 300), (128, 4, 1)])
def test_split_hub_row_on_duplicate_columns(tile, waves, threshold):
    crow, col = _duplicates_graph(512, 8, seed=tile + waves, hub_degree=400)
    x = np.random.default_rng(5).standard_normal((512, 128)).astype(np.float32)
    d_crow, d_col, d_x = to_dev(crow, col, x)
    out = torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, tile, waves, threshold)
    assert bitwise_equal(out, oracle.spmm_seq(crow, col, None, x))
    assert torch.allclose(out, _sparse_mm_gpu(d_crow, d_col, None, d_x), rtol=1e-4, atol=3e-3)
