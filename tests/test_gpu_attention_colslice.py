"""GPU parity of the column-sliced attention (``autosage::csr_attention_colslice``).

Online softmax per (row, column slice) with fp32 partial states merged per
row: checked against the oracle's fp64 attention at the 1e-5 relative /
1e-6 absolute bar for fp32 results; deterministic across calls and across
partial-state chunks; graphs whose columns do not ascend run on their
row-sorted copy; selected by ``csr_attention_forward`` only after a
full-graph timing."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import autosage_amd
import oracle
from autosage_amd import _native
from tests.gpu_common import case_graph, require_gpu, to_dev

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _inputs(fqk, fv, seed, rows=2500, degree=10, hubs=6, hub_degree=1500, empty=0.05):
    crow, col = case_graph(rows, degree, seed=seed, hubs=hubs, hub_degree=hub_degree, empty=empty)
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((rows, fqk)).astype(np.float32)
    k = rng.standard_normal((rows, fqk)).astype(np.float32)
    v = rng.standard_normal((rows, fv)).astype(np.float32)
    return crow, col, q, k, v


def _check(got: np.ndarray, exact: np.ndarray) -> None:
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= ATOL + RTOL * np.abs(exact)), float(np.max(err / (ATOL + RTOL * np.abs(exact))))


@pytest.mark.parametrize("fqk, fv", [(64, 128), (16, 16), (32, 64), (4, 256), (128, 128), (256, 64), (100, 36)])
def test_colslice_attention_against_fp64(fqk, fv):
    crow, col, q, k, v = _inputs(fqk, fv, seed=fqk + fv)
    assert (np.diff(crow) >= 128).sum() >= 6 and (np.diff(crow) == 0).any()
    d = to_dev(crow, col, q, k, v)
    got = torch.ops.autosage.csr_attention_colslice(*d, 0.125).cpu().numpy()
    _check(got, oracle.attention_f64(crow, col, q, k, v, scale=0.125))
    # the fp32 reference composition, at the north star's bar too
    ref = oracle.attention_ref(crow, col, q, k, v, scale=0.125)
    assert np.all(np.abs(got - ref) <= ATOL + RTOL * np.abs(ref))
    assert np.all(got[np.diff(crow) == 0] == 0)


def test_colslice_attention_deterministic_and_chunked(monkeypatch):
    crow, col, q, k, v = _inputs(64, 128, seed=3, rows=6000, hubs=40, hub_degree=2000)
    d = to_dev(crow, col, q, k, v)
    first = torch.ops.autosage.csr_attention_colslice(*d, 0.5)
    assert torch.equal(first, torch.ops.autosage.csr_attention_colslice(*d, 0.5))
    # room for ~3 sliced rows of partial states: the 40+ hub rows run in chunks
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", str((6000 * 40 + 4096 + 3 * 8 * 130 * 4 + 768) / 2**20))
    assert torch.equal(first, torch.ops.autosage.csr_attention_colslice(*d, 0.5))
    _check(first.cpu().numpy(), oracle.attention_f64(crow, col, q, k, v, scale=0.5))


def test_colslice_attention_unsorted_columns_and_rejections():
    crow, col, q, k, v = _inputs(64, 128, seed=5)
    r = int(np.argmax(np.diff(crow)))
    shuffled = col.copy()
    shuffled[crow[r]:crow[r + 1]] = shuffled[crow[r]:crow[r + 1]][::-1]
    # a graph whose columns do not ascend runs on its row-sorted copy: the
    # same result as the sorted graph, and the fp64 bar of the shuffled one
    # (scale 1/8 as in the benchmark configuration: the fp32 scores then stay
    # small enough for the 1e-6 absolute bar on near-cancelling outputs)
    d_crow, d_col, d_q, d_k, d_v = to_dev(crow, shuffled, q, k, v)
    got = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, d_q, d_k, d_v, 0.125)
    d_sorted = torch.from_numpy(col).cuda()
    assert torch.equal(got, torch.ops.autosage.csr_attention_colslice(d_crow, d_sorted, d_q, d_k, d_v, 0.125))
    _check(got.cpu().numpy(), oracle.attention_f64(crow, shuffled, q, k, v, scale=0.125))
    d = to_dev(crow, col, q[:, :3].copy(), k[:, :3].copy(), v)
    with pytest.raises(ValueError, match="multiples of 4"):
        torch.ops.autosage.csr_attention_colslice(*d, 1.0)


def test_attention_forward_times_and_caches_the_variant(monkeypatch, tmp_path):
    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "on")
    crow, col, q, k, v = _inputs(64, 128, seed=11, rows=8000, hubs=30, hub_degree=3000)
    d = to_dev(crow, col, q, k, v)
    out, info = autosage_amd.csr_attention_forward(*d, scale=0.125)
    assert info["fused"] and info["variant"] in ("fused", "colslice")
    fg = info["attention"]["full_graph"]
    assert fg["fused_ms"] > 0 and fg["colslice_ms"] > 0
    assert info["variant"] == min(("fused", "colslice"), key=lambda name: fg[f"{name}_ms"])
    exact = oracle.attention_f64(crow, col, q, k, v, scale=0.125)
    _check(out.cpu().numpy(), exact)
    again, info2 = autosage_amd.csr_attention_forward(*d, scale=0.125)
    assert info2["attention"]["from_cache"] and info2["variant"] == info["variant"]
    assert torch.equal(out, again)
    # off: the exact fused kernel, bit-identical to the native stages
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "off")
    off, info3 = autosage_amd.csr_attention_forward(*d, scale=0.125)
    assert info3["variant"] == "fused"
    assert torch.equal(off, torch.ops.autosage.csr_attention(*d, 0.125))
