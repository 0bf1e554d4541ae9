"""Parity at the benchmark configurations' full sizes.

The GPU runs the whole graph; the CPU oracle checks a seeded sample of rows
(always including the longest ones), through sub-CSRs of those rows.  Bars as
in the small-size tests: bit-identical for SpMM (exact modes) and SDDMM,
|Δ| <= 1e-6 + 1e-5·|ref| for softmax/attention, fp64 bound for split64.
Size-independent properties are checked on the full outputs: every split
variant equals the whole-graph kernel bit for bit, fused attention equals
the unfused stages bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import synth
from tests.gpu_common import bitwise_equal, elementwise_parity, require_gpu

pytestmark = pytest.mark.gpu

RTOL = 1e-5
ATOL = 1e-6


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def sample_rows(crow: np.ndarray, count: int, seed: int, longest: int = 8) -> np.ndarray:
    deg = np.diff(crow)
    rng = np.random.default_rng(seed)
    picked = rng.choice(deg.size, size=min(count, deg.size), replace=False)
    top = np.argsort(deg)[-longest:]
    return np.unique(np.concatenate([picked, top]))


def sub_csr(crow: np.ndarray, col: np.ndarray, rows: np.ndarray):
    starts, ends = crow[rows], crow[rows + 1]
    sub_crow = np.concatenate([[0], np.cumsum(ends - starts)]).astype(np.int64)
    edges = np.concatenate([np.arange(s, e) for s, e in zip(starts, ends)]).astype(np.int64)
    return sub_crow, col[edges], edges


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_config2_weighted_spmm():
    w = synth.config2(seed=0)
    d_crow, d_col, d_val, d_x = dev(w.crow), dev(w.col), dev(w.val), dev(w.dense["x"])
    whole = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x)
    split = torch.ops.autosage.spmm_csr_split(d_crow, d_col, d_val, d_x, 128, 2, 16)
    assert torch.equal(whole, split)
    rows = sample_rows(w.crow, 3000, seed=1)
    ref = oracle.spmm_seq(w.crow, w.col, w.val, w.dense["x"], rows=rows)
    assert bitwise_equal(whole[torch.from_numpy(rows).cuda()], ref)


@pytest.mark.parametrize("features", [64, 128, 256])
def test_config3_skewed_spmm(features, monkeypatch):
    w = synth.config3(seed=0, features=features)
    d_crow, d_col, d_x = dev(w.crow), dev(w.col), dev(w.dense["x"])
    deg = np.diff(w.crow)
    q95 = int(np.rint(np.quantile(deg, 0.95)))
    whole = torch.ops.autosage.spmm_csr(d_crow, d_col, None, d_x)
    for cand in ((128, 2, q95), (64, 4, 512), (128, 8, 2048)):
        assert torch.equal(torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, *cand), whole), cand
    rows = sample_rows(w.crow, 1500, seed=features)
    ref = oracle.spmm_seq(w.crow, w.col, None, w.dense["x"], rows=rows)
    d_rows = torch.from_numpy(rows).cuda()
    assert bitwise_equal(whole[d_rows], ref)
    # reassociating hub mode: hub rows within 1e-6 of fp64, light rows exact
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", "split64")
    s64 = torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, 128, 4, q95)[d_rows].cpu().numpy()
    exact = oracle.spmm_f64(w.crow, w.col, None, w.dense["x"], rows=rows)
    heavy = deg[rows] >= q95
    assert heavy.sum() >= 8
    assert np.all(np.abs(s64[heavy] - exact[heavy]) <= 1e-6 * np.abs(exact[heavy]) + 1e-9)
    assert np.array_equal(s64[~heavy], ref[~heavy])
    # column-sliced SpMM (fp64 partials): every sampled row within 1e-6 of
    # fp64; repeated calls, and a call in row chunks, give the same bits
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", "exact")
    sliced = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, d_x)
    got = sliced[d_rows].cpu().numpy()
    assert np.all(np.abs(got - exact) <= 1e-6 * np.abs(exact) + 1e-9)
    assert np.all(np.abs(got - exact) <= RTOL * np.abs(exact) + ATOL)
    assert torch.equal(torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, d_x), sliced)
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", "300")
    assert torch.equal(torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, d_x), sliced)
    # the sequential fp32 order (the reference's) is itself further than
    # 1e-5 from the fp64 sums on rows that nearly cancel; the sliced sums are not
    worst_seq = np.max(np.abs(ref - exact) / (RTOL * np.abs(exact) + ATOL))
    worst_sliced = np.max(np.abs(got - exact) / (RTOL * np.abs(exact) + ATOL))
    assert worst_sliced < 0.1 and worst_sliced < worst_seq
    # against the reference's CPU result: max relative error (max|d| / max|ref|)
    # below 1e-5, and the reference's own GPU test bar (its
    # tests/test_cuda.py:40: rtol 1e-4, atol 3e-3)
    assert np.max(np.abs(got - ref)) <= RTOL * np.max(np.abs(ref))
    assert np.allclose(got, ref, rtol=1e-4, atol=3e-3)
    # element by element against the reference's fp32 result (the sequential
    # CPU product, torch.sparse.mm): each output is within 1e-5·|ref| + 1e-6
    # of it, or the reference is itself off that bar against fp64 (or within
    # 1e-6·|fp64| + 1e-9 of being off it) and the sliced output is within
    # 1e-6·|fp64| + 1e-9 of fp64 and closer to it than the reference
    elementwise_parity(got, ref, exact, tight_rel=1e-6, tight_abs=1e-9)


def test_config3_shuffled_columns_take_the_sliced_schedule():
    """cfg3 at F = 128 with the columns of every row in a random order (what
    ``edge_index_to_csr`` gives for an edge list not sorted by source): the
    column-sliced schedule runs on the row-sorted copy, ``spmm_csr_auto``
    still chooses it, and the sampled rows are within 1e-6·|fp64|."""
    import autosage_amd

    w = synth.config3(seed=0, features=128)
    d_crow, d_col, d_x = dev(w.crow), dev(w.col), dev(w.dense["x"])
    n = w.rows
    edge_rows = torch.repeat_interleave(torch.arange(n, device="cuda"), d_crow[1:] - d_crow[:-1],
                                        output_size=w.nnz)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    noise = torch.randint(0, 1 << 31, (w.nnz,), generator=gen, device="cuda")
    shuffled = d_col.index_select(0, torch.argsort(edge_rows * (1 << 31) + noise)).contiguous()
    del edge_rows, noise, d_col
    from autosage_amd import _native

    assert not _native.columns_ascending(d_crow, shuffled)
    out, info = autosage_amd.spmm_csr_auto(d_crow, shuffled, None, d_x)
    timed = {tuple(c["candidate"]) if isinstance(c["candidate"], list) else c["candidate"]: c["best_ms"]
             for c in info["full_graph"]["candidates"]}
    assert info["candidate"] == "colslice", timed
    rows = sample_rows(w.crow, 1500, seed=3)
    exact = oracle.spmm_f64(w.crow, shuffled.cpu().numpy(), None, w.dense["x"], rows=rows)
    got = out[torch.from_numpy(rows).cuda()].cpu().numpy()
    assert np.all(np.abs(got - exact) <= 1e-6 * np.abs(exact) + 1e-9)
    # cached: the same choice, the same bits
    again, cached = autosage_amd.spmm_csr_auto(d_crow, shuffled, None, d_x)
    assert cached["from_cache"] and torch.equal(again, out)


@pytest.mark.parametrize("features", [64, 128])
def test_config4_sddmm(features):
    w = synth.config4(seed=0, features=features)
    d_crow, d_col, d_q, d_k = dev(w.crow), dev(w.col), dev(w.dense["q"]), dev(w.dense["k"])
    whole = torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, d_k)
    for waves, threshold in ((4, 256), (8, 4096), (2, 60000)):
        assert torch.equal(torch.ops.autosage.sddmm_csr_split(d_crow, d_col, d_q, d_k, waves, threshold), whole)
    rows = sample_rows(w.crow, 2000, seed=features, longest=6)
    s_crow, s_col, edges = sub_csr(w.crow, w.col, rows)
    ref = oracle.sddmm_ref(s_crow, s_col, w.dense["q"][rows], w.dense["k"])
    assert bitwise_equal(whole[torch.from_numpy(edges).cuda()], ref)


def test_config5_attention():
    w = synth.config5(seed=0)
    q, k, v = w.dense["q"], w.dense["k"], w.dense["v"]
    d_crow, d_col, d_q, d_k, d_v = dev(w.crow), dev(w.col), dev(q), dev(k), dev(v)
    fused = torch.ops.autosage.csr_attention(d_crow, d_col, d_q, d_k, d_v, 0.125)
    scores = torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, d_k) * 0.125
    probs = torch.ops.autosage.csr_row_softmax(d_crow, scores)
    del scores
    unfused = torch.ops.autosage.spmm_csr(d_crow, d_col, probs, d_v)
    assert torch.equal(fused, unfused)
    rows = sample_rows(w.crow, 1500, seed=5)
    s_crow, s_col, edges = sub_csr(w.crow, w.col, rows)
    ref = oracle.attention_ref(s_crow, s_col, q[rows], k, v, scale=0.125)
    got = fused[torch.from_numpy(rows).cuda()].cpu().numpy()
    assert np.all(np.abs(got - ref) <= ATOL + RTOL * np.abs(ref)), float(np.max(np.abs(got - ref)))
    p_ref = oracle.row_softmax(s_crow, oracle.sddmm_ref(s_crow, s_col, q[rows], k) * np.float32(0.125))
    p_got = probs[torch.from_numpy(edges).cuda()].cpu().numpy()
    assert np.all(np.abs(p_got - p_ref) <= ATOL + RTOL * np.abs(p_ref))
    # the column-sliced attention on the same graph: within the bar of the
    # fp64 attention on the sampled rows (hubs included), and repeatable
    del probs, unfused
    sliced = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, d_q, d_k, d_v, 0.125)
    assert torch.equal(sliced, torch.ops.autosage.csr_attention_colslice(d_crow, d_col, d_q, d_k, d_v, 0.125))
    exact = oracle.attention_f64(s_crow, s_col, q[rows], k, v, scale=0.125)
    got_s = sliced[torch.from_numpy(rows).cuda()].cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got_s - exact) <= ATOL + RTOL * np.abs(exact)), float(np.max(np.abs(got_s - exact)))
    # element by element against the reference's fp32 composition (SDDMM,
    # row softmax, sequential SpMM): within 1e-5·|ref| + 1e-6 of it, or the
    # reference is itself off that bar against fp64 while the sliced output
    # (fp32 online softmax, fp32 partial states) is within it and closer
    elementwise_parity(got_s, ref, exact, tight_rel=RTOL, tight_abs=ATOL)
    # the fused kernel (the reference's stage order) against the same result
    elementwise_parity(got, ref, exact, tight_rel=RTOL, tight_abs=ATOL)
