"""Parity at the benchmark configurations' full sizes, on every output.

The GPU runs the whole graph and the CPU oracle (OpenMP over rows, the same
bits on any thread count) computes every output of the same graph.  Bars as
in the small-size tests: bit-identical for the exact SpMM schedules (the
whole-graph, split and feature-sliced kernels) and SDDMM; for the
reassociating kernels (column-sliced SpMM, attention) every element is
within 1e-5·|ref| + 1e-6 of the reference's fp32 result or arbitrated
against fp64 (``tests/gpu_common.elementwise_parity_rows``: the reference
itself off that bar while the kernel is within its own bound of fp64 and
closer to it), with the counts of each case printed as ``[parity]`` lines.
Size-independent properties are checked too: every split variant equals
the whole-graph kernel bit for bit, fused attention equals the unfused
stages bit for bit, repeated calls give the same bits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import synth
from tests.gpu_common import bitwise_equal, elementwise_parity_rows, mismatch_report, require_gpu

pytestmark = pytest.mark.gpu

RTOL = 1e-5
ATOL = 1e-6


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _step(name: str) -> None:
    print(f"[fullsize] {name}", flush=True)


def test_config2_weighted_spmm():
    w = synth.config2(seed=0)
    d_crow, d_col, d_val, d_x = dev(w.crow), dev(w.col), dev(w.val), dev(w.dense["x"])
    _step("cfg2 oracle")
    want = oracle.spmm_seq(w.crow, w.col, w.val, w.dense["x"])
    _step("cfg2 gpu")
    whole = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x)
    assert bitwise_equal(whole, want), mismatch_report(whole, want)
    for out in (torch.ops.autosage.spmm_csr_split(d_crow, d_col, d_val, d_x, 128, 2, 16),
                torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, d_val, d_x)):
        assert torch.equal(out, whole)


@pytest.mark.parametrize("features", [64, 128, 256])
def test_config3_skewed_spmm(features, monkeypatch, tmp_path):
    w = synth.config3(seed=0, features=features)
    x = w.dense["x"]
    d_crow, d_col, d_x = dev(w.crow), dev(w.col), dev(x)
    deg = np.diff(w.crow)
    q95 = int(np.rint(np.quantile(deg, 0.95)))
    _step(f"cfg3 F={features} oracle (sequential fp32 and fp64, all rows)")
    ref = oracle.spmm_seq(w.crow, w.col, None, x)
    exact = oracle.spmm_f64(w.crow, w.col, None, x)
    _step(f"cfg3 F={features} exact schedules")
    whole = torch.ops.autosage.spmm_csr(d_crow, d_col, None, d_x)
    assert bitwise_equal(whole, ref), mismatch_report(whole, ref)
    for cand in ((128, 2, q95), (64, 4, 512), (128, 8, 2048)):
        assert torch.equal(torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, *cand), whole), cand
    fslice = torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, None, d_x)
    assert torch.equal(fslice, whole)
    del fslice
    # the scheduler's step (the bench line): cold, then replayed from its cache,
    # the same bits as the sequential product
    import autosage_amd

    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    auto, info = autosage_amd.spmm_csr_auto(d_crow, d_col, None, d_x)
    assert info["candidate"] == "fslice", info.get("candidate")
    assert torch.equal(auto, whole)
    again, cached = autosage_amd.spmm_csr_auto(d_crow, d_col, None, d_x)
    assert cached["from_cache"] and torch.equal(again, whole)
    del auto, again
    # reassociating hub mode: hub rows within 1e-6 of fp64, light rows exact
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", "split64")
    s64 = torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, d_x, 128, 4, q95).cpu().numpy()
    heavy = deg >= q95
    assert np.all(np.abs(s64[heavy] - exact[heavy]) <= 1e-6 * np.abs(exact[heavy]) + 1e-9)
    assert np.array_equal(s64[~heavy], ref[~heavy])
    del s64
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", "exact")
    # column-sliced SpMM (fp64 partials): every output within 1e-6 of fp64;
    # repeated calls, and a call in row chunks, give the same bits
    _step(f"cfg3 F={features} column-sliced")
    sliced = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, d_x)
    assert torch.equal(torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, d_x), sliced)
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", "300")
    assert torch.equal(torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, None, d_x), sliced)
    got = sliced.cpu().numpy()
    del sliced
    assert np.all(np.abs(got - exact) <= 1e-6 * np.abs(exact) + 1e-9)
    # max relative error (max|d| / max|ref|) against the reference's CPU
    # result below 1e-5, and the reference's own GPU test bar (its
    # tests/test_cuda.py:40: rtol 1e-4, atol 3e-3)
    assert np.max(np.abs(got - ref)) <= RTOL * np.max(np.abs(ref))
    assert np.allclose(got, ref, rtol=1e-4, atol=3e-3)
    # element by element against the reference's fp32 result: within
    # 1e-5·|ref| + 1e-6 of it, or arbitrated against fp64 with the sliced
    # kernel's bound 1e-6·|fp64| + 1e-9
    counts = elementwise_parity_rows(got, ref, exact, tight_rel=1e-6, tight_abs=1e-9,
                                     label=f"colslice cfg3 F={features}")
    assert counts["elements"] == w.rows * features
    # the sequential fp32 order (the reference's) is itself further than
    # 1e-5 from the fp64 sums on outputs that nearly cancel; the sliced sums are not
    assert counts["worst_reference_error_over_bar"] > 1.0 > 0.1 > counts["worst_kernel_error_over_bar"]


def test_config3_backward_dx_is_the_sequential_transposed_product():
    """cfg3 at F = 128 through autograd: dX = Aᵀ·dY runs on the feature-sliced
    SpMM over the transposed graph (whose columns ascend, so it runs in two
    column phases) and equals the sequential CPU product over Aᵀ on every
    output, weighted (dval is not asked for) and not."""
    from autosage_amd import _native
    from autosage_amd._autograd import csr_transpose

    w = synth.config3(seed=0, features=128)
    n = w.rows
    d_crow, d_col = dev(w.crow), dev(w.col)
    rng = np.random.default_rng(21)
    g = rng.standard_normal((n, 128)).astype(np.float32)
    val = rng.standard_normal(w.nnz).astype(np.float32)
    crow_t, col_t, perm = csr_transpose(d_crow, d_col)
    assert _native.fslice_phases(crow_t, col_t, n) == 2
    h_crow_t, h_col_t, h_perm = (t.cpu().numpy() for t in (crow_t, col_t, perm))
    for weights in (None, val):
        x = dev(w.dense["x"]).requires_grad_(True)
        d_val = None if weights is None else dev(weights)
        _step(f"cfg3 backward dX weighted={weights is not None}")
        torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, d_val, x).backward(dev(g))
        want = oracle.spmm_seq(h_crow_t, h_col_t, None if weights is None else weights[h_perm], g)
        assert bitwise_equal(x.grad, want), mismatch_report(x.grad, want)
        del x


def test_config3_shuffled_columns():
    """cfg3 at F = 128 with the columns of every row in a random order (what
    ``edge_index_to_csr`` gives for an edge list not sorted by source):
    ``spmm_csr_auto`` times the schedules on it, and whatever it chooses
    meets that schedule's contract on every output (the exact schedules keep
    the shuffled CSR order bit for bit; the column-sliced one runs on a
    row-sorted copy, within 1e-6·|fp64|)."""
    import autosage_amd
    from autosage_amd import _native

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
    assert not _native.columns_ascending(d_crow, shuffled)
    out, info = autosage_amd.spmm_csr_auto(d_crow, shuffled, None, d_x)
    timed = [c["candidate"] for c in info["full_graph"]["candidates"]]
    assert "fslice" in timed and "colslice" in timed, timed
    h_shuffled = shuffled.cpu().numpy()
    if info["candidate"] == "colslice":
        exact = oracle.spmm_f64(w.crow, h_shuffled, None, w.dense["x"])
        assert np.all(np.abs(out.cpu().numpy() - exact) <= 1e-6 * np.abs(exact) + 1e-9)
    else:
        assert info["choice"] == "autosage", info
        want = oracle.spmm_seq(w.crow, h_shuffled, None, w.dense["x"])
        assert bitwise_equal(out, want), mismatch_report(out, want)
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
    _step(f"cfg4 F={features} oracle (all edges)")
    ref = oracle.sddmm_ref(w.crow, w.col, w.dense["q"], w.dense["k"])
    assert bitwise_equal(whole, ref), mismatch_report(whole, ref)


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
    del unfused
    _step("cfg5 oracle: fp32 composition and fp64 attention, all rows")
    s_ref = oracle.sddmm_ref(w.crow, w.col, q, k) * np.float32(0.125)
    p_ref = oracle.row_softmax(w.crow, s_ref)
    del s_ref
    p_got = probs.cpu().numpy()
    del probs
    assert np.all(np.abs(p_got - p_ref) <= ATOL + RTOL * np.abs(p_ref))
    del p_got
    ref = oracle.spmm_seq(w.crow, w.col, p_ref, v)
    del p_ref
    exact = oracle.attention_f64(w.crow, w.col, q, k, v, scale=0.125)
    got = fused.cpu().numpy()
    del fused
    # the fused kernel (the reference's stage order; its softmax's exp and
    # division are the GPU's): every output within the bar of the
    # reference's fp32 composition, or arbitrated against fp64
    counts = elementwise_parity_rows(got, ref, exact, tight_rel=RTOL, tight_abs=ATOL, label="fused attention cfg5")
    assert counts["elements"] == w.rows * v.shape[1]
    # the column-sliced attention on the same graph: within the bar of the
    # fp64 attention on every output, repeatable, and held to the same
    # element-wise rule against the reference's fp32 composition
    sliced = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, d_q, d_k, d_v, 0.125)
    assert torch.equal(sliced, torch.ops.autosage.csr_attention_colslice(d_crow, d_col, d_q, d_k, d_v, 0.125))
    got_s = sliced.cpu().numpy()
    del sliced
    worst = 0.0
    for start in range(0, got_s.shape[0], 262144):
        part = slice(start, start + 262144)
        err = np.abs(got_s[part].astype(np.float64) - exact[part])
        worst = max(worst, float(np.max(err / (ATOL + RTOL * np.abs(exact[part])))))
    print(f"[parity] colslice attention cfg5 worst |got - fp64| / bar = {worst:.4f}", flush=True)
    assert worst <= 1.0
    elementwise_parity_rows(got_s, ref, exact, tight_rel=RTOL, tight_abs=ATOL, label="colslice attention cfg5")


def _edges_of(crow: np.ndarray, rows: np.ndarray):
    """(edge ids of `rows` in CSR order, the position in `rows` of each edge's row)."""
    starts, ends = crow[rows], crow[rows + 1]
    counts = ends - starts
    owner = np.repeat(np.arange(rows.size), counts)
    offsets = np.arange(counts.sum()) - np.repeat(np.cumsum(counts) - counts, counts)
    return np.repeat(starts, counts) + offsets, owner


def _row_softmax_stats(crow, col, q, k, v, g, rows, scale, chunk=1 << 20):
    """fp64 per-row softmax statistics of the attention for `rows`: the max
    score m, the denominator d and t = sum_e p_e·<g_row, v_col>."""
    edges, owner = _edges_of(crow, rows)
    m = np.full(rows.size, -np.inf)
    s = np.empty(edges.size)
    dp = np.empty(edges.size)
    for a in range(0, edges.size, chunk):
        e, o = edges[a:a + chunk], owner[a:a + chunk]
        s[a:a + chunk] = scale * np.einsum("ij,ij->i", q[rows[o]].astype(np.float64), k[col[e]].astype(np.float64))
        dp[a:a + chunk] = np.einsum("ij,ij->i", g[rows[o]].astype(np.float64), v[col[e]].astype(np.float64))
    np.maximum.at(m, owner, s)
    ex = np.exp(s - m[owner])
    d = np.bincount(owner, weights=ex, minlength=rows.size)
    t = np.bincount(owner, weights=ex / d[owner] * dp, minlength=rows.size)
    return m, d, t


def _attention_grad_samples(crow, col, crow_t, col_t, perm, q, k, v, g, rows, cols, scale):
    """fp64 dQ of `rows` and dK, dV of `cols` of out = softmax_row(scale·QKᵀ)·V
    with upstream gradient g, each with the sum of its terms' magnitudes
    (want, magnitude): dQ[r] = scale·sum_e ds_e·K[c_e], dK[c] = scale·sum_e
    ds_e·Q[r_e], dV[c] = sum_e p_e·g[r_e], ds_e = p_e·(<g_r, V_c> - t_r)."""
    f64 = lambda a: a.astype(np.float64)
    m, d, t = _row_softmax_stats(crow, col, q, k, v, g, rows, scale)
    edges, owner = _edges_of(crow, rows)
    r, c = rows[owner], col[edges]
    p = np.exp(scale * np.einsum("ij,ij->i", f64(q[r]), f64(k[c])) - m[owner]) / d[owner]
    ds = p * (np.einsum("ij,ij->i", f64(g[r]), f64(v[c])) - t[owner])
    dq = np.zeros((rows.size, q.shape[1]))
    dq_mag = np.zeros_like(dq)
    np.add.at(dq, owner, scale * ds[:, None] * f64(k[c]))
    np.add.at(dq_mag, owner, np.abs(scale * ds[:, None] * f64(k[c])))
    # the edges into the sampled columns and the softmax of every row they sit in
    in_edges, in_owner = _edges_of(crow_t, cols)
    e_ids, e_rows = perm[in_edges], col_t[in_edges]
    involved, where = np.unique(e_rows, return_inverse=True)
    m2, d2, t2 = _row_softmax_stats(crow, col, q, k, v, g, involved, scale)
    cc = cols[in_owner]
    p2 = np.exp(scale * np.einsum("ij,ij->i", f64(q[e_rows]), f64(k[cc])) - m2[where]) / d2[where]
    ds2 = p2 * (np.einsum("ij,ij->i", f64(g[e_rows]), f64(v[cc])) - t2[where])
    dk = np.zeros((cols.size, k.shape[1]))
    dk_mag = np.zeros_like(dk)
    dv = np.zeros((cols.size, v.shape[1]))
    dv_mag = np.zeros_like(dv)
    np.add.at(dk, in_owner, scale * ds2[:, None] * f64(q[e_rows]))
    np.add.at(dk_mag, in_owner, np.abs(scale * ds2[:, None] * f64(q[e_rows])))
    np.add.at(dv, in_owner, p2[:, None] * f64(g[e_rows]))
    np.add.at(dv_mag, in_owner, np.abs(p2[:, None] * f64(g[e_rows])))
    assert np.array_equal(col[e_ids], cc)
    return (dq, dq_mag), (dk, dk_mag), (dv, dv_mag)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config5_attention_gradients_sampled(dtype):
    """The attention backward at full size (cfg5: 2.45M rows, 124M edges), on
    sampled rows (dQ) and columns (dK, dV), the longest ones included,
    against fp64.  fp32: every sampled element within 1e-5·|want| + 1e-6, or,
    where the sum nearly cancels, within 1e-5 of the sum of its terms'
    magnitudes; bf16 (inputs, upstream gradient and gradients in bf16): within
    a unit of the type's rounding plus 2e-5 of the largest element."""
    from autosage_amd._autograd import csr_transpose

    w = synth.config5(seed=0)
    n = w.rows
    scale = 0.125
    rng = np.random.default_rng(55)
    g32 = rng.standard_normal(w.dense["v"].shape).astype(np.float32)
    d_crow, d_col = dev(w.crow), dev(w.col)
    leaves = [dev(w.dense[name]).to(dtype).requires_grad_(True) for name in ("q", "k", "v")]
    d_g = dev(g32).to(dtype)
    op = torch.ops.autosage.csr_attention if dtype == torch.float32 else torch.ops.autosage.csr_attention_colslice
    _step(f"cfg5 attention backward {dtype}")
    op(d_crow, d_col, *leaves, scale).backward(d_g)
    # the values the kernels saw (16-bit: converted exactly)
    q, k, v = (t.detach().float().cpu().numpy() for t in leaves)
    g = d_g.float().cpu().numpy()
    deg = np.diff(w.crow)
    rows = np.unique(np.concatenate([np.argsort(deg)[-8:], rng.choice(n, 1500, replace=False)]))
    crow_t, col_t, perm = (t.cpu().numpy() for t in csr_transpose(d_crow, d_col))
    in_deg = np.diff(crow_t)
    cols = np.unique(np.concatenate([np.argsort(in_deg)[-4:], rng.choice(n, 300, replace=False)]))
    _step(f"cfg5 fp64 gradients of {rows.size} rows and {cols.size} columns")
    wants = _attention_grad_samples(w.crow, w.col, crow_t, col_t, perm, q, k, v, g, rows, cols, scale)
    picks = (rows, cols, cols)
    for name, leaf, (want, mag), pick in zip("QKV", leaves, wants, picks):
        got = leaf.grad[torch.from_numpy(pick).cuda()].double().cpu().numpy()
        err = np.abs(got - want)
        if dtype == torch.float32:
            plain = err <= RTOL * np.abs(want) + ATOL
            bound = err <= RTOL * mag + ATOL
            print(f"[parity] cfg5 d{name} fp32: {got.size} sampled elements, {int(plain.sum())} within "
                  f"1e-5·|want| + 1e-6, all within 1e-5·sum|terms| + 1e-6: {bool(bound.all())}, worst "
                  f"err / (1e-5·|want| + 1e-6) = {float(np.max(err / (RTOL * np.abs(want) + ATOL))):.3f}, worst "
                  f"err / (1e-5·sum|terms| + 1e-6) = {float(np.max(err / (RTOL * mag + ATOL))):.3f}", flush=True)
            assert bound.all(), (name, float(np.max(err - RTOL * mag - ATOL)))
        else:
            bar = 2.0 ** -8 * np.abs(want) + 2e-5 * np.max(np.abs(want))
            print(f"[parity] cfg5 d{name} bf16: {got.size} sampled elements, worst err / bar = "
                  f"{float(np.max(err / bar)):.3f}", flush=True)
            assert np.all(err <= bar), (name, float(np.max(err - bar)))


def _round16(values: np.ndarray, dtype) -> np.ndarray:
    """fp64 -> fp32 -> dtype, round to nearest even both times, back to fp64."""
    return torch.from_numpy(values).to(torch.float32).to(dtype).to(torch.float64).numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config3_16bit_spmm_every_schedule(dtype):
    """cfg3 at F = 128 in bf16 and fp16: every 16-bit schedule (rows whole,
    edge slices, column slices) and ``spmm_csr_auto`` equal the rounded oracle
    (fp64 sum of the exact products, rounded to fp32 and then to the type) on
    every output; the sums are exact in fp64 here, so the order is free.  Then
    dX = Aᵀ·dY through autograd equals the rounded oracle over Aᵀ."""
    import autosage_amd
    from autosage_amd import _native
    from autosage_amd._autograd import csr_transpose

    w = synth.config3(seed=0, features=128)
    x16 = torch.from_numpy(w.dense["x"]).to(dtype)
    d_crow, d_col, d_x = dev(w.crow), dev(w.col), x16.cuda()
    _step(f"cfg3 {dtype} oracle (fp64 sums, all rows)")
    want = oracle.spmm_rounded_16(w.crow, w.col, None, x16, dtype).view(torch.int16)
    outs = {
        "rows": _native.spmm_rows_16_impl(d_crow, d_col, None, d_x),
        "edges": _native.spmm_rounded_16_impl(d_crow, d_col, None, d_x, column_slices=False),
        "columns": _native.spmm_rounded_16_impl(d_crow, d_col, None, d_x, column_slices=True),
        "op": torch.ops.autosage.spmm_csr(d_crow, d_col, None, d_x),
    }
    for name, got in outs.items():
        assert torch.equal(got.cpu().view(torch.int16), want), name
    auto, info = autosage_amd.spmm_csr_auto(d_crow, d_col, None, d_x)
    assert torch.equal(auto.cpu().view(torch.int16), want), info.get("candidate")
    del auto, outs
    # the backward: dX = Aᵀ·dY on the 16-bit kernels
    g16 = torch.from_numpy(np.random.default_rng(8).standard_normal((w.rows, 128)).astype(np.float32)).to(dtype)
    leaf = d_x.clone().requires_grad_(True)
    torch.ops.autosage.spmm_csr(d_crow, d_col, None, leaf).backward(g16.cuda())
    crow_t, col_t, _ = csr_transpose(d_crow, d_col)
    _step(f"cfg3 {dtype} backward oracle")
    want_dx = oracle.spmm_rounded_16(crow_t.cpu().numpy(), col_t.cpu().numpy(), None, g16, dtype).view(torch.int16)
    assert torch.equal(leaf.grad.cpu().view(torch.int16), want_dx)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config4_16bit_sddmm(dtype):
    """cfg4 at F = 64 in bf16 and fp16: the edge-block SDDMM (the op's
    schedule) and a degree split equal the rounded oracle on every edge."""
    w = synth.config4(seed=0, features=64)
    q16 = torch.from_numpy(w.dense["q"]).to(dtype)
    k16 = torch.from_numpy(w.dense["k"]).to(dtype)
    d_crow, d_col, d_q, d_k = dev(w.crow), dev(w.col), q16.cuda(), k16.cuda()
    _step(f"cfg4 {dtype} oracle (fp64 dots, all edges)")
    want = oracle.sddmm_rounded_16(w.crow, w.col, q16, k16, dtype).view(torch.int16)
    got = torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, d_k).cpu().view(torch.int16)
    assert torch.equal(got, want)
    got = torch.ops.autosage.sddmm_csr_split(d_crow, d_col, d_q, d_k, 4, 1024).cpu().view(torch.int16)
    assert torch.equal(got, want)


def test_config5_bf16_attention():
    """cfg5 in bf16 (``csr_attention_colslice``, one kernel with fp32 inside):
    every one of the 313M outputs lies between the rounded ends of
    [exact − ε, exact + ε], ε = 1e-5·|exact| + 1e-6, against the fp64
    attention of the same bf16 inputs (rounding is monotone)."""
    w = synth.config5(seed=0)
    q, k, v = (torch.from_numpy(w.dense[name]).to(torch.bfloat16) for name in ("q", "k", "v"))
    d_crow, d_col = dev(w.crow), dev(w.col)
    got = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, q.cuda(), k.cuda(), v.cuda(), 0.125)
    got = got.cpu().to(torch.float64).numpy()
    _step("cfg5 bf16 fp64 attention, all rows")
    exact = oracle.attention_f64(w.crow, w.col, q.float().numpy(), k.float().numpy(), v.float().numpy(), scale=0.125)
    bad = 0
    same = 0
    for start in range(0, exact.shape[0], 262144):
        part = slice(start, start + 262144)
        e = exact[part]
        eps = RTOL * np.abs(e) + ATOL
        lo, hi = _round16(e - eps, torch.bfloat16), _round16(e + eps, torch.bfloat16)
        g = got[part]
        bad += int(((g < lo) | (g > hi)).sum())
        same += int((g == _round16(e, torch.bfloat16)).sum())
    print(f"[parity] cfg5 bf16 attention: {got.size} outputs, {bad} outside the rounded bar, "
          f"{same / got.size:.4f} equal to round(exact)", flush=True)
    assert bad == 0
