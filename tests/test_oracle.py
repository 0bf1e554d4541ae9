"""Pins the CPU oracle (oracle/) against independent references.

Each oracle function is checked against something that does not share its
code: PyTorch's own CSR product (the reference CPU path), brute-force dense
products in float64, reference known answers, numpy restatements and
closed forms — chosen so that a dropped term, a wrong index or a transposed
operand fails at least one check.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import synth


def _graph(rows, degree, seed, hubs=0, hub_degree=0, empty=0.0):
    crow, col = synth.random_csr(rows, degree, seed=seed, hub_rows=hubs, hub_degree=hub_degree,
                                 empty_fraction=empty)
    return crow, col


def _dense(crow, col, val, n):
    a = np.zeros((n, n), dtype=np.float64)
    for r in range(n):
        for e in range(crow[r], crow[r + 1]):
            a[r, col[e]] += 1.0 if val is None else float(val[e])
    return a


# --- SpMM -------------------------------------------------------------------


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [1, 7, 64, 128])
def test_spmm_seq_is_bit_identical_to_torch_cpu(weighted, features):
    crow, col = _graph(300, 9, seed=features, hubs=2, hub_degree=250, empty=0.1)
    rng = np.random.default_rng(1)
    val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
    x = rng.standard_normal((300, features)).astype(np.float32)
    expect = oracle.torch_cpu_spmm(torch.from_numpy(crow), torch.from_numpy(col),
                                   None if val is None else torch.from_numpy(val), torch.from_numpy(x))
    got = oracle.spmm_seq(crow, col, val, x)
    assert np.array_equal(got, expect.numpy())


@pytest.mark.parametrize("threads", [1, 4])
def test_spmm_seq_matches_torch_cpu_across_thread_counts(threads):
    old = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        crow, col = _graph(2000, 30, seed=5, hubs=3, hub_degree=1500)
        x = np.random.default_rng(2).standard_normal((2000, 64)).astype(np.float32)
        val = np.random.default_rng(3).random(col.size).astype(np.float32)
        expect = oracle.torch_cpu_spmm(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(val),
                                       torch.from_numpy(x))
        assert np.array_equal(oracle.spmm_seq(crow, col, val, x), expect.numpy())
    finally:
        torch.set_num_threads(old)


def test_spmm_reference_known_answers():
    # reference tests/test_cpu.py:25-32 (weights and an empty row)
    crow = np.array([0, 2, 2, 3])
    col = np.array([1, 2, 0])
    val = np.array([0.5, 2.0, -1.0], dtype=np.float32)
    x = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], dtype=np.float32)
    assert np.array_equal(oracle.spmm_seq(crow, col, val, x), [[11.5, 14.0], [0.0, 0.0], [-1.0, -2.0]])
    # reference tests/test_cpu.py:16-22 (destination rows)
    crow, col = oracle.numpy_edge_index_to_csr(np.array([[0, 1, 2, 3], [1, 2, 3, 0]]), 4)
    x = np.arange(12, dtype=np.float32).reshape(4, 3)
    y = oracle.spmm_seq(crow, col, None, x)
    assert np.array_equal(y[0], x[3]) and np.array_equal(y[1], x[0])


def test_spmm_order_is_sequential_not_pairwise():
    # 1e8 followed by eight 1s: a left-to-right fp32 chain keeps 1e8 (each +1
    # is below half an ulp), a pairwise or reassociated sum gives 1e8 + 8.
    crow = np.array([0, 9, 9])
    col = np.array([0] + [1] * 8)
    x = np.array([[1e8], [1.0]], dtype=np.float32)
    got = oracle.spmm_seq(crow, col, None, x)
    assert got[0, 0] == np.float32(1e8)
    assert np.float32(1e8) + np.float32(8.0) != np.float32(1e8)
    expect = oracle.torch_cpu_spmm(torch.from_numpy(crow), torch.from_numpy(col), None, torch.from_numpy(x))
    assert np.array_equal(got, expect.numpy())


def test_spmm_f64_matches_dense_brute_force():
    crow, col = _graph(40, 6, seed=11, hubs=1, hub_degree=30)
    rng = np.random.default_rng(4)
    val = rng.standard_normal(col.size).astype(np.float32)
    x = rng.standard_normal((40, 5)).astype(np.float32)
    expect = _dense(crow, col, val, 40) @ x.astype(np.float64)
    assert np.allclose(oracle.spmm_f64(crow, col, val, x), expect, rtol=1e-13, atol=1e-13)
    rows = np.array([3, 0, 39])
    assert np.allclose(oracle.spmm_f64(crow, col, val, x, rows=rows), expect[rows], rtol=1e-13, atol=1e-13)


def test_spmm_seq_row_subset_matches_full():
    crow, col = _graph(500, 12, seed=9)
    x = np.random.default_rng(0).standard_normal((500, 33)).astype(np.float32)
    full = oracle.spmm_seq(crow, col, None, x)
    rows = np.array([499, 0, 17, 17, 250])
    assert np.array_equal(oracle.spmm_seq(crow, col, None, x, rows=rows), full[rows])


# --- binning ------------------------------------------------------------------


@pytest.mark.parametrize("threshold", [1, 2, 9, 100, 10**9])
def test_bin_rows_matches_flatnonzero(threshold):
    crow, _ = _graph(1000, 8, seed=3, hubs=5, hub_degree=120, empty=0.05)
    deg = np.diff(crow)
    heavy, light = oracle.bin_rows(crow, threshold)
    assert np.array_equal(heavy, np.flatnonzero(deg >= threshold).astype(np.int32))
    assert np.array_equal(light, np.flatnonzero(deg < threshold).astype(np.int32))


def test_bin_rows_known_answer():
    crow = np.array([0, 3, 3, 10, 11, 16])  # degrees 3 0 7 1 5
    heavy, light = oracle.bin_rows(crow, 3)
    assert heavy.tolist() == [0, 2, 4] and light.tolist() == [1, 3]


# --- SDDMM --------------------------------------------------------------------


def test_sddmm_reference_known_answer():
    # reference tests/test_cpu.py:45-53
    crow = np.array([0, 2, 3])
    col = np.array([0, 1, 0])
    q = np.array([[1.0, 2.0], [3.0, 4.0]], dtype=np.float32)
    k = np.array([[2.0, 1.0], [1.0, 3.0]], dtype=np.float32)
    assert oracle.sddmm_ref(crow, col, q, k).tolist() == [4.0, 7.0, 10.0]


@pytest.mark.parametrize("features", [1, 17, 32, 64, 100, 128, 256])
def test_sddmm_ref_against_fp64_and_gather_dot(features):
    crow, col = _graph(200, 7, seed=features, hubs=2, hub_degree=150)
    rng = np.random.default_rng(features)
    q = rng.standard_normal((200, features)).astype(np.float32)
    k = rng.standard_normal((200, features)).astype(np.float32)
    got = oracle.sddmm_ref(crow, col, q, k)
    exact = oracle.sddmm_f64(crow, col, q, k)
    rows = np.repeat(np.arange(200), np.diff(crow))
    bound = 2 * features * np.finfo(np.float32).eps * (np.abs(q[rows]) * np.abs(k[col])).sum(1)
    assert np.all(np.abs(got - exact) <= bound + 1e-30)
    gd = oracle.torch_gather_dot(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(q),
                                 torch.from_numpy(k)).numpy()
    assert np.all(np.abs(got - gd) <= 2 * bound + 1e-30)


def test_sddmm_f64_matches_brute_force():
    crow, col = _graph(30, 5, seed=1)
    rng = np.random.default_rng(8)
    q = rng.standard_normal((30, 9)).astype(np.float32)
    k = rng.standard_normal((30, 9)).astype(np.float32)
    rows = np.repeat(np.arange(30), np.diff(crow))
    expect = np.einsum("ef,ef->e", q[rows].astype(np.float64), k[col].astype(np.float64))
    assert np.allclose(oracle.sddmm_f64(crow, col, q, k), expect, rtol=1e-14, atol=1e-14)


def test_sddmm_tree_order_differs_from_sequential():
    # Feature 0 carries a large value and features 1..32 small ones: the
    # reference order adds partial 0 (q0k0 + q32k32) last in its tree, so the
    # result differs from a left-to-right fp32 sum; the oracle must give the
    # tree value.
    f = 33
    q = np.ones((1, f), dtype=np.float32)
    k = np.full((1, f), 2.0 ** -24, dtype=np.float32)
    k[0, 0] = 1.0
    crow, col = np.array([0, 1]), np.array([0])
    got = oracle.sddmm_ref(crow, col, q, k)[0]
    # partials: p0 = 1 + 2^-24 -> 1 (rounds to even), p1..p31 = 2^-24; tree of
    # p1..p31 is exact (31·2^-24) and added to p0 in the final steps.
    seq = np.float32(0)
    for j in range(f):
        seq = np.float32(seq + q[0, j] * k[0, j])
    p = [np.float32(1.0)] + [np.float32(2.0 ** -24)] * 31
    for o in (16, 8, 4, 2, 1):
        for lane in range(o):
            p[lane] = np.float32(p[lane] + p[lane + o])
    assert got == p[0]
    assert got != seq


# --- softmax / attention --------------------------------------------------------


def test_row_softmax_known_answers():
    crow = np.array([0, 2, 3, 3])
    s = np.array([4.0, 7.0, 10.0], dtype=np.float32)
    p = oracle.row_softmax(crow, s)
    assert abs(p[:2].sum() - 1.0) < 1e-7
    assert p[2] == 1.0
    assert np.isclose(p[1] / p[0], np.exp(3.0), rtol=1e-6)


def test_row_softmax_against_torch_and_fp64():
    crow, col = _graph(400, 10, seed=21, hubs=3, hub_degree=300, empty=0.1)
    s = (np.random.default_rng(5).standard_normal(col.size) * 4).astype(np.float32)
    got = oracle.row_softmax(crow, s)
    ref = oracle.torch_row_softmax(torch.from_numpy(crow), torch.from_numpy(s)).numpy()
    exact = oracle.row_softmax_f64(crow, s.astype(np.float64))
    assert np.allclose(got, ref, rtol=2e-6, atol=1e-9)
    assert np.allclose(got, exact, rtol=2e-6, atol=1e-9)
    sums = np.add.reduceat(got, crow[:-1][np.diff(crow) > 0])
    assert np.allclose(sums, 1.0, atol=1e-5)


def test_attention_composition_against_fp64():
    crow, col = _graph(120, 6, seed=2, hubs=1, hub_degree=100)
    rng = np.random.default_rng(6)
    q = rng.standard_normal((120, 64)).astype(np.float32)
    k = rng.standard_normal((120, 64)).astype(np.float32)
    v = rng.standard_normal((120, 32)).astype(np.float32)
    got = oracle.attention_ref(crow, col, q, k, v, scale=0.125)
    exact = oracle.attention_f64(crow, col, q, k, v, scale=0.125)
    assert np.allclose(got, exact, rtol=1e-4, atol=1e-5)


def test_attention_f64_matches_dense_brute_force():
    """The fp64 attention the column-sliced kernels are held to, against a
    dense restatement: an N x N score matrix with -inf off the graph, a
    row-wise softmax (rows without edges give zeros) and a dense product."""
    crow, col = _graph(90, 7, seed=8, hubs=2, hub_degree=60, empty=0.1)
    rng = np.random.default_rng(9)
    # fp32 inputs (what the kernels take), widened exactly for the dense form
    q, k, v = (rng.standard_normal(shape).astype(np.float32).astype(np.float64)
               for shape in ((90, 16), (90, 16), (90, 12)))
    scores = np.full((90, 90), -np.inf)
    for r in range(90):
        for e in range(crow[r], crow[r + 1]):
            scores[r, col[e]] = 0.5 * (q[r] @ k[col[e]])
    has = np.isfinite(scores).any(axis=1)
    p = np.zeros_like(scores)
    p[has] = np.exp(scores[has] - scores[has].max(axis=1, keepdims=True))
    p[has] /= p[has].sum(axis=1, keepdims=True)
    got = oracle.attention_f64(crow, col, q, k, v, scale=0.5)
    assert np.allclose(got, p @ v, rtol=1e-12, atol=1e-13)
    assert np.all(got[~has] == 0)


def test_attention_f64_closed_forms():
    # zero scores: every row's output is the mean of its neighbours' V rows
    crow, col = _graph(60, 5, seed=3, empty=0.2)
    v = np.random.default_rng(1).standard_normal((60, 8)).astype(np.float32).astype(np.float64)
    zeros = np.zeros((60, 4))
    got = oracle.attention_f64(crow, col, zeros, zeros, v)
    for r in range(60):
        s, e = crow[r], crow[r + 1]
        want = v[col[s:e]].mean(axis=0) if e > s else np.zeros(8)
        assert np.allclose(got[r], want, rtol=1e-13, atol=1e-14)
    # two edges with scores 1 and 0: weights e/(1+e) and 1/(1+e); a row of
    # one edge gives that neighbour's V row; an empty row gives zeros
    crow2 = np.array([0, 2, 3, 3], dtype=np.int64)
    col2 = np.array([0, 1, 1], dtype=np.int64)
    q2 = np.array([[1.0], [1.0], [1.0]])
    k2 = np.array([[1.0], [0.0], [5.0]])
    v2 = np.array([[4.0], [8.0], [0.0]])
    got2 = oracle.attention_f64(crow2, col2, q2, k2, v2)
    e = np.e
    assert np.isclose(got2[0, 0], (4.0 * e + 8.0) / (1.0 + e), rtol=1e-15)
    assert got2[1, 0] == 8.0 and got2[2, 0] == 0.0


def test_edge_index_to_csr_restatement_matches_package():
    from autosage_amd.utils.csr import edge_index_to_csr

    rng = np.random.default_rng(0)
    ei = rng.integers(0, 50, size=(2, 400))
    crow, col = oracle.numpy_edge_index_to_csr(ei, 50)
    t_crow, t_col = edge_index_to_csr(torch.from_numpy(ei), 50)
    assert np.array_equal(crow, t_crow.numpy()) and np.array_equal(col, t_col.numpy())


# --- bf16 / fp16 SpMM -----------------------------------------------------------


def _round_16(exact: float, dtype) -> float:
    """Rounds a correctly rounded double to fp32 and then to dtype."""
    return torch.tensor([np.float32(exact)], dtype=torch.float32).to(dtype).float().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("weighted", [False, True])
def test_spmm_rounded_16_matches_exact_rational_sums(dtype, weighted):
    from fractions import Fraction

    crow, col = _graph(40, 6, seed=3, hubs=1, hub_degree=35, empty=0.1)
    rng = np.random.default_rng(11)
    x = torch.from_numpy(rng.standard_normal((40, 5)).astype(np.float32)).to(dtype)
    val = torch.from_numpy(rng.standard_normal(col.size).astype(np.float32)).to(dtype) if weighted else None
    got = oracle.spmm_rounded_16(crow, col, val, x, dtype).float().numpy()
    xf = x.float().numpy().astype(np.float64)
    vf = None if val is None else val.float().numpy().astype(np.float64)
    for r in range(40):
        for f in range(5):
            exact = Fraction(0)
            for e in range(crow[r], crow[r + 1]):
                w = Fraction(1) if vf is None else Fraction(vf[e])
                exact += w * Fraction(xf[col[e], f])
            assert got[r, f] == _round_16(float(exact), dtype), (r, f)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sddmm_rounded_16_matches_exact_rational_dots(dtype):
    from fractions import Fraction

    crow, col = _graph(30, 5, seed=4, hubs=1, hub_degree=25, empty=0.1)
    rng = np.random.default_rng(12)
    q = torch.from_numpy(rng.standard_normal((30, 13)).astype(np.float32)).to(dtype)
    k = torch.from_numpy(rng.standard_normal((30, 13)).astype(np.float32)).to(dtype)
    got = oracle.sddmm_rounded_16(crow, col, q, k, dtype).float().numpy()
    qf = q.float().numpy().astype(np.float64)
    kf = k.float().numpy().astype(np.float64)
    for r in range(30):
        for e in range(crow[r], crow[r + 1]):
            exact = sum((Fraction(qf[r, f]) * Fraction(kf[col[e], f]) for f in range(13)), Fraction(0))
            assert got[e] == _round_16(float(exact), dtype), (r, e)


def test_sddmm_rounded_16_exact_products_ties_and_overflow():
    crow = np.array([0, 1, 2, 3, 3], dtype=np.int64)
    col = np.array([1, 2, 3], dtype=np.int64)
    q = np.zeros((4, 2), dtype=np.float32)
    k = np.zeros((4, 2), dtype=np.float32)
    # row 0 · key 1: (1 + 2^-7)(1 + 2^-5) - 1 = 2^-5 + 2^-7 + 2^-12, i.e.
    # 2^-5·(1 + 2^-2 + 2^-7): exact in bf16.  Rounding the product to bf16
    # first would drop the 2^-12 and give 2^-5 + 2^-7.
    q[0] = [1 + 2.0**-7, -1.0]
    k[1] = [1 + 2.0**-5, 1.0]
    # row 1 · key 2: 1 + 2^-8, halfway between bf16 neighbours: even -> 1
    q[1] = [1.0, 2.0**-8]
    k[2] = [1.0, 1.0]
    # row 2 · key 3: 60000 + 60000 overflows fp16
    q[2] = [60000.0, 60000.0]
    k[3] = [1.0, 1.0]
    bf = oracle.sddmm_rounded_16(crow, col, q, k, torch.bfloat16).float().numpy()
    assert bf[0] == 2.0**-5 + 2.0**-7 + 2.0**-12
    assert bf[1] == 1.0
    h = oracle.sddmm_rounded_16(crow, col, q, k, torch.float16).float().numpy()
    assert h[2] == np.inf
    assert h[1] == 1.00390625  # fp16 holds 1 + 2^-8


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_row_softmax_rounded_16_closed_forms(dtype):
    """Rows of 4 equal scores, 1 score, scores (1, 0) and 1,000 equal scores:
    1/4, 1, e/(1+e) and 1/1000, each rounded once to the 16-bit type (a
    softmax computed in the 16-bit type itself, e.g. its denominator summed
    in bf16, stalls at 256 and gives 1/256 for the last row)."""
    crow = np.array([0, 4, 5, 7, 1007], dtype=np.int64)
    scores = np.zeros(1007, dtype=np.float32)
    scores[4] = 3.0
    scores[5] = 1.0
    got = oracle.row_softmax_rounded_16(crow, scores, dtype).float().numpy()
    assert np.all(got[:4] == 0.25) and got[4] == 1.0
    e = np.exp(1.0)
    assert got[5] == _round_16(e / (1 + e), dtype) and got[6] == _round_16(1 / (1 + e), dtype)
    assert np.all(got[7:] == _round_16(1e-3, dtype))


def _softmax_backward_lane_order(crow, probs, grad):
    """Independent restatement of the lane order in numpy float32, for values
    whose products and partial sums are exact in fp64 (so each fmaf is one
    rounding to fp32)."""
    out = np.zeros(probs.size, dtype=np.float32)
    for r in range(crow.size - 1):
        s0, s1 = crow[r], crow[r + 1]
        if s0 == s1:
            continue
        lanes = [np.float32(0.0)] * 64
        for e in range(s0, s1):
            lanes[(e - s0) % 64] = np.float32(np.float64(grad[e]) * np.float64(probs[e]) + np.float64(lanes[(e - s0) % 64]))
        for o in (32, 16, 8, 4, 2, 1):
            lanes = [np.float32(lanes[l] + lanes[l ^ o]) for l in range(64)]
        t = lanes[0]
        out[s0:s1] = probs[s0:s1] * (grad[s0:s1] - t)
    return out


def test_row_softmax_backward_lane_order():
    rng = np.random.default_rng(21)
    deg = np.array([200, 64, 1, 65, 0, 130])
    crow = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    nnz = int(crow[-1])
    # probabilities k/2^14, gradients j/2^8 in [0, 8): exact products, sums
    # that outgrow fp32's 24 bits (so the order of the additions shows)
    probs = (rng.integers(0, 1 << 14, nnz) / float(1 << 14)).astype(np.float32)
    grad = (rng.integers(0, 1 << 11, nnz) / 256.0).astype(np.float32)
    got = oracle.row_softmax_backward(crow, probs, grad)
    want = _softmax_backward_lane_order(crow, probs, grad)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the order matters here: a sequential fp32 sum gives other bits somewhere
    seq = np.zeros(nnz, dtype=np.float32)
    for r in range(deg.size):
        s0, s1 = crow[r], crow[r + 1]
        t = np.float32(0.0)
        for e in range(s0, s1):
            t = np.float32(np.float64(grad[e]) * np.float64(probs[e]) + np.float64(t))
        seq[s0:s1] = probs[s0:s1] * (grad[s0:s1] - t)
    assert not np.array_equal(seq, want)


def test_row_softmax_backward_closed_forms_and_fp64():
    # uniform probabilities with a constant gradient, and a one-entry row: 0
    crow = np.array([0, 4, 5], dtype=np.int64)
    probs = np.array([0.25, 0.25, 0.25, 0.25, 1.0], dtype=np.float32)
    grad = np.array([3.0, 3.0, 3.0, 3.0, -7.5], dtype=np.float32)
    assert np.all(oracle.row_softmax_backward(crow, probs, grad) == 0.0)
    # torch autograd of the fp64 softmax
    crow, col = _graph(60, 12, seed=9, hubs=1, hub_degree=300, empty=0.1)
    rng = np.random.default_rng(10)
    scores = torch.from_numpy(rng.standard_normal(col.size) * 3).requires_grad_(True)
    rows = torch.repeat_interleave(torch.arange(60), torch.from_numpy(np.diff(crow)))
    m = torch.zeros(60, dtype=torch.float64).scatter_reduce(0, rows, scores.detach(), "amax", include_self=False)
    ex = (scores - m[rows]).exp()
    p64 = ex / torch.zeros(60, dtype=torch.float64).index_add(0, rows, ex)[rows]
    g = torch.from_numpy(rng.standard_normal(col.size))
    (p64 * g).sum().backward()
    got = oracle.row_softmax_backward(crow, p64.detach().numpy().astype(np.float32), g.numpy().astype(np.float32))
    want = scores.grad.numpy()
    assert np.max(np.abs(got - want)) <= 1e-6 * max(1.0, np.max(np.abs(want)))


def test_spmm_rounded_16_ties_and_overflow():
    crow = np.array([0, 2, 4, 7, 9], dtype=np.int64)
    col = np.array([0, 1, 0, 2, 0, 1, 3, 4, 4], dtype=np.int64)
    # x[:, 0]: 1, 2^-8, 3·2^-8, 2^-30, 60000
    x = np.array([[1.0], [2.0**-8], [3 * 2.0**-8], [2.0**-30], [60000.0]], dtype=np.float32)
    bf = oracle.spmm_rounded_16(crow, col, None, x, torch.bfloat16).float().numpy()[:, 0]
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7: even -> 1
    assert bf[0] == 1.0
    # 1 + 3·2^-8 is halfway between 1 + 2^-7 and 1 + 2^-6: even -> 1 + 2^-6
    assert bf[1] == 1.0 + 2.0**-6
    # 1 + 2^-8 + 2^-30 is above the tie, but fp32 drops the 2^-30 first: 1
    assert bf[2] == 1.0
    h = oracle.spmm_rounded_16(crow, col, None, x, torch.float16).float().numpy()[:, 0]
    assert h[3] == np.inf  # 120000 overflows fp16
    assert h[0] == 1.00390625  # fp16 represents 1 + 2^-8 exactly


def test_oracle_results_do_not_depend_on_the_thread_count(tmp_path):
    """The row loops run on OpenMP threads, one row per thread: the same bits
    with one thread (a child process with OMP_NUM_THREADS=1) as with many."""
    import subprocess
    import sys

    crow, col = _graph(3000, 20, seed=31, hubs=3, hub_degree=2000, empty=0.1)
    rng = np.random.default_rng(32)
    val = rng.standard_normal(col.size).astype(np.float32)
    x = rng.standard_normal((3000, 24)).astype(np.float32)
    q = rng.standard_normal((3000, 8)).astype(np.float32)
    np.savez(tmp_path / "in.npz", crow=crow, col=col, val=val, x=x, q=q)
    script = (
        "import sys, numpy as np; sys.path.insert(0, sys.argv[1]); import oracle; d = np.load(sys.argv[2]);"
        "np.savez(sys.argv[3], seq=oracle.spmm_seq(d['crow'], d['col'], d['val'], d['x']),"
        " f64=oracle.spmm_f64(d['crow'], d['col'], d['val'], d['x']),"
        " dot=oracle.sddmm_ref(d['crow'], d['col'], d['q'], d['q']),"
        " att=oracle.attention_f64(d['crow'], d['col'], d['q'], d['q'], d['x'], 0.3))"
    )
    root = str(Path(oracle.__file__).resolve().parent.parent)
    env = {**__import__("os").environ, "OMP_NUM_THREADS": "1"}
    subprocess.run([sys.executable, "-c", script, root, str(tmp_path / "in.npz"), str(tmp_path / "one.npz")],
                   check=True, env=env)
    one = np.load(tmp_path / "one.npz")
    many = {
        "seq": oracle.spmm_seq(crow, col, val, x),
        "f64": oracle.spmm_f64(crow, col, val, x),
        "dot": oracle.sddmm_ref(crow, col, q, q),
        "att": oracle.attention_f64(crow, col, q, q, x, 0.3),
    }
    for name, value in many.items():
        assert np.array_equal(one[name].view(np.uint8), value.view(np.uint8)), name
