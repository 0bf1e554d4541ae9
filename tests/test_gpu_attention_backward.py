"""GPU parity of the row-softmax backward and of the attention backward.

The reference registers no autograd; these gradients are checked against the
oracle's restatement of the softmax backward (bit for bit: the kernel has no
``exp``) and against torch autograd of an fp64 composition of the attention
(SDDMM, row softmax, SpMM) on the CPU: every gradient element within
1e-5·|fp64| + 1e-6, and within that bar of the reference's own fp32 autograd
gradient or, where not, both on opposite sides of the fp64 gradient within its
bar, or the reference off the bar and the kernel closer.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_common import case_graph, elementwise_parity, require_gpu, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _probs_and_grad(crow, nnz, seed):
    rng = np.random.default_rng(seed)
    scores = (rng.standard_normal(nnz) * 2).astype(np.float32)
    probs = oracle.row_softmax(crow, scores)
    grad = rng.standard_normal(nnz).astype(np.float32)
    return scores, probs, grad


def test_softmax_backward_matches_the_oracle_bitwise():
    from autosage_amd import _native

    crow, col = case_graph(3000, 9, seed=3, hubs=3, hub_degree=2500, empty=0.05)
    _, probs, grad = _probs_and_grad(crow, col.size, 4)
    d_crow, d_p, d_g = to_dev(crow, probs, grad)
    got = _native.csr_row_softmax_backward_impl(d_crow, d_p, d_g).cpu().numpy()
    want = oracle.row_softmax_backward(crow, probs, grad)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for dtype in (torch.bfloat16, torch.float16):
        p16, g16 = torch.from_numpy(probs).to(dtype), torch.from_numpy(grad).to(dtype)
        got16 = _native.csr_row_softmax_backward_impl(d_crow, p16.cuda(), g16.cuda()).cpu()
        want16 = oracle.row_softmax_backward_rounded_16(crow, p16, g16, dtype)
        assert torch.equal(got16.view(torch.int16), want16.view(torch.int16)), dtype


def test_softmax_op_autograd():
    crow, col = case_graph(2000, 12, seed=5, hubs=2, hub_degree=1800, empty=0.05)
    scores, _, grad = _probs_and_grad(crow, col.size, 6)
    d_crow, = to_dev(crow)
    d_s = torch.from_numpy(scores).cuda().requires_grad_(True)
    p = torch.ops.autosage.csr_row_softmax(d_crow, d_s)
    p.backward(torch.from_numpy(grad).cuda())
    want = oracle.row_softmax_backward(crow, p.detach().cpu().numpy(), grad)
    assert np.array_equal(d_s.grad.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _attention_torch(crow, col, q, k, v, scale, dtype=torch.float64):
    """out = softmax_row(scale·<q[row], k[col]>)·v with torch autograd on the
    CPU: in fp64 the near-exact gradients, in fp32 the reference's own
    (its composition, autosage/_auto.py:744-780, has no custom backward)."""
    n = crow.size - 1
    rows = torch.repeat_interleave(torch.arange(n), torch.from_numpy(np.diff(crow)))
    c = torch.from_numpy(col)
    qq, kk, vv = (torch.from_numpy(a).to(dtype).requires_grad_(True) for a in (q, k, v))
    s = (qq[rows] * kk[c]).sum(1) * scale
    m = torch.full((n,), -torch.inf, dtype=dtype).scatter_reduce(0, rows, s.detach(), "amax")
    ex = (s - m[rows]).exp()
    p = ex / torch.zeros(n, dtype=dtype).index_add(0, rows, ex)[rows]
    out = torch.zeros(n, v.shape[1], dtype=dtype).index_add(0, rows, p[:, None] * vv[c])
    return out, (qq, kk, vv)


def _attention_fp64(crow, col, q, k, v, scale):
    return _attention_torch(crow, col, q, k, v, scale, torch.float64)


RTOL = 1e-5
ATOL = 1e-6


def _assert_gradients_per_element(got_grads, crow, col, q, k, v, g, scale, label):
    """Every element of dQ, dK, dV within 1e-5·|want| + 1e-6 of the fp64
    autograd gradient, and within that bar of the reference's fp32 autograd
    gradient or arbitrated against fp64 (``elementwise_parity`` with case (d):
    the reference's autograd sums each gradient's terms in its own order, so
    two results on opposite sides of the exact one, both within its bar,
    count as agreeing)."""
    exact_out, exact = _attention_torch(crow, col, q, k, v, scale, torch.float64)
    exact_out.backward(torch.from_numpy(g).double())
    ref_out, ref = _attention_torch(crow, col, q, k, v, scale, torch.float32)
    ref_out.backward(torch.from_numpy(g))
    for name, got, e_leaf, r_leaf in zip("QKV", got_grads, exact, ref):
        want = e_leaf.grad.numpy()
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= RTOL * np.abs(want) + ATOL), (label, name, float(np.max(err / (RTOL * np.abs(want) + ATOL))))
        elementwise_parity(got, r_leaf.grad.numpy(), want, tight_rel=RTOL, tight_abs=ATOL,
                           accept_both_within_bar=True)


@pytest.mark.parametrize("variant", ["fused", "colslice", "stages"])
def test_attention_gradients(variant):
    crow, col = case_graph(1500, 10, seed=8, hubs=2, hub_degree=1200, empty=0.05)
    rng = np.random.default_rng(9)
    q = (rng.standard_normal((1500, 64)) * 0.25).astype(np.float32)
    k = (rng.standard_normal((1500, 64)) * 0.25).astype(np.float32)
    v = rng.standard_normal((1500, 32)).astype(np.float32)
    g = rng.standard_normal((1500, 32)).astype(np.float32)
    scale = 0.125
    d_crow, d_col = to_dev(crow, col)
    d_q, d_k, d_v = (torch.from_numpy(a).cuda().requires_grad_(True) for a in (q, k, v))
    if variant == "fused":
        out = torch.ops.autosage.csr_attention(d_crow, d_col, d_q, d_k, d_v, scale)
    elif variant == "colslice":
        out = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, d_q, d_k, d_v, scale)
    else:
        # the three op stages, each with its own backward
        s = torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, d_k) * scale
        p = torch.ops.autosage.csr_row_softmax(d_crow, s)
        out = torch.ops.autosage.spmm_csr(d_crow, d_col, p, d_v)
    out.backward(torch.from_numpy(g).cuda())
    ref, _ = _attention_fp64(crow, col, q, k, v, scale)
    assert np.max(np.abs(out.detach().cpu().numpy() - ref.detach().numpy())) <= 1e-5 * np.max(np.abs(ref.detach().numpy()))
    _assert_gradients_per_element([t.grad.cpu().numpy() for t in (d_q, d_k, d_v)], crow, col, q, k, v, g, scale,
                                  variant)


def test_colslice_attention_backward_schedules(monkeypatch):
    """With column slices off the column-sliced op's backward is the fused
    op's recomputing chain (same bits); with them on it runs the two native
    passes, deterministic and within 2e-5 (max-norm) of that chain."""
    crow, col = case_graph(1200, 12, seed=10, hubs=2, hub_degree=1100, empty=0.05)
    rng = np.random.default_rng(11)
    arrays = [(rng.standard_normal((1200, f)) * 0.25).astype(np.float32) for f in (64, 64, 48)]
    g = torch.from_numpy(rng.standard_normal((1200, 48)).astype(np.float32)).cuda()
    d_crow, d_col = to_dev(crow, col)

    def grads(op):
        leaves = [torch.from_numpy(a).cuda().requires_grad_(True) for a in arrays]
        op(d_crow, d_col, *leaves, 0.125).backward(g)
        return [leaf.grad for leaf in leaves]

    sliced = grads(torch.ops.autosage.csr_attention_colslice)
    assert all(torch.equal(a, b) for a, b in zip(sliced, grads(torch.ops.autosage.csr_attention_colslice)))
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "off")
    fused = grads(torch.ops.autosage.csr_attention)
    off = grads(torch.ops.autosage.csr_attention_colslice)
    assert all(torch.equal(a, b) for a, b in zip(off, fused))
    for a, b in zip(sliced, fused):
        assert torch.max(torch.abs(a - b)) <= 2e-5 * torch.max(torch.abs(b))


def _symmetric_hub_graph(n, seed):
    """A = H ∪ Hᵀ for a hub graph H: symmetric, so its hubs are also hubs of
    Aᵀ (both backward passes slice rows), with empty rows and the columns of
    every row shuffled (the op sorts a copy)."""
    h_crow, h_col = case_graph(n, 9, seed=seed, hubs=3, hub_degree=1800, empty=0.05)
    rows = np.concatenate([np.repeat(np.arange(n), np.diff(h_crow)), h_col])
    cols = np.concatenate([h_col, np.repeat(np.arange(n), np.diff(h_crow))])
    keys = np.unique(rows * n + cols)
    r, c = keys // n, keys % n
    crow = np.concatenate([[0], np.cumsum(np.bincount(r, minlength=n))]).astype(np.int64)
    rng = np.random.default_rng(seed)
    perm = np.concatenate([rng.permutation(np.arange(crow[i], crow[i + 1])) for i in range(n)])
    col = c[perm].astype(np.int64)
    assert np.diff(crow).max() >= 1800
    return crow, col, rng


@pytest.mark.parametrize("fqk, fv", [(64, 128), (32, 48), (128, 128), (256, 64), (4, 8)])
def test_two_pass_attention_backward(fqk, fv):
    """The column-sliced op's backward runs the two native passes: on a graph
    with out- and in-degree hubs (both passes slice rows), empty rows and
    columns out of order, every gradient element meets the per-element bars,
    and a second run gives the same bits.  The comparison with the
    recomputing chain is in the schedules test above."""
    n = 2500
    crow, col, rng = _symmetric_hub_graph(n, seed=fqk + fv)
    q = (rng.standard_normal((n, fqk)) * 0.25).astype(np.float32)
    k = (rng.standard_normal((n, fqk)) * 0.25).astype(np.float32)
    v = rng.standard_normal((n, fv)).astype(np.float32)
    g = rng.standard_normal((n, fv)).astype(np.float32)
    d_crow, d_col = to_dev(crow, col)
    leaves = [torch.from_numpy(a).cuda().requires_grad_(True) for a in (q, k, v)]
    out = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *leaves, 0.125)
    out.backward(torch.from_numpy(g).cuda())
    _assert_gradients_per_element([t.grad.cpu().numpy() for t in leaves], crow, col, q, k, v, g, 0.125,
                                  f"two-pass {fqk}/{fv}")
    # deterministic
    again = [torch.from_numpy(a).cuda().requires_grad_(True) for a in (q, k, v)]
    torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *again, 0.125).backward(torch.from_numpy(g).cuda())
    assert all(torch.equal(a.grad, b.grad) for a, b in zip(leaves, again))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_two_pass_attention_backward_rows_without_edges_and_chunks(dtype, monkeypatch):
    """Rows and columns without edges get zero gradients; a small workspace
    (partial states for a few sliced rows) runs the sliced rows in chunks
    with the same bits."""
    n = 3000
    crow, col = case_graph(n, 7, seed=4, hubs=30, hub_degree=900, empty=0.2)
    col = col * (n - 100) // n  # columns n - 100 .. n - 1 get no edge (order kept, repeats allowed)
    rng = np.random.default_rng(5)
    arrays = [(rng.standard_normal((n, f)) * 0.25).astype(np.float32) for f in (64, 64, 128)]
    g = torch.from_numpy(rng.standard_normal((n, 128)).astype(np.float32)).cuda().to(dtype)
    d_crow, d_col = to_dev(crow, col)
    half = dtype != torch.float32

    def grads():
        leaves = [torch.from_numpy(a).cuda().to(dtype).requires_grad_(True) for a in arrays]
        torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *leaves, 0.125).backward(g)
        return [leaf.grad for leaf in leaves]

    first = grads()
    empty_rows = torch.from_numpy(np.diff(crow) == 0).cuda()
    assert torch.count_nonzero(first[0][empty_rows]).item() == 0
    unused = torch.from_numpy(np.bincount(col, minlength=n) == 0).cuda()
    assert unused.any() and torch.count_nonzero(first[1][unused]).item() == 0
    assert torch.count_nonzero(first[2][unused]).item() == 0
    from autosage_amd import _native

    lib = _native.library()
    # the preferred size less one row of partials (8 slices of the larger of
    # pass 1's and pass 2's states) and the alignment slack (5·256 bytes)
    row = 8 * max(64 * (2 if half else 1) + 3, 64 + 128) * 4
    fixed = lib.as_csr_attention_backward_workspace_bytes(n, 0, 64, 128, 1 if half else 0) - row - 1280
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", str((fixed + 3 * row + 1280) / 2**20))
    chunked = grads()
    assert all(torch.equal(a, b) for a, b in zip(first, chunked))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_attention_plans_give_the_bits_of_per_call_set_up(dtype, monkeypatch):
    """Per-graph plans (slice points and row order of A, and for the backward
    of Aᵀ) give the bits of calls that build them each time, forward and
    backward; the plans go with their graphs."""
    import gc

    from autosage_amd import _native

    n = 3000
    crow, col = case_graph(n, 9, seed=12, hubs=20, hub_degree=1200, empty=0.05)
    rng = np.random.default_rng(13)
    arrays = [(rng.standard_normal((n, f)) * 0.25).astype(np.float32) for f in (64, 64, 128)]
    g = torch.from_numpy(rng.standard_normal((n, 128)).astype(np.float32)).cuda().to(dtype)
    d_crow, d_col = to_dev(crow, col)
    before = len(_native._PLAN_MEMO)

    def run():
        leaves = [torch.from_numpy(a).cuda().to(dtype).requires_grad_(True) for a in arrays]
        out = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *leaves, 0.125)
        out.backward(g)
        return [out] + [leaf.grad for leaf in leaves]

    planned = run()
    # the plan of A (forward and pass 1) and of Aᵀ (pass 2)
    assert len(_native._PLAN_MEMO) == before + 2
    monkeypatch.setenv("AUTOSAGE_COLSLICE_PLAN", "off")
    unplanned = run()
    monkeypatch.delenv("AUTOSAGE_COLSLICE_PLAN")
    assert all(torch.equal(a, b) for a, b in zip(planned, unplanned))
    assert torch.equal(planned[0], run()[0])
    from autosage_amd import _autograd

    del d_col
    _autograd._TRANSPOSE_MEMO.clear()
    gc.collect()
    assert len(_native._PLAN_MEMO) == before


# Rounding of a gradient to the 16-bit type: at most half an ulp, 2^-9 of the
# value for bf16 and 2^-11 for fp16 (normal range); the bars allow twice that
# plus fp32 error relative to the largest gradient.
UNIT_16 = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -10}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fqk, fv", [(64, 128), (32, 48), (128, 128), (256, 64), (8, 8), (512, 16)])
def test_two_pass_attention_backward_16(dtype, fqk, fv, monkeypatch):
    """bf16 / fp16: the two native passes in fp32, each gradient rounded once.
    Every element is within UNIT_16·|exact| + 2e-5·max|exact| of fp64 autograd
    of the composition on the same (exactly converted) 16-bit inputs; the
    result is deterministic and at least as accurate (root-mean-square error)
    as the chain of native 16-bit stages (column slices off), which rounds
    scores and probabilities."""
    n = 2500
    crow, col, rng = _symmetric_hub_graph(n, seed=fqk + 7 * fv)
    arrays = [torch.from_numpy((rng.standard_normal((n, f)) * s_).astype(np.float32)).to(dtype)
              for f, s_ in ((fqk, 0.25), (fqk, 0.25), (fv, 1.0), (fv, 1.0))]
    q, k, v, g = arrays
    d_crow, d_col = to_dev(crow, col)

    def grads():
        leaves = [t.cuda().requires_grad_(True) for t in (q, k, v)]
        torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *leaves, 0.125).backward(g.cuda())
        return [leaf.grad for leaf in leaves]

    got = grads()
    assert all(t.dtype == dtype for t in got)
    ref, ref_leaves = _attention_fp64(crow, col, *(t.float().numpy() for t in (q, k, v)), 0.125)
    ref.backward(g.double())
    errors = []
    for t, leaf in zip(got, ref_leaves):
        want = leaf.grad.numpy()
        err = np.abs(t.cpu().double().numpy() - want)
        bar = UNIT_16[dtype] * np.abs(want) + 2e-5 * np.max(np.abs(want))
        assert np.all(err <= bar), (float(np.max(err - bar)), float(np.max(np.abs(want))))
        errors.append(float(np.sqrt(np.mean(err ** 2))))
    assert all(torch.equal(a, b) for a, b in zip(got, grads()))
    # root-mean-square errors: both results carry the final rounding, the
    # chain also the rounding of every score and probability
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "off")
    chained = grads()
    for t, leaf, e in zip(chained, ref_leaves, errors):
        assert e <= float(np.sqrt(np.mean((t.cpu().double().numpy() - leaf.grad.numpy()) ** 2)))
