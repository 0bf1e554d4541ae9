"""GPU parity of the row-softmax backward and of the attention backward.

The reference registers no autograd; these gradients are checked against the
oracle's restatement of the softmax backward (bit for bit: the kernel has no
``exp``) and against torch autograd of an fp64 composition of the attention
(SDDMM, row softmax, SpMM) on the CPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_common import case_graph, require_gpu, to_dev

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


def _attention_fp64(crow, col, q, k, v, scale):
    """out = softmax_row(scale·<q[row], k[col]>)·v in fp64 with torch autograd."""
    n = crow.size - 1
    rows = torch.repeat_interleave(torch.arange(n), torch.from_numpy(np.diff(crow)))
    c = torch.from_numpy(col)
    q64, k64, v64 = (torch.from_numpy(a).double().requires_grad_(True) for a in (q, k, v))
    s = (q64[rows] * k64[c]).sum(1) * scale
    m = torch.full((n,), -torch.inf, dtype=torch.float64).scatter_reduce(0, rows, s.detach(), "amax")
    ex = (s - m[rows]).exp()
    p = ex / torch.zeros(n, dtype=torch.float64).index_add(0, rows, ex)[rows]
    out = torch.zeros(n, v.shape[1], dtype=torch.float64).index_add(0, rows, p[:, None] * v64[c])
    return out, (q64, k64, v64)


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
    ref, leaves = _attention_fp64(crow, col, q, k, v, scale)
    ref.backward(torch.from_numpy(g).double())
    assert np.max(np.abs(out.detach().cpu().numpy() - ref.detach().numpy())) <= 1e-5 * np.max(np.abs(ref.detach().numpy()))
    for got, leaf in zip((d_q, d_k, d_v), leaves):
        want = leaf.grad.numpy()
        err = np.max(np.abs(got.grad.cpu().numpy() - want))
        assert err <= 2e-5 * np.max(np.abs(want)), (variant, err, np.max(np.abs(want)))


def test_colslice_attention_backward_schedules(monkeypatch):
    """The backward recomputes from the saved inputs, so the column-sliced
    op's gradients equal the fused op's bit for bit once column slices are
    off, and are deterministic with them on."""
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
