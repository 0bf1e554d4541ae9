"""Backward formulas of the native operators (no reference counterpart: the
reference registers no autograd).

CPU: the CSR transpose used by the backward.  GPU: gradients through
torch.ops.autosage.* equal the oracle's sequential products bit for bit
(dX = Aᵀ·dY over the transposed CSR, dval / dQ / dK as SDDMM / SpMM), and
agree with a float64 dense autograd reference within 1e-5 relative."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from autosage_amd._autograd import csr_transpose
from tests.gpu_common import bitwise_equal, case_graph, require_gpu, to_dev


def test_csr_transpose_matches_dense_transpose():
    crow, col = case_graph(300, 6, seed=3, hubs=2, hub_degree=200, empty=0.1)
    t_crow, t_col, perm = csr_transpose(torch.from_numpy(crow), torch.from_numpy(col))
    n = 300
    rows = np.repeat(np.arange(n), np.diff(crow))
    # rows of Aᵀ list source rows ascending; perm maps edges of Aᵀ to edges of A
    order = np.lexsort((np.arange(col.size), col))
    assert np.array_equal(perm.numpy(), order)
    assert np.array_equal(t_col.numpy(), rows[order])
    assert np.array_equal(t_crow.numpy(), np.concatenate([[0], np.cumsum(np.bincount(col, minlength=n))]))


def test_csr_transpose_memo_is_per_tensor_object():
    crow = torch.tensor([0, 2, 3, 3])
    col = torch.tensor([2, 0, 0])
    first = csr_transpose(crow, col)
    assert csr_transpose(crow, col) is first
    col[0] = 1
    second = csr_transpose(crow, col)
    assert second is not first
    # A rows: 0 -> {1, 0}, 1 -> {0}; Aᵀ rows: 0 <- {0, 1}, 1 <- {0}
    assert second[0].tolist() == [0, 2, 3, 3]
    assert second[1].tolist() == [0, 1, 0]
    assert second[2].tolist() == [1, 2, 0]


def _dense(crow, col, val, n):
    a = torch.zeros(n, n, dtype=torch.float64)
    rows = torch.repeat_interleave(torch.arange(n), torch.from_numpy(np.diff(crow)))
    a.index_put_((rows, torch.from_numpy(col)), torch.from_numpy(val).double(), accumulate=True)
    return a


@pytest.mark.gpu
@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("features", [64, 128, 33])
def test_spmm_backward(split, features):
    require_gpu()
    n = 800
    crow, col = case_graph(n, 9, seed=features, hubs=3, hub_degree=600, empty=0.05)
    rng = np.random.default_rng(features)
    val = rng.standard_normal(col.size).astype(np.float32)
    x = rng.standard_normal((n, features)).astype(np.float32)
    g = rng.standard_normal((n, features)).astype(np.float32)
    d_crow, d_col = to_dev(crow, col)
    d_val = torch.from_numpy(val).cuda().requires_grad_(True)
    d_x = torch.from_numpy(x).cuda().requires_grad_(True)
    if split:
        y = torch.ops.autosage.spmm_csr_split(d_crow, d_col, d_val, d_x, 128, 2, 300)
    else:
        y = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x)
    y.backward(torch.from_numpy(g).cuda())
    t_crow, t_col, perm = csr_transpose(torch.from_numpy(crow), torch.from_numpy(col))
    assert bitwise_equal(d_x.grad, oracle.spmm_seq(t_crow, t_col, val[perm.numpy()], g))
    assert bitwise_equal(d_val.grad, oracle.sddmm_ref(crow, col, g, x))
    # float64 dense reference
    a = _dense(crow, col, val, n).requires_grad_(True)
    x64 = torch.from_numpy(x).double().requires_grad_(True)
    (a @ x64).backward(torch.from_numpy(g).double())
    rows = torch.repeat_interleave(torch.arange(n), torch.from_numpy(np.diff(crow)))
    dval64 = a.grad[rows, torch.from_numpy(col)].numpy()
    assert np.allclose(d_x.grad.cpu().numpy(), x64.grad.numpy(), rtol=1e-5, atol=1e-4)
    assert np.allclose(d_val.grad.cpu().numpy(), dval64, rtol=1e-5, atol=1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("features", [64, 128])
def test_spmm_backward_with_in_degree_hubs(features):
    """A = Hᵀ for a graph H with hub rows: A's columns have in-degree hubs, so
    the transposed CSR of the backward (= H) has rows of 3,000 edges.  dX of
    the exact op then runs the degree-split schedule (rows of >= 1024 edges
    split over waves) and must still equal the oracle's sequential product
    over Aᵀ bit for bit; dX of the column-sliced op slices those rows and
    must be within 1e-6·|fp64| of the fp64 product."""
    require_gpu()
    n = 6000
    h_crow, h_col = case_graph(n, 6, seed=features, hubs=4, hub_degree=3000, empty=0.05)
    a_crow, a_col, _ = csr_transpose(torch.from_numpy(h_crow), torch.from_numpy(h_col))
    crow, col = a_crow.numpy(), a_col.numpy()
    t_crow, t_col, perm = csr_transpose(a_crow, a_col)
    assert np.diff(t_crow.numpy()).max() >= 3000 and np.diff(crow).max() < 1024
    rng = np.random.default_rng(features + 1)
    val = rng.standard_normal(col.size).astype(np.float32)
    x = rng.standard_normal((n, features)).astype(np.float32)
    g = rng.standard_normal((n, features)).astype(np.float32)
    d_crow, d_col = to_dev(crow, col)
    for sliced in (False, True):
        d_val = torch.from_numpy(val).cuda().requires_grad_(True)
        d_x = torch.from_numpy(x).cuda().requires_grad_(True)
        op = torch.ops.autosage.spmm_csr_colslice if sliced else torch.ops.autosage.spmm_csr
        op(d_crow, d_col, d_val, d_x).backward(torch.from_numpy(g).cuda())
        v_t = val[perm.numpy()]
        if sliced:
            exact = oracle.spmm_f64(t_crow.numpy(), t_col.numpy(), v_t, g)
            got = d_x.grad.cpu().numpy()
            assert np.all(np.abs(got - exact) <= 1e-6 * np.abs(exact) + 1e-9)
        else:
            assert bitwise_equal(d_x.grad, oracle.spmm_seq(t_crow, t_col, v_t, g))
        assert bitwise_equal(d_val.grad, oracle.sddmm_ref(crow, col, g, x))


@pytest.mark.gpu
def test_spmm_backward_unweighted_and_no_grad_inputs():
    require_gpu()
    crow, col = case_graph(500, 8, seed=1)
    x = torch.randn(500, 64, device="cuda", requires_grad=True)
    d_crow, d_col = to_dev(crow, col)
    y = torch.ops.autosage.spmm_csr(d_crow, d_col, None, x)
    g = torch.randn_like(y)
    y.backward(g)
    t_crow, t_col, _ = csr_transpose(torch.from_numpy(crow), torch.from_numpy(col))
    assert bitwise_equal(x.grad, oracle.spmm_seq(t_crow, t_col, None, g.cpu()))


@pytest.mark.gpu
@pytest.mark.parametrize("split", [False, True])
def test_sddmm_backward(split):
    require_gpu()
    n, f = 700, 64
    crow, col = case_graph(n, 10, seed=7, hubs=2, hub_degree=500)
    rng = np.random.default_rng(7)
    q = rng.standard_normal((n, f)).astype(np.float32)
    k = rng.standard_normal((n, f)).astype(np.float32)
    gs = rng.standard_normal(col.size).astype(np.float32)
    d_crow, d_col = to_dev(crow, col)
    d_q = torch.from_numpy(q).cuda().requires_grad_(True)
    d_k = torch.from_numpy(k).cuda().requires_grad_(True)
    if split:
        s = torch.ops.autosage.sddmm_csr_split(d_crow, d_col, d_q, d_k, 4, 256)
    else:
        s = torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, d_k)
    s.backward(torch.from_numpy(gs).cuda())
    assert bitwise_equal(d_q.grad, oracle.spmm_seq(crow, col, gs, k))
    t_crow, t_col, perm = csr_transpose(torch.from_numpy(crow), torch.from_numpy(col))
    assert bitwise_equal(d_k.grad, oracle.spmm_seq(t_crow, t_col, gs[perm.numpy()], q))
    rows = np.repeat(np.arange(n), np.diff(crow))
    q64 = torch.from_numpy(q).double().requires_grad_(True)
    k64 = torch.from_numpy(k).double().requires_grad_(True)
    s64 = (q64[torch.from_numpy(rows)] * k64[torch.from_numpy(col)]).sum(1)
    s64.backward(torch.from_numpy(gs).double())
    assert np.allclose(d_q.grad.cpu().numpy(), q64.grad.numpy(), rtol=1e-5, atol=1e-4)
    assert np.allclose(d_k.grad.cpu().numpy(), k64.grad.numpy(), rtol=1e-5, atol=1e-4)


@pytest.mark.gpu
def test_conv_layer_trains_on_native_kernels():
    require_gpu()
    import autosage_amd

    torch.manual_seed(0)
    n, fin, fout = 600, 32, 8
    crow, col = case_graph(n, 6, seed=11)
    rows = np.repeat(np.arange(n), np.diff(crow))
    edge_index = torch.from_numpy(np.stack([col, rows])).cuda()  # src -> dst
    x = torch.randn(n, fin, device="cuda")
    w = torch.rand(col.size, device="cuda", requires_grad=True)
    layer = autosage_amd.AutoSAGEConv(fin, fout, mode="native").cuda()
    out = layer(x, edge_index, w)
    loss = out.square().mean()
    loss.backward()
    assert w.grad is not None and layer.linear.weight.grad is not None
    # float64 CPU reference of the same layer
    ref = autosage_amd.AutoSAGEConv(fin, fout, mode="native").double()
    ref.load_state_dict({k: v.double().cpu() for k, v in layer.state_dict().items()})
    w64 = w.detach().double().cpu().requires_grad_(True)
    # edges are already in destination order, so they are the CSR edges
    indices = torch.stack([torch.from_numpy(rows), torch.from_numpy(col)])
    out64 = ref.linear(torch.sparse_coo_tensor(indices, w64, (n, n)) @ x.double().cpu())
    out64.square().mean().backward()
    assert np.allclose(out.detach().cpu().numpy(), out64.detach().numpy(), rtol=1e-4, atol=1e-5)
    assert np.allclose(w.grad.cpu().numpy(), w64.grad.numpy(), rtol=1e-4, atol=1e-7)
    assert np.allclose(layer.linear.weight.grad.cpu().numpy(), ref.linear.weight.grad.numpy(), rtol=1e-4, atol=1e-6)
