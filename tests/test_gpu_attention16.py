"""GPU parity of the 16-bit attention kernel (``autosage::csr_attention_colslice``
on bf16 / fp16 query, key and value).

The kernel converts every input exactly to fp32, runs the online softmax of
the fp32 column-sliced attention and rounds each output once to the element
type.  Its fp32 value y is within ε = 1e-5·|exact| + 1e-6 of the exact
attention (the bar the fp32 kernel meets against the fp64 oracle), and
rounding is monotone, so every output must lie between the rounded ends of
[exact − ε, exact + ε]: round(exact − ε) <= got <= round(exact + ε), with the
same fp32-then-16-bit round-to-nearest-even as the kernel.  The exact
attention is ``oracle.attention_f64`` of the (exactly converted) 16-bit
inputs.  Almost every output equals round(exact) itself.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import autosage_amd
import oracle
from tests.gpu_common import case_graph, require_gpu

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]
RTOL = 1e-5
ATOL = 1e-6


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _inputs(fqk, fv, dtype, seed, rows=2500, degree=10, hubs=6, hub_degree=1500, empty=0.05):
    crow, col = case_graph(rows, degree, seed=seed, hubs=hubs, hub_degree=hub_degree, empty=empty)
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.standard_normal((rows, fqk)).astype(np.float32)).to(dtype)
    k = torch.from_numpy(rng.standard_normal((rows, fqk)).astype(np.float32)).to(dtype)
    v = torch.from_numpy(rng.standard_normal((rows, fv)).astype(np.float32)).to(dtype)
    return crow, col, q, k, v


def _round(values: np.ndarray, dtype) -> np.ndarray:
    """fp64 -> fp32 -> dtype, round to nearest even both times (the kernel's
    rounding of its fp32 result), back to fp64."""
    return torch.from_numpy(values).to(torch.float32).to(dtype).to(torch.float64).numpy()


def _check(got: torch.Tensor, crow, col, q, k, v, scale, dtype) -> float:
    exact = oracle.attention_f64(crow, col, q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                 scale=scale)
    eps = RTOL * np.abs(exact) + ATOL
    lo, hi = _round(exact - eps, dtype), _round(exact + eps, dtype)
    g = got.cpu().to(torch.float64).numpy()
    bad = (g < lo) | (g > hi)
    assert not bad.any(), (int(bad.sum()), g[bad][:4], exact[bad][:4])
    return float((g == _round(exact, dtype)).mean())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("fqk, fv", [(64, 128), (64, 64), (128, 128), (8, 8), (32, 512), (256, 64), (72, 136),
                                     (512, 16)])
def test_attention16_against_fp64(dtype, fqk, fv):
    crow, col, q, k, v = _inputs(fqk, fv, dtype, seed=fqk + fv)
    assert (np.diff(crow) >= 128).sum() >= 6 and (np.diff(crow) == 0).any()
    d_crow, d_col = torch.from_numpy(crow).cuda(), torch.from_numpy(col).cuda()
    got = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, q.cuda(), k.cuda(), v.cuda(), 0.125)
    assert got.dtype == dtype and got.shape == (crow.size - 1, fv)
    same = _check(got, crow, col, q, k, v, 0.125, dtype)
    assert same > 0.97, same
    # rows without edges are zero
    assert torch.count_nonzero(got[torch.from_numpy(np.diff(crow) == 0).cuda()]).item() == 0


@pytest.mark.parametrize("dtype", DTYPES)
def test_attention16_deterministic_chunked_and_any_column_order(dtype, monkeypatch):
    crow, col, q, k, v = _inputs(64, 128, dtype, seed=3, rows=6000, hubs=40, hub_degree=3000)
    d_crow, d_col = torch.from_numpy(crow).cuda(), torch.from_numpy(col).cuda()
    d = (q.cuda(), k.cuda(), v.cuda())
    first = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *d, 0.125)
    assert torch.equal(first, torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *d, 0.125))
    # partial states for ~3 sliced rows: the 40+ hub rows run in many chunks
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", str((6000 * 40 + 4096 + 3 * 8 * 130 * 4 + 768) / 2**20))
    assert torch.equal(first, torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *d, 0.125))
    monkeypatch.delenv("AUTOSAGE_COLSLICE_WORKSPACE_MB")
    # the same rows with their columns reversed: the row-sorted copy, same bits
    rev = np.concatenate([col[crow[r]:crow[r + 1]][::-1] for r in range(crow.size - 1)])
    got = torch.ops.autosage.csr_attention_colslice(d_crow, torch.from_numpy(rev).cuda(), *d, 0.125)
    assert torch.equal(got, first)
    _check(first, crow, col, q, k, v, 0.125, dtype)


def test_attention16_edge_cases_and_rejections():
    dtype = torch.bfloat16
    # a graph without edges: zeros
    crow = torch.zeros(11, dtype=torch.long, device="cuda")
    col = torch.zeros(0, dtype=torch.long, device="cuda")
    q = torch.ones(10, 16, dtype=dtype, device="cuda")
    out = torch.ops.autosage.csr_attention_colslice(crow, col, q, q, q, 1.0)
    assert torch.count_nonzero(out).item() == 0
    # widths that are not multiples of 8, or mixed element types
    crow2, col2, q2, k2, v2 = _inputs(64, 64, dtype, seed=1, rows=300, hubs=0)
    d_crow, d_col = torch.from_numpy(crow2).cuda(), torch.from_numpy(col2).cuda()
    with pytest.raises(ValueError, match=r"of 8 in \[8, 512\]"):
        torch.ops.autosage.csr_attention_colslice(d_crow, d_col, q2[:, :12].contiguous().cuda(),
                                                  k2[:, :12].contiguous().cuda(), v2.cuda(), 1.0)
    with pytest.raises(RuntimeError, match="dtype"):
        torch.ops.autosage.csr_attention_colslice(d_crow, d_col, q2.cuda(), k2.cuda(), v2.float().cuda(), 1.0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_attention_forward_runs_one_16_bit_kernel(dtype):
    """``csr_attention_forward`` on 16-bit inputs: with ``fused`` (the default)
    one kernel, the op's result; ``fused=False`` the three native stages, whose
    scores and probabilities are rounded to 16 bits (less accurate)."""
    crow, col, q, k, v = _inputs(64, 128, dtype, seed=11, rows=4000, hubs=20, hub_degree=2500)
    d_crow, d_col = torch.from_numpy(crow).cuda(), torch.from_numpy(col).cuda()
    d = (q.cuda(), k.cuda(), v.cuda())
    out, info = autosage_amd.csr_attention_forward(d_crow, d_col, *d, scale=0.125)
    assert info["fused"] and info["variant"] == "colslice16"
    assert torch.equal(out, torch.ops.autosage.csr_attention_colslice(d_crow, d_col, *d, 0.125))
    staged, info2 = autosage_amd.csr_attention_forward(d_crow, d_col, *d, scale=0.125, fused=False)
    assert set(info2) == {"sddmm", "spmm"}
    exact = oracle.attention_f64(crow, col, q.double().numpy(), k.double().numpy(), v.double().numpy(), scale=0.125)
    err_fused = np.abs(out.cpu().double().numpy() - exact).max()
    err_staged = np.abs(staged.cpu().double().numpy() - exact).max()
    assert err_fused <= err_staged
    # the backward: the two native gather passes, gradients in the input type
    qq, kk, vv = (t.clone().requires_grad_(True) for t in d)
    y = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, qq, kk, vv, 0.125)
    y.float().sum().backward()
    for t in (qq, kk, vv):
        assert t.grad is not None and t.grad.dtype == dtype and torch.isfinite(t.grad.float()).all()
