"""GPU parity of the bf16 / fp16 SpMM (``autosage::spmm_csr`` and
``spmm_csr_colslice`` on 16-bit features).

The reference has no kernel for these types (its op raises, its scheduler
runs torch.sparse.mm).  The rule here: every output is the fp64 sum of the
exact products rounded to fp32 and then to the 16-bit type.  An exact fp64
sum does not depend on the order of the additions; an inexact one differs
between orders by less than 2^-52 of its largest partial, which changes the
rounded result only for a sum that close to a tie (random inputs do not
produce one).  So the bar is bit-identity with the oracle
(``oracle.spmm_rounded_16``, an fp64 sum in CSR order) for every schedule:
column slices (ascending columns), edge slices (shuffled columns), grouped
and one-wave short rows, hub rows, empty rows, any F.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import _native
from tests.gpu_common import case_graph, require_gpu, to_dev

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _inputs(features, weighted, dtype, seed=0, rows=3000, degree=9, hubs=3, hub_degree=2500, empty=0.08):
    crow, col = case_graph(rows, degree, seed=seed, hubs=hubs, hub_degree=hub_degree, empty=empty)
    rng = np.random.default_rng(seed + 7)
    x = torch.from_numpy(rng.standard_normal((rows, features)).astype(np.float32)).to(dtype)
    val = torch.from_numpy(rng.standard_normal(col.size).astype(np.float32)).to(dtype) if weighted else None
    return crow, col, val, x


def _shuffle_within_rows(crow, seed) -> np.ndarray:
    """A permutation of the edges that keeps every edge in its row and
    shuffles the order inside each row."""
    rng = np.random.default_rng(seed)
    idx = np.arange(crow[-1])
    for r in range(crow.size - 1):
        s, e = crow[r], crow[r + 1]
        if e - s > 1:
            idx[s:e] = s + rng.permutation(e - s)
    return idx


def _same_bits(got: torch.Tensor, want: torch.Tensor) -> bool:
    a = got.detach().cpu().view(torch.int16)
    b = want.view(torch.int16)
    return a.shape == b.shape and torch.equal(a, b)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [8, 16, 64, 72, 128, 136, 256, 264, 512, 7, 33])
def test_rounded_spmm_equals_oracle_on_every_schedule(dtype, weighted, features):
    crow, col, val, x = _inputs(features, weighted, dtype, seed=features)
    want = oracle.spmm_rounded_16(crow, col, val, x, dtype)
    d_crow, d_col = to_dev(crow, col)
    d_x = x.cuda()
    d_val = None if val is None else val.cuda()
    # ascending columns: column slices (spmm_csr picks them; the colslice op
    # takes them explicitly)
    got = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x)
    assert got.dtype == dtype
    assert _same_bits(got, want), (got.float().cpu() - want.float()).abs().max()
    assert _same_bits(torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x), want)
    # the same rows with shuffled columns: edge slices, same bits (the
    # weights move with their columns)
    idx = _shuffle_within_rows(crow, seed=features)
    s_col = col[idx]
    s_val = None if val is None else val[torch.from_numpy(idx)]
    d_scol, = to_dev(s_col)
    assert not _native.columns_ascending(d_crow, d_scol) or crow[-1] == 0
    got_s = torch.ops.autosage.spmm_csr(d_crow, d_scol, None if s_val is None else s_val.cuda(), d_x)
    assert _same_bits(got_s, want)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rounded_spmm_edge_cases(dtype):
    # no edges, empty rows only, one row, F = 1
    crow = np.zeros(6, dtype=np.int64)
    col = np.zeros(0, dtype=np.int64)
    x = torch.ones(5, 16, dtype=dtype)
    d_crow, d_col = to_dev(crow, col)
    got = torch.ops.autosage.spmm_csr(d_crow, d_col, None, x.cuda())
    assert torch.count_nonzero(got).item() == 0
    crow, col, val, x = _inputs(1, True, dtype, seed=5, rows=500, hub_degree=400)
    d_crow, d_col = to_dev(crow, col)
    got = torch.ops.autosage.spmm_csr(d_crow, d_col, val.cuda(), x.cuda())
    assert _same_bits(got, oracle.spmm_rounded_16(crow, col, val, x, dtype))
    # hubs of 20,000 edges (column slices of ~2,500 edges each)
    crow, col, val, x = _inputs(128, False, dtype, seed=6, rows=6000, degree=5, hubs=2, hub_degree=20000)
    d_crow, d_col = to_dev(crow, col)
    want = oracle.spmm_rounded_16(crow, col, None, x, dtype)
    assert _same_bits(torch.ops.autosage.spmm_csr(d_crow, d_col, None, x.cuda()), want)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rounded_spmm_is_deterministic_and_chunk_independent(dtype, monkeypatch):
    crow, col, val, x = _inputs(128, True, dtype, seed=9, rows=20000, degree=40, hubs=8, hub_degree=6000)
    d_crow, d_col = to_dev(crow, col)
    d_val, d_x = val.cuda(), x.cuda()
    first = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x)
    assert torch.equal(first, torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x))
    monkeypatch.setenv("AUTOSAGE_COLSLICE_WORKSPACE_MB", "8")
    assert torch.equal(first, torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x))


def test_rounded_spmm_rejects_mixed_types():
    crow, col, _, x = _inputs(16, False, torch.bfloat16, rows=100, hubs=0, degree=4)
    d_crow, d_col = to_dev(crow, col)
    val32 = torch.ones(col.size, device="cuda")
    with pytest.raises(RuntimeError, match="val must be contiguous and of x's dtype"):
        torch.ops.autosage.spmm_csr(d_crow, d_col, val32, x.cuda())
    with pytest.raises(RuntimeError, match="x must be float32"):
        torch.ops.autosage.spmm_csr_split(d_crow, d_col, None, x.cuda(), 128, 2, 16)


@pytest.mark.parametrize("dtype", DTYPES)
def test_ops_api_and_scheduler_on_16_bit_features(dtype, monkeypatch, tmp_path):
    from autosage_amd import ops
    from autosage_amd._auto import ROUNDED16, ROUNDED16_EDGES, spmm_csr_auto

    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    crow, col, val, x = _inputs(64, True, dtype, seed=12, rows=4000)
    want = oracle.spmm_rounded_16(crow, col, val, x, dtype)
    d_crow, d_col = to_dev(crow, col)
    # the Python front end casts fp32 weights to x's dtype, as the reference does
    got = ops.spmm_csr(d_crow, d_col, val.float().cuda(), x.cuda())
    assert _same_bits(got, want)
    # the scheduler runs the native SpMM (the PyTorch baseline is not run for
    # 16-bit types: it aborts the process on PyTorch-ROCm) and caches it
    out, info = spmm_csr_auto(d_crow, d_col, val.float().cuda(), x.cuda())
    assert info["operation"] == "spmm" and info["from_cache"] is False
    # both slicings are timed (the columns ascend); either gives the same bits
    assert info["choice"] == "autosage" and info["candidate"] in (ROUNDED16, ROUNDED16_EDGES)
    assert {c["candidate"] for c in info["candidates"]} == {ROUNDED16, ROUNDED16_EDGES}
    assert _same_bits(out, want)
    assert info["autosage_probe_ms"] > 0 and info["baseline_probe_ms"] is None
    out2, info2 = spmm_csr_auto(d_crow, d_col, val.float().cuda(), x.cuda())
    assert info2["from_cache"] is True and info2["candidate"] == info["candidate"]
    assert torch.equal(out2, out)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rounded_spmm_backward_for_x(dtype):
    from autosage_amd._autograd import csr_transpose

    crow, col, _, x = _inputs(64, False, dtype, seed=13, rows=1500, hub_degree=1200)
    d_crow, d_col = to_dev(crow, col)
    d_x = x.cuda().requires_grad_(True)
    y = torch.ops.autosage.spmm_csr(d_crow, d_col, None, d_x)
    g = torch.randn(y.shape, generator=torch.Generator().manual_seed(3)).to(dtype)
    y.backward(g.cuda())
    t_crow, t_col, _ = csr_transpose(torch.from_numpy(crow), torch.from_numpy(col))
    assert _same_bits(d_x.grad, oracle.spmm_rounded_16(t_crow.numpy(), t_col.numpy(), None, g, dtype))
    # weight gradients of 16-bit SpMM are not implemented
    d_val = torch.ones(col.size, dtype=dtype, device="cuda", requires_grad=True)
    y = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, x.cuda())
    with pytest.raises(NotImplementedError, match="weight gradient"):
        y.backward(g.cuda())


def test_fp16_rounding_at_the_ends_of_the_range():
    """Rows whose sums land on fp16's overflow threshold and on ties among
    subnormals, each checked against the oracle (torch's conversions)."""
    u = 2.0**-24  # smallest fp16 subnormal
    rows = [
        [(65504.0, 1.0), (8.0, 1.0)],  # 65512 -> 65504
        [(65504.0, 1.0), (16.0, 1.0)],  # 65520: tie -> even -> inf
        [(-65504.0, 1.0), (-32.0, 1.0)],  # -65536 -> -inf
        [(u, 0.5)],  # half a unit: tie -> 0
        [(u, 0.75)],  # 0.75 units -> 1 unit
        [(u, 1.5)],  # 1.5 units: tie -> 2 units
        [(u, 2.5)],  # 2.5 units: tie -> 2 units
        [(2.0**-14, 1.0)],  # the smallest normal
        [(2.0**-14, 1.0), (-u, 1.0)],  # the largest subnormal
        [(1.0, 1.0), (2.0**-11, 1.0)],  # 1 + half an ulp: tie -> 1
    ]
    n = len(rows)
    xs = [v for r in rows for v, _ in r]
    # edge e gathers X row e (all features equal); the graph is square, so
    # rows past the n above are empty
    x = torch.tensor(xs, dtype=torch.float16)[:, None].repeat(1, 8)
    crow = np.cumsum([0] + [len(r) for r in rows]).astype(np.int64)
    crow_full = np.concatenate([crow, np.full(len(xs) - n, crow[-1])]).astype(np.int64)
    col = np.arange(len(xs), dtype=np.int64)
    val = torch.tensor([w for r in rows for _, w in r], dtype=torch.float16)
    want = oracle.spmm_rounded_16(crow_full, col, val, x, torch.float16)
    d_crow, d_col = to_dev(crow_full, col)
    got = torch.ops.autosage.spmm_csr(d_crow, d_col, val.cuda(), x.cuda())
    assert _same_bits(got, want), (got.float().cpu()[:n, 0], want.float()[:n, 0])
    expected = [65504.0, float("inf"), float("-inf"), 0.0, u, 2 * u, 2 * u, 2.0**-14, 2.0**-14 - u, 1.0]
    assert want.float()[:n, 0].tolist() == expected
