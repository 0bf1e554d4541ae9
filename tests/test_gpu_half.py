"""GPU parity of the bf16 / fp16 SpMM (``autosage::spmm_csr`` and
``spmm_csr_colslice`` on 16-bit features) and SDDMM (``sddmm_csr``,
``sddmm_csr_split``), their gradients and their scheduler paths.

The reference has no kernel for these types (its op raises, its scheduler
runs torch.sparse.mm).  The rule here: every output is the fp64 sum of the
exact products rounded to fp32 and then to the 16-bit type.  An exact fp64
sum does not depend on the order of the additions; an inexact one differs
between orders by less than 2^-52 of its largest partial, which changes the
rounded result only for a sum that close to a tie (random inputs do not
produce one).  So the bar is bit-identity with the oracle
(``oracle.spmm_rounded_16``, an fp64 sum in CSR order) for every schedule:
column slices (ascending columns), edge slices (shuffled columns), grouped
and one-wave short rows, hub rows, empty rows, any F; for the SDDMM, rows
split by degree and blocks of 64 edges whatever the rows.
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
    # ascending columns: column slices (the colslice op takes them
    # explicitly), rows whole (spmm_csr on this small graph)
    got = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x)
    assert got.dtype == dtype
    assert _same_bits(got, want), (got.float().cpu() - want.float()).abs().max()
    assert _same_bits(torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x), want)
    assert _same_bits(_native.spmm_rounded_16_impl(d_crow, d_col, d_val, d_x, column_slices=True), want)
    assert _same_bits(_native.spmm_rows_16_impl(d_crow, d_col, d_val, d_x), want)
    # the same rows with shuffled columns: edge slices, same bits (the
    # weights move with their columns)
    idx = _shuffle_within_rows(crow, seed=features)
    s_col = col[idx]
    s_val = None if val is None else val[torch.from_numpy(idx)]
    d_scol, = to_dev(s_col)
    assert not _native.columns_ascending(d_crow, d_scol) or crow[-1] == 0
    d_sval = None if s_val is None else s_val.cuda()
    got_s = torch.ops.autosage.spmm_csr(d_crow, d_scol, d_sval, d_x)
    assert _same_bits(got_s, want)
    # the colslice op runs column slices on the row-sorted copy: same bits
    assert _same_bits(torch.ops.autosage.spmm_csr_colslice(d_crow, d_scol, d_sval, d_x), want)
    assert _same_bits(_native.spmm_rounded_16_impl(d_crow, d_scol, d_sval, d_x, column_slices=False), want)
    assert _same_bits(_native.spmm_rows_16_impl(d_crow, d_scol, d_sval, d_x), want)


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
    # hubs of 20,000 edges (column slices of ~2,500 edges each), every schedule
    crow, col, val, x = _inputs(128, False, dtype, seed=6, rows=6000, degree=5, hubs=2, hub_degree=20000)
    d_crow, d_col = to_dev(crow, col)
    want = oracle.spmm_rounded_16(crow, col, None, x, dtype)
    assert _same_bits(torch.ops.autosage.spmm_csr(d_crow, d_col, None, x.cuda()), want)
    for columns in (True, False):
        assert _same_bits(_native.spmm_rounded_16_impl(d_crow, d_col, None, x.cuda(), column_slices=columns), want)
    assert _same_bits(_native.spmm_rows_16_impl(d_crow, d_col, None, x.cuda()), want)


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
    from autosage_amd._auto import ROUNDED16, ROUNDED16_EDGES, ROUNDED16_ROWS, spmm_csr_auto

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
    # all three schedules are timed (the columns ascend); each gives the same bits
    assert info["choice"] == "autosage" and info["candidate"] in (ROUNDED16, ROUNDED16_EDGES, ROUNDED16_ROWS)
    assert {c["candidate"] for c in info["candidates"]} == {ROUNDED16, ROUNDED16_EDGES, ROUNDED16_ROWS}
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
    # the weight gradient: the 16-bit SDDMM <dY[row], X[col]>
    d_val = torch.ones(col.size, dtype=dtype, device="cuda", requires_grad=True)
    y = torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, x.cuda())
    y.backward(g.cuda())
    assert _same_bits(d_val.grad, oracle.sddmm_rounded_16(crow, col, g, x, dtype))


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


# ---- SDDMM ------------------------------------------------------------------


def _sddmm_inputs(features, dtype, seed=0, rows=3000, degree=9, hubs=3, hub_degree=2500, empty=0.08):
    crow, col = case_graph(rows, degree, seed=seed, hubs=hubs, hub_degree=hub_degree, empty=empty)
    rng = np.random.default_rng(seed + 17)
    q = torch.from_numpy(rng.standard_normal((rows, features)).astype(np.float32)).to(dtype)
    k = torch.from_numpy(rng.standard_normal((rows, features)).astype(np.float32)).to(dtype)
    return crow, col, q, k


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("features", [1, 7, 8, 16, 24, 33, 64, 72, 128, 136, 256, 264, 512, 520])
def test_rounded_sddmm_equals_oracle_on_every_split(dtype, features):
    """16-byte lanes for F a multiple of 8 up to 512 (1 to 32 lanes per edge,
    two chunks per lane above 256), element lanes otherwise; hub rows of 2,500
    edges cut into 2048-edge chunks, or into many at threshold 64."""
    crow, col, q, k = _sddmm_inputs(features, dtype, seed=features)
    want = oracle.sddmm_rounded_16(crow, col, q, k, dtype)
    d_crow, d_col = to_dev(crow, col)
    d_q, d_k = q.cuda(), k.cuda()
    got = torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, d_k)
    assert got.dtype == dtype
    assert _same_bits(got, want), (got.float().cpu() - want.float()).abs().max()
    for waves, threshold in ((2, 64), (8, 2**31 - 1), (4, 1024)):
        assert _same_bits(torch.ops.autosage.sddmm_csr_split(d_crow, d_col, d_q, d_k, waves, threshold), want)


def _edge_block_graphs(rows_seed: int):
    """Row layouts for the edge-block schedule: hub rows and 8 % empty rows;
    90 % empty rows (blocks of 64 edges spanning far more than 64 rows); one
    edge per row (exactly 64 rows a block); runs of hundreds of empty rows
    between short rows and a hub as the last row; fewer edges than a block."""
    rng = np.random.default_rng(rows_seed)
    yield "hubs", case_graph(3000, 9, seed=rows_seed, hubs=3, hub_degree=2500, empty=0.08)
    yield "mostly empty", case_graph(5000, 3, seed=rows_seed + 1, empty=0.9)
    n = 700
    yield "one edge a row", (np.arange(n + 1, dtype=np.int64), np.sort(rng.integers(0, n, n)).astype(np.int64))
    deg = np.zeros(900, dtype=np.int64)
    deg[[0, 130, 131, 400, 650]] = [3, 1, 70, 2, 5]
    deg[-1] = 4000
    crow = np.concatenate(([0], np.cumsum(deg))).astype(np.int64)
    col = np.concatenate([np.sort(rng.integers(0, deg.size, d)) for d in deg]).astype(np.int64)
    yield "empty runs, hub last", (crow, col)
    yield "one block", (np.array([0, 5, 5, 20], dtype=np.int64), np.sort(rng.integers(0, 3, 20)).astype(np.int64))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("features", [1, 7, 8, 16, 24, 64, 128, 136, 264, 512, 520])
def test_rounded_sddmm_edge_blocks(dtype, features):
    """``sddmm_edges_16_impl``: blocks of 64 edges whatever the rows, each
    edge's row found from crow in the wavefront; bitwise the oracle's (and
    so the split schedules') result on every layout."""
    for name, (crow, col) in _edge_block_graphs(features):
        n = crow.size - 1
        rng = np.random.default_rng(features + 3)
        q = torch.from_numpy(rng.standard_normal((n, features)).astype(np.float32)).to(dtype)
        k = torch.from_numpy(rng.standard_normal((n, features)).astype(np.float32)).to(dtype)
        want = oracle.sddmm_rounded_16(crow, col, q, k, dtype)
        d_crow, d_col = to_dev(crow, col)
        got = _native.sddmm_edges_16_impl(d_crow, d_col, q.cuda(), k.cuda())
        assert got.dtype == dtype
        assert _same_bits(got, want), (name, (got.float().cpu() - want.float()).abs().max())


@pytest.mark.parametrize("dtype", DTYPES)
def test_rounded_sddmm_edge_cases(dtype):
    # rows that are not 16-byte aligned take the element lanes
    crow, col, q, k = _sddmm_inputs(64, dtype, seed=31, rows=800, hub_degree=700)
    want = oracle.sddmm_rounded_16(crow, col, q, k, dtype)
    d_crow, d_col = to_dev(crow, col)
    flat = torch.empty(q.numel() + 1, dtype=dtype, device="cuda")
    flat[1:] = q.reshape(-1).cuda()
    d_q = flat[1:].view(q.shape)
    assert d_q.data_ptr() % 16 != 0 and d_q.is_contiguous()
    assert _same_bits(torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, k.cuda()), want)
    # no edges; F = 0
    crow0 = np.zeros(6, dtype=np.int64)
    d_crow0, d_col0 = to_dev(crow0, np.zeros(0, dtype=np.int64))
    q0 = torch.ones(5, 16, dtype=dtype, device="cuda")
    assert torch.ops.autosage.sddmm_csr(d_crow0, d_col0, q0, q0).numel() == 0
    out = torch.ops.autosage.sddmm_csr(d_crow, d_col, q[:, :0].contiguous().cuda(), k[:, :0].contiguous().cuda())
    assert out.shape == (col.size,) and torch.count_nonzero(out).item() == 0
    # mixed types are rejected
    with pytest.raises(RuntimeError, match="query and key must use the same dtype"):
        torch.ops.autosage.sddmm_csr(d_crow, d_col, q.cuda(), k.cuda().to(torch.float16 if dtype == torch.bfloat16
                                                                            else torch.bfloat16))


@pytest.mark.parametrize("dtype", DTYPES)
def test_rounded_sddmm_gradients(dtype):
    from autosage_amd._autograd import csr_transpose

    crow, col, q, k = _sddmm_inputs(64, dtype, seed=41, rows=1500, hub_degree=1200)
    d_crow, d_col = to_dev(crow, col)
    d_q = q.cuda().requires_grad_(True)
    d_k = k.cuda().requires_grad_(True)
    s = torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, d_k)
    gs = torch.randn(col.size, generator=torch.Generator().manual_seed(5)).to(dtype)
    s.backward(gs.cuda())
    assert _same_bits(d_q.grad, oracle.spmm_rounded_16(crow, col, gs, k, dtype))
    t_crow, t_col, perm = csr_transpose(torch.from_numpy(crow), torch.from_numpy(col))
    assert _same_bits(d_k.grad, oracle.spmm_rounded_16(t_crow.numpy(), t_col.numpy(), gs[perm], q, dtype))


@pytest.mark.parametrize("dtype", DTYPES)
def test_sddmm_scheduler_on_16_bit_inputs(dtype, monkeypatch, tmp_path):
    from autosage_amd._auto import sddmm_csr_auto

    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    crow, col, q, k = _sddmm_inputs(128, dtype, seed=51, rows=4000)
    want = oracle.sddmm_rounded_16(crow, col, q, k, dtype)
    d_crow, d_col = to_dev(crow, col)
    out, info = sddmm_csr_auto(d_crow, d_col, q.cuda(), k.cuda())
    assert info["operation"] == "sddmm" and info["choice"] == "autosage" and info["from_cache"] is False
    assert info["candidate"] in (None, [4, 1024], [8, 4096]) and len(info["candidates"]) == 3
    assert info["baseline_probe_ms"] is None and _same_bits(out, want)
    out2, info2 = sddmm_csr_auto(d_crow, d_col, q.cuda(), k.cuda())
    assert info2["from_cache"] is True and info2["candidate"] == info["candidate"]
    assert torch.equal(out2, out)


@pytest.mark.parametrize("dtype", DTYPES)
def test_row_softmax_on_16_bit_scores(dtype):
    """fp32 softmax of the exactly converted scores, rounded once: within one
    16-bit unit of the oracle's fp32 softmax rounded the same way (the two
    exp implementations differ by an fp32 ulp or so, which moves a rounding
    only near a tie), and nearly always equal."""
    crow, col, _, _ = _sddmm_inputs(8, dtype, seed=71, rows=3000, hub_degree=2500)
    scores = torch.randn(col.size, generator=torch.Generator().manual_seed(7)).mul(4).to(dtype)
    want = oracle.row_softmax_rounded_16(crow, scores, dtype)
    d_crow, = to_dev(crow)
    got = torch.ops.autosage.csr_row_softmax(d_crow, scores.cuda())
    assert got.dtype == dtype
    diff = (got.cpu().view(torch.int16).int() - want.view(torch.int16).int()).abs()
    assert diff.max().item() <= 1
    assert (diff == 0).float().mean().item() > 0.99


def test_attention_on_bf16_inputs_runs_the_native_stages(monkeypatch, tmp_path):
    """bf16 attention: native SDDMM, native row softmax (fp32 inside, rounded
    once), native SpMM; close to the fp32 result at bf16 precision, hub rows
    included."""
    from autosage_amd._auto import csr_attention_forward

    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    crow, col, q, k = _sddmm_inputs(64, torch.float32, seed=61, rows=2000, hub_degree=1500)
    v = torch.randn(2000, 32, generator=torch.Generator().manual_seed(6))
    d_crow, d_col = to_dev(crow, col)
    q, k = q * 0.125, k * 0.125
    ref, _ = csr_attention_forward(d_crow, d_col, q.cuda(), k.cuda(), v.cuda(), fused=False)
    out, info = csr_attention_forward(d_crow, d_col, q.bfloat16().cuda(), k.bfloat16().cuda(),
                                      v.bfloat16().cuda(), fused=False)
    assert out.dtype == torch.bfloat16
    assert info["sddmm"]["choice"] == "autosage" and info["spmm"]["choice"] == "autosage"
    assert (out.float() - ref).abs().max().item() < 0.03
    # the default (fused): one kernel in fp32 arithmetic, each output rounded
    # once, so within one bf16 rounding of the fp32 result
    fused, finfo = csr_attention_forward(d_crow, d_col, q.bfloat16().cuda(), k.bfloat16().cuda(),
                                         v.bfloat16().cuda())
    assert finfo["fused"] and fused.dtype == torch.bfloat16
    ref16 = csr_attention_forward(d_crow, d_col, q.bfloat16().float().cuda(), k.bfloat16().float().cuda(),
                                  v.bfloat16().float().cuda(), fused=False)[0]
    assert (fused.float() - ref16).abs().max().item() <= 2.0 ** -8 * ref16.abs().max().item() + 1e-5


@pytest.mark.parametrize("dtype", DTYPES)
def test_torch_baseline_raises_for_16_bit_cuda_features(monkeypatch, dtype):
    """``_prepare_spmm_baseline`` and the baseline branch of
    ``_run_spmm_choice`` raise RuntimeError on 16-bit CUDA features instead
    of calling torch.sparse.mm, which aborts the process for bf16 CSR on
    PyTorch-ROCm.  The sparse entry points are replaced by functions that
    fail the test, so the real call is never reached even if the guard were
    missing."""
    from autosage_amd import _auto

    def never(*args, **kwargs):
        raise AssertionError("torch.sparse must not be reached for 16-bit CUDA features")

    monkeypatch.setattr(torch.sparse, "mm", never)
    monkeypatch.setattr(torch, "sparse_csr_tensor", never)
    crow, col, val, x = _inputs(16, True, dtype, seed=3, rows=200, hubs=0)
    d_crow, d_col = to_dev(crow, col)
    d_val, d_x = val.cuda(), x.cuda()
    with pytest.raises(RuntimeError, match="torch.sparse.mm"):
        _auto._prepare_spmm_baseline(d_crow, d_col, d_val, d_x)
    with pytest.raises(RuntimeError, match="torch.sparse.mm"):
        _auto._run_spmm_choice("baseline", None, d_crow, d_col, None, d_x)
    # the drop-in import path reaches the same guard
    from autosage._auto import _prepare_spmm_baseline

    with pytest.raises(RuntimeError, match="native 16-bit SpMM"):
        _prepare_spmm_baseline(d_crow, d_col, None, d_x)
