"""GPU parity of row shards (one GPU's share of a graph split by rows).

A shard is the CSR of rows [r0, r1) of a graph, crow rebased to 0 and the
columns unchanged, multiplied with the whole X.  Its product must be rows
[r0, r1) of the whole graph's product:

* ``exact=True``: bit-identical to the sequential oracle (the reference's
  CPU product order) on those rows;
* the column-sliced schedule: within the fp64 bound of the oracle
  (|gpu - fp64| <= 1e-6·|fp64| + 1e-9), and bit-identical to the whole
  graph's column-sliced product, because the column slices cut the whole
  column space [0, N) and each row is summed the same way in both;
* bf16 / fp16: the bits of the rounded fp64 oracle.
The shards are cut at nnz-balanced row prefixes (``shard.cut_rows``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import _native, shard
from tests.gpu_common import case_graph, require_gpu, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _inputs(features, weighted, seed, rows=4000, degree=9, hubs=4, hub_degree=3000, empty=0.08):
    crow, col = case_graph(rows, degree, seed=seed, hubs=hubs, hub_degree=hub_degree, empty=empty)
    rng = np.random.default_rng(seed + 7)
    val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
    x = rng.standard_normal((rows, features)).astype(np.float32)
    return crow, col, val, x


def _assert_fp64_close(got: np.ndarray, exact: np.ndarray) -> None:
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= 1e-6 * np.abs(exact) + 1e-9), float(np.max(err - 1e-6 * np.abs(exact)))


@pytest.mark.parametrize("parts", [1, 3, 8])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("features", [33, 64, 128, 256])
def test_shards_are_rows_of_the_whole_product(features, weighted, parts):
    crow, col, val, x = _inputs(features, weighted, seed=features + 10 * parts + weighted)
    d_crow, d_col, d_val, d_x = to_dev(crow, col, val, x)
    whole = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x)
    exact64 = oracle.spmm_f64(crow, col, val, x)
    seq = oracle.spmm_seq(crow, col, val, x)
    cuts = shard.cut_rows(d_crow, parts)
    sliced, exact = [], []
    for r0, r1 in zip(cuts, cuts[1:]):
        s_crow, s_col, s_val = shard.shard_csr(d_crow, d_col, d_val, r0, r1)
        got = shard.spmm_csr_shard(s_crow, s_col, s_val, d_x)
        assert got.shape == (r1 - r0, features)
        _assert_fp64_close(got.cpu().numpy(), exact64[r0:r1])
        sliced.append(got)
        exact.append(shard.spmm_csr_shard(s_crow, s_col, s_val, d_x, exact=True))
    assert torch.equal(torch.cat(sliced), whole)
    got_exact = torch.cat(exact).cpu().numpy()
    assert np.array_equal(got_exact.view(np.uint32), seq.view(np.uint32))


def test_shard_with_columns_out_of_order_runs_row_sorted():
    """A shard whose columns do not ascend within rows, with columns up to
    N - 1 beyond its own row count: the row-sorted copy keys (row, column)
    over the whole column space, and the product is unchanged."""
    crow, col, val, x = _inputs(128, True, seed=91)
    rng = np.random.default_rng(92)
    shuffled_col, shuffled_val = col.copy(), val.copy()
    for r in range(crow.size - 1):
        perm = rng.permutation(crow[r + 1] - crow[r]) + crow[r]
        shuffled_col[crow[r]:crow[r + 1]] = col[perm]
        shuffled_val[crow[r]:crow[r + 1]] = val[perm]
    d_crow, d_col, d_val, d_x = to_dev(crow, shuffled_col, shuffled_val, x)
    exact64 = oracle.spmm_f64(crow, col, val, x)
    cuts = shard.cut_rows(d_crow, 4)
    for r0, r1 in zip(cuts, cuts[1:]):
        s_crow, s_col, s_val = shard.shard_csr(d_crow, d_col, d_val, r0, r1)
        assert not _native.columns_ascending(s_crow, s_col, d_x.size(0)) or r1 == r0
        got = shard.spmm_csr_shard(s_crow, s_col, s_val, d_x)
        _assert_fp64_close(got.cpu().numpy(), exact64[r0:r1])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_16_bit_shards_have_the_oracle_bits(dtype):
    crow, col, val, x = _inputs(128, True, seed=93, rows=6000, hubs=3, hub_degree=5000)
    x16 = torch.from_numpy(x).to(dtype)
    v16 = torch.from_numpy(val).to(dtype)
    want = oracle.spmm_rounded_16(crow, col, v16, x16, dtype)
    d_crow, d_col = to_dev(crow, col)
    d_val, d_x = v16.cuda(), x16.cuda()
    cuts = shard.cut_rows(d_crow, 8)
    for r0, r1 in zip(cuts, cuts[1:]):
        s_crow, s_col, s_val = shard.shard_csr(d_crow, d_col, d_val, r0, r1)
        got = shard.spmm_csr_shard(s_crow, s_col, s_val, d_x).cpu()
        assert torch.equal(got.view(torch.int16), want[r0:r1].view(torch.int16)), (r0, r1)


def test_shard_rejects_columns_beyond_x_when_validating(monkeypatch):
    crow, col, val, x = _inputs(64, False, seed=94, rows=500, hubs=0)
    d_crow, d_col, _, d_x = to_dev(crow, col, None, x)
    s_crow, s_col, _ = shard.shard_csr(d_crow, d_col, None, 0, 100)
    monkeypatch.setenv("AUTOSAGE_VALIDATE", "1")
    # the whole X has 500 rows; a 200-row X leaves columns out of range
    with pytest.raises(ValueError, match="invalid CSR graph"):
        shard.spmm_csr_shard(s_crow, s_col, None, d_x[:200])
    assert shard.spmm_csr_shard(s_crow, s_col, None, d_x).shape == (100, 64)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_sddmm_and_attention_shards_are_the_whole_graph_outputs(dtype):
    """The shard SDDMM (the shard's rows of Q against the whole K) gives the
    whole graph's SDDMM on the shard's edges bit for bit (the same per-edge
    arithmetic), and the shard attention (column slices over the whole column
    space) the whole graph's column-sliced attention rows bit for bit."""
    rows = 5000
    crow, col = case_graph(rows, 9, seed=95, hubs=4, hub_degree=3000, empty=0.05)
    rng = np.random.default_rng(96)
    q = torch.from_numpy(rng.standard_normal((rows, 64)).astype(np.float32)).to(dtype).cuda()
    k = torch.from_numpy(rng.standard_normal((rows, 64)).astype(np.float32)).to(dtype).cuda()
    v = torch.from_numpy(rng.standard_normal((rows, 128)).astype(np.float32)).to(dtype).cuda()
    d_crow, d_col = to_dev(crow, col)
    whole_scores = torch.ops.autosage.sddmm_csr(d_crow, d_col, q, k)
    whole_att = torch.ops.autosage.csr_attention_colslice(d_crow, d_col, q, k, v, 0.125)
    cuts = shard.cut_rows(d_crow, 5)
    scores, att = [], []
    for r0, r1 in zip(cuts, cuts[1:]):
        s_crow, s_col, _ = shard.shard_csr(d_crow, d_col, None, r0, r1)
        scores.append(shard.sddmm_csr_shard(s_crow, s_col, q[r0:r1], k))
        att.append(shard.csr_attention_shard(s_crow, s_col, q[r0:r1], k, v, 0.125))
    assert torch.equal(torch.cat(scores), whole_scores)
    assert torch.equal(torch.cat(att), whole_att)
    if dtype == torch.float32:
        want = oracle.sddmm_ref(crow, col, q.cpu().numpy(), k.cpu().numpy())
        assert np.array_equal(torch.cat(scores).cpu().numpy().view(np.uint32), want.view(np.uint32))
