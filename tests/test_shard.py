"""Row shards on the CPU: the nnz-balanced cut points and the CPU shard
product (no GPU).

The cut points are pinned by the properties that define them, not by a
second copy of their formula: they cover [0, N] in order; each inner cut
r_k is the first row whose first edge index reaches t_k = ceil(k·nnz / P)
(crow[r_k] >= t_k, and crow[r_k - 1] < t_k unless r_k = 0), which a linear
scan finds independently; and every shard's edge count lies within the
largest degree of nnz / P.  The CPU shard product is the reference's CPU
path (torch.sparse.mm on a CSR tensor, autosage/ops.py:124-143) on the
shard's rows, bit-identical to the sequential oracle on those rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import shard, synth


def _linear_scan_cut(crow: np.ndarray, target: int) -> int:
    for r, start in enumerate(crow[:-1]):
        if start >= target:
            return r
    return crow.size - 1


def _graphs():
    yield "hubs", *synth.random_csr(2000, 7, seed=1, hub_rows=5, hub_degree=1500, empty_fraction=0.1)
    yield "uniform", *synth.random_csr(1000, 12, seed=2)
    yield "one hub", *synth.random_csr(50, 1, seed=3, hub_rows=1, hub_degree=49)
    empty_tail = np.concatenate([[0, 5, 9], np.full(6, 9)]).astype(np.int64)
    yield "empty rows at the end", empty_tail, np.arange(9, dtype=np.int64) % 8
    yield "no edges", np.zeros(11, dtype=np.int64), np.zeros(0, dtype=np.int64)
    yield "no rows", np.zeros(1, dtype=np.int64), np.zeros(0, dtype=np.int64)


@pytest.mark.parametrize("parts", [1, 2, 3, 8, 13, 64])
def test_cut_points_cover_balance_and_are_first_rows(parts):
    for name, crow, _ in _graphs():
        n = crow.size - 1
        nnz = int(crow[-1])
        cuts = shard.cut_rows(torch.from_numpy(crow), parts)
        assert len(cuts) == parts + 1, name
        assert cuts[0] == 0 and cuts[-1] == n, name
        assert all(a <= b for a, b in zip(cuts, cuts[1:])), name
        max_degree = int(np.diff(crow).max()) if n else 0
        for k in range(1, parts):
            target = -(-k * nnz // parts)
            assert cuts[k] == _linear_scan_cut(crow, target), (name, k)
        for k in range(parts):
            edges = int(crow[cuts[k + 1]] - crow[cuts[k]])
            assert abs(edges - nnz / parts) <= max_degree + 1, (name, k, edges)


def test_cut_points_accept_int32_and_reject_bad_arguments():
    crow, _ = synth.random_csr(300, 5, seed=4)
    assert shard.cut_rows(torch.from_numpy(crow).int(), 4) == shard.cut_rows(torch.from_numpy(crow), 4)
    with pytest.raises(ValueError):
        shard.cut_rows(torch.from_numpy(crow), 0)
    with pytest.raises(TypeError):
        shard.cut_rows(torch.from_numpy(crow).float(), 2)
    with pytest.raises(ValueError):
        shard.shard_csr(torch.from_numpy(crow), torch.zeros(0, dtype=torch.long), None, 5, 4)


@pytest.mark.parametrize("weighted", [False, True])
def test_cpu_shards_are_the_rows_of_the_whole_product(weighted):
    crow, col = synth.random_csr(1500, 9, seed=5, hub_rows=4, hub_degree=900, empty_fraction=0.05)
    rng = np.random.default_rng(6)
    val = rng.standard_normal(col.size).astype(np.float32) if weighted else None
    x = rng.standard_normal((crow.size - 1, 48)).astype(np.float32)
    t_crow, t_col = torch.from_numpy(crow), torch.from_numpy(col)
    t_val = None if val is None else torch.from_numpy(val)
    t_x = torch.from_numpy(x)
    want = oracle.spmm_seq(crow, col, val, x)
    cuts = shard.cut_rows(t_crow, 5)
    pieces = []
    for r0, r1 in zip(cuts, cuts[1:]):
        s_crow, s_col, s_val = shard.shard_csr(t_crow, t_col, t_val, r0, r1)
        assert int(s_crow[0]) == 0 and s_col.numel() == int(s_crow[-1])
        got = shard.spmm_csr_shard(s_crow, s_col, s_val, t_x)
        assert got.shape == (r1 - r0, 48)
        assert np.array_equal(got.numpy(), want[r0:r1])
        pieces.append(got)
    assert np.array_equal(torch.cat(pieces).numpy(), want)


def test_cpu_sddmm_and_attention_shards_are_the_whole_graph_rows():
    """The CPU shard SDDMM / attention (the reference's gather-dot and
    composition on the shard's rows) give the whole graph's outputs on the
    shard's edges and rows: bitwise against the same composition over all
    rows (one shard of everything), which is within the reference's bar
    (1e-5 relative, 1e-6 absolute) of the oracle's reference-order
    attention."""
    crow, col = synth.random_csr(1200, 8, seed=8, hub_rows=3, hub_degree=700, empty_fraction=0.05)
    rng = np.random.default_rng(9)
    q = rng.standard_normal((crow.size - 1, 16)).astype(np.float32)
    k = rng.standard_normal((crow.size - 1, 16)).astype(np.float32)
    v = rng.standard_normal((crow.size - 1, 24)).astype(np.float32)
    t_crow, t_col = torch.from_numpy(crow), torch.from_numpy(col)
    tq, tk, tv = (torch.from_numpy(a) for a in (q, k, v))
    whole_scores = oracle.torch_gather_dot(t_crow, t_col, tq, tk).numpy()
    whole_att = shard.csr_attention_shard(t_crow, t_col, tq, tk, tv, 0.125).numpy()
    ref_att = oracle.attention_ref(crow, col, q, k, v, 0.125)
    assert np.all(np.abs(whole_att - ref_att) <= 1e-5 * np.abs(ref_att) + 1e-6)
    cuts = shard.cut_rows(t_crow, 4)
    for r0, r1 in zip(cuts, cuts[1:]):
        s_crow, s_col, _ = shard.shard_csr(t_crow, t_col, None, r0, r1)
        got = shard.sddmm_csr_shard(s_crow, s_col, tq[r0:r1], tk).numpy()
        assert np.array_equal(got, whole_scores[crow[r0]:crow[r1]])
        att = shard.csr_attention_shard(s_crow, s_col, tq[r0:r1], tk, tv, 0.125).numpy()
        assert att.shape == (r1 - r0, 24)
        assert np.array_equal(att, whole_att[r0:r1])
    with pytest.raises(ValueError):
        shard.sddmm_csr_shard(t_crow, t_col, tq[:5], tk)
