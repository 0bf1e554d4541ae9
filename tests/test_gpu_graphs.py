"""The native operators under HIP graph capture (torch.cuda.CUDAGraph).

The kernels take their workspaces from the caller, record no memset and no
host synchronisation, so a captured call replays the same launches.  The
per-graph checks (ascending columns) are memoised by an eager call before
capture.  Every replay is checked against eager results, with eager work and
synchronisations between replays, and after the inputs change in place."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gpu_common import case_graph, require_gpu, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def test_native_ops_replay_in_a_hip_graph():
    crow, col = case_graph(6000, 20, seed=4, hubs=12, hub_degree=4000, empty=0.05)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((6000, 128)).astype(np.float32)
    q = rng.standard_normal((6000, 64)).astype(np.float32)
    k = rng.standard_normal((6000, 64)).astype(np.float32)
    w = rng.standard_normal(col.size).astype(np.float32)
    d_crow, d_col, d_x, d_q, d_k, d_w = to_dev(crow, col, x, q, k, w)
    ops = torch.ops.autosage
    calls = [
        lambda: ops.spmm_csr(d_crow, d_col, None, d_x),
        lambda: ops.spmm_csr_split(d_crow, d_col, None, d_x, 128, 2, 1024),
        # the feature-sliced SpMM: relayout of X and product on the graph's
        # plan (built by the eager call), weighted and not
        lambda: ops.spmm_csr_fslice(d_crow, d_col, None, d_x),
        lambda: ops.spmm_csr_fslice(d_crow, d_col, d_w, d_x),
        lambda: ops.spmm_csr_colslice(d_crow, d_col, None, d_x),
        lambda: ops.sddmm_csr_split(d_crow, d_col, d_q, d_k, 4, 1024),
        lambda: ops.csr_attention(d_crow, d_col, d_q, d_k, d_x, 0.125),
        lambda: ops.csr_attention_colslice(d_crow, d_col, d_q, d_k, d_x, 0.125),
    ]
    _replay_matches_eager(calls, lambda: (d_x.mul_(2.0), d_q.mul_(0.5), d_w.mul_(-1.5)))


def test_16_bit_ops_replay_in_a_hip_graph():
    """bf16: the SDDMM in blocks of 64 edges, the rounded SpMM (rows whole,
    and column slices on the graph's plan, built by the eager call) and the
    16-bit column-sliced attention."""
    crow, col = case_graph(6000, 20, seed=5, hubs=12, hub_degree=4000, empty=0.05)
    rng = np.random.default_rng(5)
    x, q, k = (torch.from_numpy(rng.standard_normal((6000, f)).astype(np.float32)).to(torch.bfloat16).cuda()
               for f in (128, 64, 64))
    d_crow, d_col = to_dev(crow, col)
    ops = torch.ops.autosage
    calls = [
        lambda: ops.sddmm_csr(d_crow, d_col, q, k),
        lambda: ops.spmm_csr(d_crow, d_col, None, x),
        lambda: ops.spmm_csr_colslice(d_crow, d_col, None, x),
        lambda: ops.csr_attention_colslice(d_crow, d_col, q, k, x, 0.125),
    ]
    _replay_matches_eager(calls, lambda: (x.mul_(2.0), q.mul_(0.5)))


def _replay_matches_eager(calls, change_inputs):
    """Captures ``calls`` in one graph and checks three replays (eager work
    and a sync between them) against eager results, then a replay after
    ``change_inputs`` against fresh eager results."""
    # eager results, and warm-up on a side stream (default priority) as
    # graph capture wants
    eager = [c() for c in calls]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in calls:
            c()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = [c() for c in calls]
    for replay in range(3):
        # unrelated eager work and a sync between replays
        scratch = torch.randn(1 << 20, device="cuda")
        scratch.mul_(2.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(captured, eager)):
            assert torch.equal(got, want), (replay, i)
    # inputs changed in place: the replay sees them
    change_inputs()
    fresh = [c() for c in calls]
    graph.replay()
    torch.cuda.synchronize()
    for i, (got, want) in enumerate(zip(captured, fresh)):
        assert torch.equal(got, want), i
