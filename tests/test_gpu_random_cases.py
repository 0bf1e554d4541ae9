"""Seeded random sweep over graph shapes, feature widths, weights and types,
every op against its oracle at its own bar:

* ``spmm_csr`` / ``spmm_csr_split`` / ``spmm_csr_fslice`` (fp32, the latter
  in 1 to 4 column phases): bit-identical to the sequential CSR product
  (``oracle.spmm_seq``);
* ``spmm_csr_colslice`` (fp32, ascending columns): |gpu − fp64| ≤
  1e-6·|fp64| + 1e-9;
* ``sddmm_csr`` / ``sddmm_csr_split`` (fp32): bit-identical to the reference
  kernel order (``oracle.sddmm_ref``);
* bf16 / fp16 SpMM and SDDMM: bit-identical to the rounded fp64 oracles;
* ``csr_row_softmax`` (fp32): within 1e-5 relative / 1e-6 absolute of the
  reference composition.

Each case draws rows, mean degree, hub rows and their degree, empty rows and
F from one seed, so a failure names a reproducible case.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from autosage_amd import _native, synth
from tests.gpu_common import require_gpu, to_dev

pytestmark = pytest.mark.gpu

CASES = 200


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    require_gpu()


def _case(seed: int):
    rng = np.random.default_rng(1000 + seed)
    rows = int(rng.choice([1, 7, 64, 300, 2000, 6000]))
    degree = float(rng.choice([0.5, 3, 12, 40]))
    hubs = int(rng.integers(0, 4)) if rows >= 64 else 0
    hub_degree = int(rng.choice([100, 700, 1500, 3000])) if hubs else 0
    empty = float(rng.choice([0.0, 0.1, 0.5]))
    features = int(rng.choice([1, 3, 8, 16, 24, 33, 64, 96, 128, 136, 256, 264, 512]))
    crow, col = synth.random_csr(rows, degree, seed=seed, hub_rows=hubs, hub_degree=hub_degree,
                                 empty_fraction=empty)
    x = rng.standard_normal((rows, features)).astype(np.float32)
    val = rng.standard_normal(col.size).astype(np.float32) if rng.random() < 0.5 else None
    q = rng.standard_normal((rows, features)).astype(np.float32)
    return crow, col, val, x, q


@pytest.mark.parametrize("seed", range(CASES))
def test_random_case(seed, monkeypatch):
    crow, col, val, x, q = _case(seed)
    d_crow, d_col, d_x, d_q = to_dev(crow, col, x, q)
    d_val = None if val is None else torch.from_numpy(val).cuda()
    tag = f"seed {seed}: rows {crow.size - 1}, nnz {col.size}, F {x.shape[1]}, weighted {val is not None}"
    # fp32 SpMM, bit-exact schedules
    want = oracle.spmm_seq(crow, col, val, x)
    assert np.array_equal(torch.ops.autosage.spmm_csr(d_crow, d_col, d_val, d_x).cpu().numpy(), want), tag
    assert np.array_equal(torch.ops.autosage.spmm_csr_split(d_crow, d_col, d_val, d_x, 64, 2, 256).cpu().numpy(),
                          want), tag
    monkeypatch.setenv("AUTOSAGE_FSLICE_PHASES", str(1 + seed % 4))
    assert np.array_equal(torch.ops.autosage.spmm_csr_fslice(d_crow, d_col, d_val, d_x).cpu().numpy(), want), \
        (tag, 1 + seed % 4)
    # column slices (the generator's columns ascend)
    exact = oracle.spmm_f64(crow, col, val, x)
    got = torch.ops.autosage.spmm_csr_colslice(d_crow, d_col, d_val, d_x).cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - exact) <= 1e-6 * np.abs(exact) + 1e-9), tag
    # fp32 SDDMM in the reference order
    ref = oracle.sddmm_ref(crow, col, q, x)
    assert np.array_equal(torch.ops.autosage.sddmm_csr(d_crow, d_col, d_q, d_x).cpu().numpy(), ref), tag
    assert np.array_equal(torch.ops.autosage.sddmm_csr_split(d_crow, d_col, d_q, d_x, 2, 128).cpu().numpy(), ref), tag
    # 16-bit SpMM and SDDMM
    dtype = torch.bfloat16 if seed % 2 == 0 else torch.float16
    x16, q16 = torch.from_numpy(x).to(dtype), torch.from_numpy(q).to(dtype)
    v16 = None if val is None else torch.from_numpy(val).to(dtype)
    want16 = oracle.spmm_rounded_16(crow, col, v16, x16, dtype).view(torch.int16)
    d_v16 = None if v16 is None else v16.cuda()
    y16 = torch.ops.autosage.spmm_csr(d_crow, d_col, d_v16, x16.cuda()).cpu()
    assert torch.equal(y16.view(torch.int16), want16), tag
    for columns in (True, False):
        y16 = _native.spmm_rounded_16_impl(d_crow, d_col, d_v16, x16.cuda(), column_slices=columns).cpu()
        assert torch.equal(y16.view(torch.int16), want16), (tag, columns)
    s16 = torch.ops.autosage.sddmm_csr(d_crow, d_col, q16.cuda(), x16.cuda()).cpu()
    assert torch.equal(s16.view(torch.int16), oracle.sddmm_rounded_16(crow, col, q16, x16, dtype).view(torch.int16)), tag
    # row softmax of the fp32 scores
    if col.size:
        p = torch.ops.autosage.csr_row_softmax(d_crow, torch.from_numpy(ref).cuda()).cpu().numpy()
        want_p = oracle.row_softmax(crow, ref)
        assert np.all(np.abs(p - want_p) <= 1e-5 * np.abs(want_p) + 1e-6), tag
