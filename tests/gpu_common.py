"""Shared helpers for the GPU parity tests."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import autosage_amd
from autosage_amd import synth


def require_gpu():
    """Skips without a GPU; with a GPU the HIP library must load (no silent
    fallback), otherwise the test fails."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not autosage_amd.load_native():
        from autosage_amd.ops import native_load_error

        pytest.fail(f"HIP library failed to load on a GPU machine: {native_load_error()}")


def case_graph(rows: int, degree: float, seed: int, hubs: int = 0, hub_degree: int = 0, empty: float = 0.0):
    crow, col = synth.random_csr(rows, degree, seed=seed, hub_rows=hubs, hub_degree=hub_degree, empty_fraction=empty)
    return crow, col


def to_dev(*arrays):
    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def bitwise_equal(gpu: torch.Tensor, ref: np.ndarray) -> bool:
    got = gpu.detach().cpu().numpy()
    return got.shape == ref.shape and np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def mismatch_report(gpu: torch.Tensor, ref: np.ndarray) -> str:
    got = gpu.detach().cpu().numpy()
    bad = np.argwhere(got != ref)
    return f"{len(bad)} mismatches, first {bad[:5].tolist()}: got {got[tuple(bad[0])] if len(bad) else None}"


def elementwise_parity(got: np.ndarray, ref: np.ndarray, exact: np.ndarray, *, tight_rel: float,
                       tight_abs: float, rtol: float = 1e-5, atol: float = 1e-6,
                       accept_both_within_bar: bool = False) -> dict:
    """Per-element parity of a reassociating kernel with the reference's fp32
    result ``ref``, against the exact (fp64) result ``exact``.  With
    bar(v) = rtol·|v| + atol and the kernel's bound δ = tight_rel·|exact| +
    tight_abs, every element must satisfy one of:

    (a) |got − ref| <= bar(ref): within the bar of the reference;
    (b) |ref − exact| > bar(exact): the reference itself misses the bar
        against the exact result, while |got − exact| <= δ and
        |got − exact| <= |ref − exact|;
    (c) bar(exact) − δ < |ref − exact| <= bar(exact): the reference is within
        δ of missing the bar, while |got − exact| <= δ and |got − exact| <=
        |ref − exact|.  If |got − exact| <= δ and (a) fails, the triangle
        inequality puts |ref − exact| above roughly bar − δ, so (c) is the
        boundary band that (a) and (b) leave between them.

    With ``accept_both_within_bar`` a fourth case counts:

    (d) |ref − exact| <= bar(exact) and |got − exact| <= δ: both results are
        within the bar of the exact one, on opposite sides of it, so neither
        is the more correct (used for gradients, where the reference's
        autograd and the kernel sum the same terms in unrelated orders).

    Returns the counts (and the largest |ref − exact| / bar(exact) among the
    elements of (b) and (c)); raises AssertionError naming them when an
    element meets none."""
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    bar_exact = rtol * np.abs(exact) + atol
    bound = tight_rel * np.abs(exact) + tight_abs
    near_ref = np.abs(got - ref) <= rtol * np.abs(ref) + atol
    ref_err = np.abs(ref - exact)
    got_err = np.abs(got - exact)
    kernel_ok = (got_err <= bound) & (got_err <= ref_err)
    ref_misses = ref_err > bar_exact
    ref_edge = ~ref_misses & (ref_err > bar_exact - bound)
    case_b = ~near_ref & ref_misses & kernel_ok
    case_c = ~near_ref & ref_edge & kernel_ok
    case_d = ~near_ref & ~case_b & ~case_c & ~ref_misses & (got_err <= bound)
    neither = ~near_ref & ~case_b & ~case_c & ~(case_d if accept_both_within_bar else np.zeros_like(case_d))
    ratio = ref_err / bar_exact
    counts = {
        "elements": int(got.size),
        "a_within_bar_of_reference": int(near_ref.sum()),
        "b_reference_off_bar_kernel_within_bound": int(case_b.sum()),
        "c_reference_at_bar_edge_kernel_within_bound": int(case_c.sum()),
        "reference_off_bar_total": int(ref_misses.sum()),
        "worst_reference_error_over_bar": float(ratio.max()) if ratio.size else 0.0,
        "min_reference_error_over_bar_in_c": float(ratio[case_c].min()) if case_c.any() else None,
        "worst_kernel_error_over_bar": float((got_err / bar_exact).max()) if got.size else 0.0,
        "neither": int(neither.sum()),
    }
    if accept_both_within_bar:
        counts["d_both_within_bar_of_exact"] = int(case_d.sum())
    print(f"[parity] {counts}", flush=True)
    assert counts["neither"] == 0, counts
    return counts


def elementwise_parity_rows(got: np.ndarray, ref: np.ndarray, exact: np.ndarray, *, tight_rel: float,
                            tight_abs: float, chunk_rows: int = 65536, label: str = "") -> dict:
    """``elementwise_parity`` over every element of large outputs, in chunks
    of rows (bounded host memory); the counts are summed and the worst
    ratios kept.  Prints one ``[parity]`` line with the totals."""
    total: dict = {}
    for start in range(0, got.shape[0], chunk_rows):
        stop = min(start + chunk_rows, got.shape[0])
        part = _parity_counts(got[start:stop], ref[start:stop], exact[start:stop], tight_rel=tight_rel,
                              tight_abs=tight_abs)
        for key, value in part.items():
            if key.startswith("worst"):
                total[key] = max(total.get(key, 0.0), value)
            elif key.startswith("min_"):
                if value is not None:
                    total[key] = value if total.get(key) is None else min(total[key], value)
                else:
                    total.setdefault(key, None)
            else:
                total[key] = total.get(key, 0) + value
    print(f"[parity] {label} {total}", flush=True)
    assert total["neither"] == 0, total
    return total


def _parity_counts(got, ref, exact, *, tight_rel, tight_abs, rtol=1e-5, atol=1e-6) -> dict:
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    exact = exact.astype(np.float64)
    bar_exact = rtol * np.abs(exact) + atol
    bound = tight_rel * np.abs(exact) + tight_abs
    near_ref = np.abs(got - ref) <= rtol * np.abs(ref) + atol
    ref_err = np.abs(ref - exact)
    got_err = np.abs(got - exact)
    kernel_ok = (got_err <= bound) & (got_err <= ref_err)
    ref_misses = ref_err > bar_exact
    ref_edge = ~ref_misses & (ref_err > bar_exact - bound)
    case_b = ~near_ref & ref_misses & kernel_ok
    case_c = ~near_ref & ref_edge & kernel_ok
    ratio = ref_err / bar_exact
    return {
        "elements": int(got.size),
        "a_within_bar_of_reference": int(near_ref.sum()),
        "b_reference_off_bar_kernel_within_bound": int(case_b.sum()),
        "c_reference_at_bar_edge_kernel_within_bound": int(case_c.sum()),
        "reference_off_bar_total": int(ref_misses.sum()),
        "worst_reference_error_over_bar": float(ratio.max()) if ratio.size else 0.0,
        "worst_kernel_error_over_bar": float((got_err / bar_exact).max()) if got.size else 0.0,
        "min_reference_error_over_bar_in_c": float(ratio[case_c].min()) if case_c.any() else None,
        "neither": int((~near_ref & ~case_b & ~case_c).sum()),
    }


def assert_spmm_contract(out: torch.Tensor, info: dict, crow, col, val, x) -> None:
    """The contract of the schedule ``spmm_csr_auto`` chose: the exact native
    schedules equal the sequential oracle bit for bit; the column-sliced one
    is within 1e-6·|fp64| + 1e-9 of the fp64 product; the PyTorch baseline
    (another summation order) within the reference suite's tolerance."""
    import oracle

    got = out.detach().cpu().numpy()
    if info["choice"] == "autosage" and info.get("candidate") == "colslice":
        exact = oracle.spmm_f64(crow, col, val, x)
        assert np.all(np.abs(got - exact) <= 1e-6 * np.abs(exact) + 1e-9)
    elif info["choice"] == "autosage":
        assert bitwise_equal(out, oracle.spmm_seq(crow, col, val, x))
    else:
        assert np.allclose(got, oracle.spmm_seq(crow, col, val, x), rtol=1e-4, atol=1e-3)
