"""Seeded synthetic workloads for the five benchmark configurations.

The reference benchmarks real graphs (Reddit, ogbn-products) and simple
synthetic ones (``scripts/benchmark.py:97-139``); the workloads here are the
five seeded configurations of the benchmark contract:

1. N=16,384, degree U{4..12}, distinct sorted uniform columns, unweighted,
   X [N, 64] ~ N(0, 1)                                  (CPU-runnable SpMM)
2. N=2^20, exactly 16 distinct sorted uniform columns per row, weights
   U(0, 1), X [N, 128]                                   (uniform SpMM)
3. N=232,965, nnz=114,615,892, truncated power-law degrees (alpha 1.8, max
   21,000), columns drawn proportionally to degree, unweighted, X [N, F]
                                                         (skewed / hub SpMM)
4. N=10^6, nnz~50M: Zipf(1.5) body (min 2, so median 8) plus 100 hub rows
   with 50k-200k nonzeros; Q, K [N, F] ~ N(0, 1/F)       (SDDMM)
5. N=2,449,029, nnz~123.7M: symmetrised power-law graph (alpha 2.1, max
   ~17,500); Q, K [N, 64] ~ N(0, 1), V [N, 128]          (attention)

Degrees and dense features come from ``numpy.random.default_rng(seed)``;
columns come from ``synth.cpp`` (per-row counter-seeded streams, OpenMP), so a
configuration is identical on every machine and thread count.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import subprocess
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "synth.cpp"
LIBRARY = HERE / "libautosage_synth.so"

_lib: Optional[ctypes.CDLL] = None


def build() -> Path:
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp", str(SOURCE), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"building the generator failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        p, i64 = ctypes.c_void_p, ctypes.c_int64
        lib.synth_fill_columns.argtypes = [p, i64, i64, ctypes.c_int, p, ctypes.c_uint64, p]
        lib.synth_fill_columns.restype = ctypes.c_int
        lib.synth_transpose.argtypes = [p, p, i64, p, p]
        lib.synth_transpose.restype = ctypes.c_int
        lib.synth_union_rows.argtypes = [p, p, p, p, i64, p, p]
        lib.synth_union_rows.restype = ctypes.c_int
        _lib = lib
    return _lib


def _crow_from_degrees(deg: np.ndarray) -> np.ndarray:
    crow = np.zeros(deg.size + 1, dtype=np.int64)
    np.cumsum(deg, out=crow[1:])
    return crow


def fill_columns(crow: np.ndarray, n_cols: int, seed: int, weights: Optional[np.ndarray] = None) -> np.ndarray:
    """Distinct ascending columns per row; uniform, or proportional to ``weights``."""
    crow = np.ascontiguousarray(crow, dtype=np.int64)
    col = np.empty(int(crow[-1]), dtype=np.int64)
    cum = None
    mode = 0
    if weights is not None:
        cum = np.zeros(n_cols + 1, dtype=np.int64)
        np.cumsum(np.asarray(weights, dtype=np.int64), out=cum[1:])
        mode = 1
    status = _load().synth_fill_columns(
        crow.ctypes.data, crow.size - 1, n_cols, mode, None if cum is None else cum.ctypes.data, seed, col.ctypes.data
    )
    if status != 0:
        raise ValueError("a row degree exceeds the number of columns")
    return col


def symmetrize(crow: np.ndarray, col: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """A ∪ Aᵀ for a square CSR with sorted unique rows."""
    n = crow.size - 1
    lib = _load()
    t_crow = np.empty(n + 1, dtype=np.int64)
    t_col = np.empty(col.size, dtype=np.int64)
    lib.synth_transpose(crow.ctypes.data, col.ctypes.data, n, t_crow.ctypes.data, t_col.ctypes.data)
    out_crow = np.empty(n + 1, dtype=np.int64)
    lib.synth_union_rows(crow.ctypes.data, col.ctypes.data, t_crow.ctypes.data, t_col.ctypes.data, n,
                         out_crow.ctypes.data, None)
    out_col = np.empty(int(out_crow[-1]), dtype=np.int64)
    lib.synth_union_rows(crow.ctypes.data, col.ctypes.data, t_crow.ctypes.data, t_col.ctypes.data, n,
                         out_crow.ctypes.data, out_col.ctypes.data)
    return out_crow, out_col


def _truncated_pareto(rng: np.random.Generator, n: int, alpha: float, lo: float, hi: float) -> np.ndarray:
    """Continuous density ∝ d^-alpha on [lo, hi], by inverse CDF."""
    u = rng.random(n)
    a, b = lo ** (1.0 - alpha), hi ** (1.0 - alpha)
    return (a + u * (b - a)) ** (1.0 / (1.0 - alpha))


def _pareto_mean(alpha: float, lo: float, hi: float) -> float:
    num = (hi ** (2.0 - alpha) - lo ** (2.0 - alpha)) / (2.0 - alpha)
    den = (hi ** (1.0 - alpha) - lo ** (1.0 - alpha)) / (1.0 - alpha)
    return num / den


def _solve_lo(alpha: float, hi: float, mean: float) -> float:
    lo_a, lo_b = 1.0, hi
    for _ in range(200):
        mid = 0.5 * (lo_a + lo_b)
        if _pareto_mean(alpha, mid, hi) < mean:
            lo_a = mid
        else:
            lo_b = mid
    return 0.5 * (lo_a + lo_b)


def _match_total(rng: np.random.Generator, deg: np.ndarray, target: int, lo: int, hi: int) -> np.ndarray:
    """Adds or removes single nonzeros at random rows (within [lo, hi]) until
    the degrees sum to ``target``."""
    deg = deg.astype(np.int64)
    diff = int(target - deg.sum())
    while diff != 0:
        step = 1 if diff > 0 else -1
        count = min(abs(diff), deg.size)
        rows = rng.choice(deg.size, size=count, replace=False)
        ok = (deg[rows] + step >= lo) & (deg[rows] + step <= hi)
        deg[rows[ok]] += step
        diff -= step * int(ok.sum())
    return deg


@dataclass
class Workload:
    name: str
    crow: np.ndarray
    col: np.ndarray
    val: Optional[np.ndarray] = None
    dense: dict = field(default_factory=dict)
    notes: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return self.crow.size - 1

    @property
    def nnz(self) -> int:
        return self.col.size

    def degree_stats(self) -> dict:
        deg = np.diff(self.crow)
        return {
            "rows": int(self.rows),
            "nnz": int(self.nnz),
            "mean_degree": float(deg.mean()) if deg.size else 0.0,
            "median_degree": float(np.median(deg)) if deg.size else 0.0,
            "max_degree": int(deg.max()) if deg.size else 0,
            "frac_deg_gt_2000": float((deg > 2000).mean()) if deg.size else 0.0,
        }

    def fingerprint(self) -> str:
        h = hashlib.sha256()
        h.update(self.crow.tobytes())
        h.update(self.col.tobytes())
        if self.val is not None:
            h.update(self.val.tobytes())
        return h.hexdigest()[:16]


def config1(seed: int = 0, features: int = 64) -> Workload:
    rng = np.random.default_rng(seed)
    n = 16_384
    deg = rng.integers(4, 13, size=n)
    crow = _crow_from_degrees(deg)
    col = fill_columns(crow, n, seed)
    x = rng.standard_normal((n, features), dtype=np.float32)
    return Workload("cfg1", crow, col, None, {"x": x})


def config2(seed: int = 0, features: int = 128, rows: int = 1 << 20) -> Workload:
    rng = np.random.default_rng(seed)
    deg = np.full(rows, 16, dtype=np.int64)
    crow = _crow_from_degrees(deg)
    col = fill_columns(crow, rows, seed)
    val = rng.random(col.size, dtype=np.float32)
    x = rng.standard_normal((rows, features), dtype=np.float32)
    return Workload("cfg2", crow, col, val, {"x": x})


CFG3_ROWS = 232_965
CFG3_NNZ = 114_615_892
CFG3_MAX_DEGREE = 21_000


def config3(seed: int = 0, features: int = 128, rows: int = CFG3_ROWS, nnz: int = CFG3_NNZ,
            max_degree: int = CFG3_MAX_DEGREE, alpha: float = 1.8, with_x: bool = True) -> Workload:
    rng = np.random.default_rng(seed)
    mean = nnz / rows
    lo = _solve_lo(alpha, float(max_degree), mean)
    deg = np.rint(_truncated_pareto(rng, rows, alpha, lo, float(max_degree))).astype(np.int64)
    deg = np.clip(deg, 1, max_degree)
    deg[int(np.argmax(deg))] = max_degree
    deg = _match_total(rng, deg, nnz, 1, max_degree)
    crow = _crow_from_degrees(deg)
    col = fill_columns(crow, rows, seed, weights=deg)
    dense = {}
    if with_x:
        dense["x"] = rng.standard_normal((rows, features), dtype=np.float32)
    return Workload("cfg3", crow, col, None, dense, {"alpha": alpha, "min_degree_param": lo})


def config4(seed: int = 0, features: int = 128, rows: int = 1_000_000, nnz: int = 50_000_000, hubs: int = 100,
            hub_range: tuple[int, int] = (50_000, 200_000), with_dense: bool = True) -> Workload:
    rng = np.random.default_rng(seed)
    hub_deg = rng.integers(hub_range[0], hub_range[1] + 1, size=hubs)
    body_target = nnz - int(hub_deg.sum())
    # Zipf(1.5) body: P(D > d) = (2/d)^0.5 for d >= 2 (median 8), capped so the
    # body sums to the target.
    u = rng.random(rows - hubs)
    raw = np.floor(2.0 * u ** (-2.0))
    cap_lo, cap_hi = 2.0, float(hub_range[0])
    for _ in range(100):
        cap = 0.5 * (cap_lo + cap_hi)
        if np.minimum(raw, cap).sum() < body_target:
            cap_lo = cap
        else:
            cap_hi = cap
    body = np.minimum(raw, np.floor(cap_lo)).astype(np.int64)
    body = _match_total(rng, body, body_target, 2, int(cap_lo) + 1)
    deg = np.concatenate([hub_deg, body])
    rng.shuffle(deg)
    crow = _crow_from_degrees(deg)
    col = fill_columns(crow, rows, seed)
    dense = {}
    if with_dense:
        scale = np.float32(1.0 / np.sqrt(features))
        dense["q"] = rng.standard_normal((rows, features), dtype=np.float32) * scale
        dense["k"] = rng.standard_normal((rows, features), dtype=np.float32) * scale
    return Workload("cfg4", crow, col, None, dense, {"body_cap": float(cap_lo)})


def config5(seed: int = 0, rows: int = 2_449_029, target_nnz: int = 123_718_280, max_degree: int = 17_500,
            alpha: float = 2.1, f_qk: int = 64, f_v: int = 128, with_dense: bool = True) -> Workload:
    rng = np.random.default_rng(seed)
    # Directed out-degrees: power-law tail alpha, body minimum calibrated so the
    # symmetrised graph lands near target_nnz (the union roughly doubles the
    # directed nonzeros, minus reciprocal pairs).
    half_max = max_degree // 2
    lo = _solve_lo(alpha, float(half_max), target_nnz / (2.0 * rows))
    deg = np.rint(_truncated_pareto(rng, rows, alpha, lo, float(half_max))).astype(np.int64)
    deg = np.clip(deg, 1, half_max)
    deg = _match_total(rng, deg, target_nnz // 2, 1, half_max)
    crow = _crow_from_degrees(deg)
    col = fill_columns(crow, rows, seed, weights=deg)
    crow, col = symmetrize(crow, col)
    dense = {}
    if with_dense:
        dense["q"] = rng.standard_normal((rows, f_qk), dtype=np.float32)
        dense["k"] = rng.standard_normal((rows, f_qk), dtype=np.float32)
        dense["v"] = rng.standard_normal((rows, f_v), dtype=np.float32)
    return Workload("cfg5", crow, col, None, dense, {"alpha": alpha})


def random_csr(rows: int, mean_degree: float, seed: int = 0, hub_rows: int = 0, hub_degree: int = 0,
               cols: Optional[int] = None, empty_fraction: float = 0.0) -> tuple[np.ndarray, np.ndarray]:
    """Small test graphs: Poisson degrees, optional hub rows and empty rows,
    distinct sorted uniform columns."""
    rng = np.random.default_rng(seed)
    cols = rows if cols is None else cols
    deg = np.minimum(rng.poisson(mean_degree, size=rows), cols).astype(np.int64)
    if empty_fraction > 0:
        deg[rng.random(rows) < empty_fraction] = 0
    if hub_rows:
        deg[rng.choice(rows, size=hub_rows, replace=False)] = min(hub_degree, cols)
    crow = _crow_from_degrees(deg)
    return crow, fill_columns(crow, cols, seed)


def erdos_renyi(rows: int = 200_000, probability: float = 2e-5, seed: int = 0, features: int = 64) -> Workload:
    """The reference benchmark's ``synth:<rows>:<p>`` graph
    (``scripts/benchmark.py:97-108``, CSR build ``:64-76``): int(p·rows²)
    (row, column) pairs drawn uniformly with ``default_rng(seed).integers``,
    duplicates removed, rows ascending and columns ascending within rows.
    The same generator calls in the same order give the same graph (the
    published run, ``artifacts/results/spmm/synth_er.csv``, has 799,994
    nonzeros for 200,000 rows at p = 2e-5, seed 0).  X [rows, features]
    ~ N(0, 1) is drawn afterwards from the same generator."""
    rng = np.random.default_rng(seed)
    count = max(1, int(probability * rows * rows))
    src = rng.integers(0, rows, size=count, dtype=np.int64)
    dst = rng.integers(0, rows, size=count, dtype=np.int64)
    # unique (row, column) keys come back sorted: rows ascending, columns
    # ascending inside each row
    keys = np.unique(src * np.int64(rows) + dst)
    row, col = keys // np.int64(rows), keys % np.int64(rows)
    crow = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(row, minlength=rows), out=crow[1:])
    x = rng.standard_normal((rows, features), dtype=np.float32)
    return Workload("er", crow, col, None, {"x": x}, {"probability": probability})


def hub_sweep_graph(rows: int = 20_000, hub_degree: int = 12_000, other_degree: int = 32, seed: int = 0,
                    device: str = "cuda"):
    """The reference hub sweep's graph (``scripts/sweep_hubs.py:15-27``):
    row 0 has ``hub_degree`` edges, every other row ``other_degree``; the
    columns are uniform draws of ``torch.randint`` from a device generator
    seeded with ``seed``, in CSR order (not sorted within rows, duplicates
    allowed).  Returns device tensors (crow, col)."""
    import torch

    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    degrees = torch.full((rows,), other_degree, device=device, dtype=torch.long)
    degrees[0] = hub_degree
    crow = torch.cat((torch.zeros(1, device=device, dtype=torch.long), degrees.cumsum(0)))
    nnz = hub_degree + (rows - 1) * other_degree
    col = torch.randint(0, rows, (nnz,), generator=generator, device=device)
    return crow, col
