"""Writes tests/golden/scheduler_golden.json from the AutoSAGE reference.

Run in the build container only (the reference tree is not on the GPU box):
    python tests/golden/make_golden.py /root/reference

It imports the reference's pure-Python modules (autosage/_cache.py,
autosage/_auto.py, autosage/utils/csr.py) and records, for small seeded CPU
inputs, the exact outputs the port must reproduce bit for bit:
graph_signature dictionaries (structure hash included), degree quantiles,
the candidate shortlist, the induced row sample (CPU generator), the
edge_index -> CSR build and the CPU row softmax.  Inputs are stored with the
outputs, so the fixture is self-contained.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "scheduler_golden.json"


def graphs():
    rng = np.random.default_rng(2024)
    cases = []
    for name, rows, deg, hubs in (("tiny", 5, 2, 0), ("small", 300, 6, 2), ("skewed", 2100, 2, 8)):
        d = rng.poisson(deg, size=rows)
        if hubs:
            d[rng.choice(rows, size=hubs, replace=False)] = rng.integers(200, 900, size=hubs)
        crow = np.concatenate([[0], np.cumsum(d)]).astype(np.int64)
        col = rng.integers(0, rows, size=int(crow[-1])).astype(np.int64)
        cases.append((name, crow, col))
    return cases


def main(reference: str) -> None:
    sys.path.insert(0, reference)
    from autosage._auto import _csr_row_softmax, _degree_quantiles, _induced_sample_csr, _spmm_candidates
    from autosage._cache import graph_signature
    from autosage.config import SchedulerConfig
    from autosage.utils.csr import edge_index_to_csr

    out = {"source": "AutoSAGE reference, autosage/_cache.py, _auto.py, utils/csr.py", "graphs": {},
           "signatures": [], "quantiles": [], "candidates": [], "samples": [], "csr": [], "softmax": []}
    for name, crow, col in graphs():
        t_crow, t_col = torch.from_numpy(crow), torch.from_numpy(col)
        val = torch.from_numpy(np.random.default_rng(len(crow)).random(col.size).astype(np.float32))
        scores = torch.from_numpy((np.random.default_rng(3).standard_normal(col.size) * 3).astype(np.float32))
        out["graphs"][name] = {"crow": crow.tolist(), "col": col.tolist(), "val": val.tolist(),
                               "scores": scores.tolist()}
        for op, weighted, dtype, f in (("spmm", False, torch.float32, 128), ("spmm", True, torch.float32, 64),
                                       ("sddmm", False, torch.float32, 64), ("spmm", False, None, 7)):
            sig = graph_signature(t_crow, t_col, f, op, weighted=weighted, dtype=dtype)
            out["signatures"].append({"name": f"{name}-{op}-{weighted}-{dtype}", "graph": name,
                                      "feature_width": f, "operation": op,
                                      "weighted": weighted, "dtype": None if dtype is None else str(dtype),
                                      "expected": sig})
        out["quantiles"].append({"name": name, "graph": name, "expected": list(_degree_quantiles(t_crow))})
        for f, k in ((64, 18), (128, 6), (256, 3)):
            cands = _spmm_candidates(t_crow, f, SchedulerConfig(candidate_count=k))
            out["candidates"].append({"name": f"{name}-F{f}-k{k}", "graph": name, "feature_width": f,
                                      "k": k, "expected": [list(c) for c in cands]})
        for frac, min_rows, seed in ((0.03, 4, 0), (0.5, 64, 7)):
            s_crow, s_col, s_val, sel = _induced_sample_csr(t_crow, t_col, val, fraction=frac, minimum_rows=min_rows,
                                                            seed=seed)
            out["samples"].append({"name": f"{name}-{frac}-{seed}", "graph": name,
                                   "fraction": frac, "minimum_rows": min_rows, "seed": seed,
                                   "expected": {"crow": s_crow.tolist(), "col": s_col.tolist(),
                                                "val": s_val.tolist(), "selected": sel.tolist()}})
        p = _csr_row_softmax(t_crow, scores)
        out["softmax"].append({"name": name, "graph": name, "expected_bits": p.numpy().view(np.uint32).tolist()})
    rng = np.random.default_rng(9)
    for n, e in ((6, 10), (50, 400), (700, 3000)):
        ei = rng.integers(0, n, size=(2, e)).astype(np.int64)
        for rows_by in ("dst", "src"):
            c, cc = edge_index_to_csr(torch.from_numpy(ei), n, rows_by=rows_by)
            out["csr"].append({"name": f"{n}-{e}-{rows_by}", "edge_index": ei.tolist(), "num_nodes": n,
                               "rows_by": rows_by, "expected": {"crow": c.tolist(), "col": cc.tolist()}})
    OUT.write_text(json.dumps(out, separators=(",", ":")))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
