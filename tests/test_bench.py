"""bench.py's bookkeeping on the CPU (no GPU): the byte formulas of the
measurement contract, the counter records under profiles/ that the bench
lines read their traffic from, the roofline object, and the refusal of more
than one GPU."""

from __future__ import annotations

import json
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

RECORD = re.compile(r"<!-- traffic: (\{.*?\}) -->")


def records():
    out = []
    for path in sorted((ROOT / "profiles").glob("*.md")):
        for m in RECORD.finditer(path.read_text(encoding="utf-8")):
            out.append((path, json.loads(m.group(1))))
    return out


def test_byte_formulas_give_the_contract_figures():
    # algorithmic and compulsory bytes of the benchmark configurations (GB)
    assert bench.spmm_bytes(232_965, 114_615_892, 128, False) / 1e9 == pytest.approx(59.72, abs=0.01)
    assert bench.spmm_compulsory_bytes(232_965, 114_615_892, 128, False) / 1e9 == pytest.approx(1.157, abs=0.001)
    assert bench.spmm_bytes(1 << 20, 16 * (1 << 20), 128, True) / 1e9 == pytest.approx(9.34, abs=0.01)
    assert bench.sddmm_bytes(1_000_000, 50_000_000, 64) / 1e9 == pytest.approx(13.66, abs=0.01)
    assert bench.attention_bytes(2_449_029, 123_718_280, 64, 128) / 1e9 == pytest.approx(97.9, abs=0.1)
    # 16-bit elements halve the feature bytes, not the index streams
    full = bench.spmm_bytes(1000, 5000, 64, True)
    half = bench.spmm_bytes(1000, 5000, 64, True, elem=2)
    assert full - half == 2 * 64 * 5000 + 2 * 64 * 1000 + 2 * 5000


def test_traffic_records_parse_and_are_unique():
    seen = {}
    recs = records()
    assert recs, "no counter records under profiles/"
    for path, rec in recs:
        for key in ("workload", "variant", "bytes", "fetch_scale", "write_scale", "source"):
            assert key in rec, (path.name, key)
        assert rec["source"] == f"profiles/{path.name}"
        key = (rec["workload"], rec["variant"])
        assert key not in seen, f"{key} recorded in {seen.get(key)} and {path.name}"
        seen[key] = path.name
        assert rec["bytes"] > 0


def test_no_record_claims_more_than_the_hbm_peak():
    for path, rec in records():
        k = rec.get("kernel")
        if k:
            gbps = k["bytes"] / (k["ms_per_step"] * 1e-3) / 1e9
            assert gbps <= bench.HBM_PEAK_GBPS * 1.02, (path.name, rec["workload"], gbps)
        if "l2_hit_rate" in rec:
            assert 0.0 <= rec["l2_hit_rate"] <= 1.0
        if "all_cached_ms" in rec:
            assert 0.0 < rec["all_cached_ms"] < k["ms_per_step"]


@pytest.mark.parametrize("workload", [
    "cfg3 SpMM fp32 F=128 unweighted",
    "cfg3 SpMM fp32 F=64 unweighted",
    "cfg3 SpMM fp32 F=256 unweighted",
    "cfg3 SpMM fp32 F=128 unweighted forward+backward (dX)",
] + [f"cfg3 SpMM fp32 F=128 unweighted, row shard {k} of 8" for k in range(8)])
def test_the_cfg3_lines_find_their_own_record(workload):
    rec = bench.profiled_traffic(workload, "colslice")
    assert rec is not None and rec["workload"] == workload and rec["variant"] == "colslice"
    # the row-sorted copy of a shuffled graph is the graph itself
    if "," not in workload and "backward" not in workload:
        shuffled = bench.profiled_traffic(workload + " shuffled columns", "colslice")
        assert shuffled["bytes"] == rec["bytes"]
    # another variant never borrows this record
    assert bench.profiled_traffic(workload, "whole") is None


def test_roofline_object_is_a_fraction_of_the_hbm_peak():
    rec = bench.profiled_traffic("cfg3 SpMM fp32 F=128 unweighted", "colslice")
    ms = rec["kernel"]["ms_per_step"]
    line = bench.roofline_record(ms, bench.spmm_bytes(232_965, 114_615_892, 128, False),
                                 bench.spmm_compulsory_bytes(232_965, 114_615_892, 128, False), rec,
                                 (114_615_892 + 232_965) * 128 * 4)
    assert line["bound"] == "hbm" and line["unit"] == "GB/s" and line["peak"] == bench.HBM_PEAK_GBPS
    assert line["traffic"] == rec["bytes"]
    assert 0.0 < line["frac"] <= 1.0
    assert line["frac"] == pytest.approx(rec["bytes"] / (ms * 1e-3) / 1e9 / bench.HBM_PEAK_GBPS, rel=1e-3)
    # the algorithmic figure (every gather in full) stays beside it, above the peak on this graph
    assert line["algorithmic_gbps"] > bench.HBM_PEAK_GBPS
    assert line["all_cached_ceiling"]["frac"] == pytest.approx(rec["all_cached_ms"] / ms, rel=1e-3)
    # without a record the compulsory bytes stand in, and the basis says so
    fallback = bench.roofline_record(ms, 10, 5, None, 10)
    assert fallback["traffic"] is None and "compulsory" in fallback["basis"]


def test_bench_measures_one_gpu_only():
    run = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=300, cwd=ROOT)
    assert run.returncode == 2
    assert "one GPU" in run.stderr
    assert run.stdout == ""
