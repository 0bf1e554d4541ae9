"""Schedule keys and cache file: the behaviour the reference's
tests/test_cache.py pins (directory read per call, schema 1, signature
fields, distinct weighted / dtype keys), plus golden and closed-form checks."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from autosage_amd._cache import ScheduleCache, cache_directory, device_signature, graph_signature, log_probe

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_cache_follows_the_directory_variable_at_each_call(tmp_path, monkeypatch):
    """AUTOSAGE_CACHE_DIR is read when a cache is opened, not at import: two
    directories keep two independent schedule files (schema 1)."""
    device = {"name": "gfx950", "torch": torch.__version__}
    graph = {"operation": "spmm", "rows": 5, "nonzeros": 9}
    for name, choice in (("first", "autosage"), ("second", "baseline")):
        monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path / name))
        assert cache_directory() == tmp_path / name
        assert ScheduleCache().lookup(device, graph) is None
        ScheduleCache().store(device, graph, {"choice": choice})
        assert ScheduleCache().lookup(device, graph)["result"] == {"choice": choice}
    for name in ("first", "second"):
        stored = json.loads((tmp_path / name / "schedules.json").read_text(encoding="utf-8"))
        assert stored["schema_version"] == 1


def test_graph_signature_counts_survive_json():
    """Row and nonzero counts are plain ints (exact in the JSON cache key)
    and the structure hash is 24 hex digits."""
    degrees = [2, 0, 5, 1]
    crow = torch.tensor([0, 2, 2, 7, 8], dtype=torch.long)
    col = torch.tensor([1, 3, 0, 1, 2, 3, 3, 0], dtype=torch.long)
    for width, operation in ((32, "spmm"), (7, "sddmm")):
        signature = graph_signature(crow, col, width, operation)
        assert (signature["rows"], signature["nonzeros"]) == (len(degrees), sum(degrees))
        assert signature["operation"] == operation
        assert type(signature["rows"]) is int and type(signature["nonzeros"]) is int
        assert json.loads(json.dumps(signature)) == signature
        assert len(signature["structure_hash"]) == 24
        int(signature["structure_hash"], 16)


def test_every_weight_and_dtype_variant_has_its_own_key():
    crow = torch.tensor([0, 2, 3], dtype=torch.long)
    col = torch.tensor([0, 1, 1], dtype=torch.long)
    keys = set()
    for weighted in (False, True):
        for dtype in (torch.float32, torch.float64, torch.bfloat16):
            keys.add(json.dumps(graph_signature(crow, col, 64, "spmm", weighted=weighted, dtype=dtype),
                                sort_keys=True))
    assert len(keys) == 6


def test_structure_hash_closed_form():
    # sha256 over little-endian int64 bytes of crow then col, each cut to its
    # first and last 1024 entries when longer than 2048.
    crow = torch.arange(0, 3001, dtype=torch.long)
    col = torch.arange(3000, dtype=torch.long) % 7
    h = hashlib.sha256()
    for arr in (crow.numpy(), col.numpy()):
        part = np.concatenate([arr[:1024], arr[-1024:]]) if arr.size > 2048 else arr
        h.update(part.astype("<i8").tobytes())
    assert graph_signature(crow, col, 8, "spmm")["structure_hash"] == h.hexdigest()[:24]


def test_degree_quantiles_in_signature():
    crow = torch.tensor([0, 1, 3, 3, 10], dtype=torch.long)  # degrees 1 2 0 7
    sig = graph_signature(crow, torch.zeros(10, dtype=torch.long), 4, "sddmm")
    # linear quantiles: q50 = 1.5 -> 2, q90 = 5.5 -> 6, q99 = 6.85 -> 7
    assert (sig["degree_q50"], sig["degree_q90"], sig["degree_q99"]) == (2, 6, 7)


def test_corrupt_or_foreign_cache_file_is_empty(tmp_path):
    path = tmp_path / "schedules.json"
    path.write_text("{not json")
    assert ScheduleCache(path).lookup({}, {}) is None
    path.write_text(json.dumps({"schema_version": 99, "records": {"x": 1}}))
    assert ScheduleCache(path)._records == {}


def test_store_is_atomic_and_sorted(tmp_path):
    path = tmp_path / "schedules.json"
    cache = ScheduleCache(path)
    cache.store({"type": "cpu"}, {"rows": 1}, {"choice": "baseline"})
    assert [p.name for p in tmp_path.iterdir()] == ["schedules.json"]
    text = path.read_text()
    assert text.endswith("\n")
    key = json.dumps({"device": {"type": "cpu"}, "graph": {"rows": 1}}, sort_keys=True, separators=(",", ":"))
    assert key in json.loads(text)["records"]


def test_probe_log_can_be_disabled(tmp_path, monkeypatch):
    monkeypatch.setenv("AUTOSAGE_CACHE_DIR", str(tmp_path))
    monkeypatch.setenv("AUTOSAGE_LOG_PROBES", "0")
    log_probe({"a": 1})
    assert not (tmp_path / "probe_logs.jsonl").exists()
    monkeypatch.setenv("AUTOSAGE_LOG_PROBES", "1")
    log_probe({"a": 1})
    assert (tmp_path / "probe_logs.jsonl").read_text() == '{"a": 1}\n'


def test_cpu_device_signature():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    assert device_signature() == {"type": "cpu", "torch": torch.__version__}


def test_signatures_match_reference_golden():
    """graph_signature dictionaries, structure hash included, equal the
    reference's for the same inputs."""
    g = json.loads((GOLDEN / "scheduler_golden.json").read_text())
    assert len(g["signatures"]) >= 12
    for case in g["signatures"]:
        gr = g["graphs"][case["graph"]]
        crow = torch.tensor(gr["crow"], dtype=torch.long)
        col = torch.tensor(gr["col"], dtype=torch.long)
        dtype = None if case["dtype"] is None else getattr(torch, case["dtype"].split(".")[-1])
        got = graph_signature(crow, col, case["feature_width"], case["operation"], weighted=case["weighted"],
                              dtype=dtype)
        assert got == case["expected"], case["name"]


def test_signature_memo_hits_only_for_the_same_unmodified_tensors():
    from autosage_amd._cache import graph_signature_memo

    crow = torch.tensor([0, 1, 3, 3], dtype=torch.long)
    col = torch.tensor([0, 1, 2], dtype=torch.long)
    first = graph_signature_memo(crow, col, 8, "spmm")
    assert first == graph_signature(crow, col, 8, "spmm")
    assert graph_signature_memo(crow, col, 8, "spmm") == first
    col[0] = 2  # in-place change bumps the version: recomputed
    changed = graph_signature_memo(crow, col, 8, "spmm")
    assert changed == graph_signature(crow, col, 8, "spmm")
    assert changed["structure_hash"] != first["structure_hash"]
    other = col.clone()  # equal content, other object: recomputed, same value
    assert graph_signature_memo(crow, other, 8, "spmm") == changed


def test_schedule_file_memo_sees_external_writes(tmp_path):
    path = tmp_path / "schedules.json"
    ScheduleCache(path).store({"type": "cpu"}, {"rows": 1}, {"choice": "baseline"})
    assert ScheduleCache(path).lookup({"type": "cpu"}, {"rows": 1})["result"] == {"choice": "baseline"}
    payload = json.loads(path.read_text())
    key = next(iter(payload["records"]))
    payload["records"][key]["result"] = {"choice": "autosage", "note": "written by another process"}
    path.write_text(json.dumps(payload, indent=2))
    assert ScheduleCache(path).lookup({"type": "cpu"}, {"rows": 1})["result"]["choice"] == "autosage"
