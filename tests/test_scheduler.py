"""Scheduler configuration and candidate shortlist: the behaviour the
reference's tests/test_scheduler.py pins (valid shortlist, env overrides
read per call, kernel policy in the signature), checked over more inputs,
plus exact-order and decision-rule checks."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from autosage_amd._auto import _degree_quantiles, _induced_sample_csr, _preferred_waves, _spmm_candidates
from autosage_amd.config import SchedulerConfig

GOLDEN = Path(__file__).resolve().parent / "golden"


def _crow_of(degrees) -> torch.Tensor:
    return torch.tensor([0, *np.cumsum(degrees).tolist()], dtype=torch.long)


@pytest.mark.parametrize("degrees", [[1, 2, 0, 7], [0] * 5 + [40], list(range(50)), [3] * 64 + [900, 2000]])
@pytest.mark.parametrize("features", [16, 64, 200])
def test_shortlist_holds_only_runnable_split_settings(degrees, features):
    """Every shortlisted (feature_tile, waves, hub_threshold) is a setting
    the split op accepts, each appears once, and the list never outgrows the
    requested count."""
    crow = _crow_of(degrees)
    for count in (1, 3, 6, 18):
        shortlist = _spmm_candidates(crow, features, SchedulerConfig(candidate_count=count))
        assert 1 <= len(shortlist) <= count
        assert len(set(shortlist)) == len(shortlist)
        for tile, waves, threshold in shortlist:
            assert tile in (64, 128) and waves in (2, 4, 8)
            assert isinstance(threshold, int) and threshold >= 1


def test_kernel_overrides_follow_the_environment_between_calls(monkeypatch):
    """AUTOSAGE_FTILE / WPB / HUB_T are parsed again whenever they change."""
    seen = []
    for tile, waves, threshold in (("128", "2", "5"), ("64", "8", "77"), ("64", "4", "1")):
        monkeypatch.setenv("AUTOSAGE_FTILE", tile)
        monkeypatch.setenv("AUTOSAGE_WPB", waves)
        monkeypatch.setenv("AUTOSAGE_HUB_T", threshold)
        config = SchedulerConfig.from_env()
        seen.append((config.feature_tile, config.warps_per_block, config.hub_threshold))
    assert seen == [(128, 2, 5), (64, 8, 77), (64, 4, 1)]
    # the pinned settings are the only candidate left
    assert _spmm_candidates(_crow_of([4, 9, 2]), 32, SchedulerConfig.from_env()) == [(64, 4, 1)]


@pytest.mark.parametrize("word", ["0", "off", "No", "FALSE"])
def test_vec4_switch_changes_the_signature(monkeypatch, word):
    """The float4 policy decides which kernels run, so a cached choice made
    with it on must not replay with it off."""
    monkeypatch.delenv("AUTOSAGE_VEC4", raising=False)
    default = SchedulerConfig.from_env().tuning_signature()
    monkeypatch.setenv("AUTOSAGE_VEC4", word)
    switched = SchedulerConfig.from_env().tuning_signature()
    assert (default["vec4"], switched["vec4"]) == (True, False)
    assert {k for k in default if default[k] != switched[k]} == {"vec4"}


def test_feature_slices_is_part_of_the_signature(monkeypatch):
    assert SchedulerConfig.from_env().tuning_signature()["feature_slices"] == "auto"
    monkeypatch.setenv("AUTOSAGE_FEATURE_SLICES", " On ")
    assert SchedulerConfig.from_env().feature_slices == "on"
    monkeypatch.setenv("AUTOSAGE_FEATURE_SLICES", "maybe")
    with pytest.raises(ValueError, match="feature_slices"):
        SchedulerConfig.from_env()


def test_exactness_margin_of_the_full_graph_decision():
    """The reassociating column-sliced SpMM wins only when it beats the best
    bit-exact option by more than the margin."""
    from autosage_amd import _auto

    keys = ["null", '"fslice"', '"colslice"']
    inexact = ('"colslice"',)
    margin = _auto._INEXACT_MARGIN
    assert _auto._prefer_exact(keys, {"null": 9.0, '"fslice"': 3.1, '"colslice"': 3.0}, inexact) == '"fslice"'
    fast = 3.1 / (1.0 + margin) - 0.01
    assert _auto._prefer_exact(keys, {"null": 9.0, '"fslice"': 3.1, '"colslice"': fast}, inexact) == '"colslice"'
    assert _auto._prefer_exact(keys, {"null": 2.0, '"fslice"': 3.1, '"colslice"': 3.0}, inexact) == "null"
    # without a bit-exact option the fastest one is taken
    assert _auto._prefer_exact(['"colslice"'], {'"colslice"': 5.0}, inexact) == '"colslice"'
    # and without inexact options the margin plays no part
    assert _auto._prefer_exact(keys, {"null": 3.0, '"fslice"': 3.1, '"colslice"': 2.0}) == '"colslice"'


def test_hub_mode_is_part_of_the_signature(monkeypatch):
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", "split64")
    assert SchedulerConfig.from_env().tuning_signature()["hub_mode"] == "split64"
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", "bogus")
    with pytest.raises(ValueError, match="hub_mode"):
        SchedulerConfig.from_env()


def test_column_slices_is_part_of_the_signature(monkeypatch):
    assert SchedulerConfig.from_env().tuning_signature()["column_slices"] == "auto"
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "OFF")
    assert SchedulerConfig.from_env().tuning_signature()["column_slices"] == "off"
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "sometimes")
    with pytest.raises(ValueError, match="column_slices"):
        SchedulerConfig.from_env()


def test_column_slices_never_eligible_without_the_native_op(monkeypatch):
    from autosage_amd import _auto

    crow = torch.arange(0, 100 * 1000 + 1, 100)
    col = torch.arange(100 * 1000) % 1000
    x = torch.zeros(1000, 10000)  # 40 MB
    monkeypatch.setattr(_auto, "native_op", lambda name: None)
    assert not _auto._colslice_eligible(crow, col, x, SchedulerConfig(column_slices="on"))
    monkeypatch.setattr(_auto, "native_op", lambda name: object())
    assert not _auto._colslice_eligible(crow, col, x, SchedulerConfig(column_slices="off"))
    assert not _auto._colslice_eligible(crow, col, x, SchedulerConfig(full_graph_check=False))
    # auto: too little X or too few edges per row
    assert not _auto._colslice_eligible(crow, col, x[:, :7000], SchedulerConfig())  # 28 MB
    assert not _auto._colslice_eligible(crow, col[: 63 * 1000], x, SchedulerConfig())
    # ... unless a row is long enough to be worth spreading over the slices
    # (the device check of the graph is stubbed out here, on the CPU)
    from autosage_amd import _native

    monkeypatch.setattr(_native, "columns_ascending", lambda crow_, col_: True)
    hub = torch.cat([torch.tensor([0, 2048]), torch.arange(1, 999) + 2048])
    hub_col = torch.arange(hub[-1].item()) % 1000
    small_x = torch.zeros(1000, 128)  # 0.5 MB
    assert _auto._colslice_eligible(hub, hub_col, small_x, SchedulerConfig())
    short = torch.cat([torch.tensor([0, 2047]), torch.arange(1, 999) + 2047])
    assert not _auto._colslice_eligible(short, hub_col[:-1], small_x, SchedulerConfig())


@pytest.mark.parametrize(
    "kwargs, message",
    [
        ({"guardrail": 0.0}, "guardrail"),
        ({"probe_fraction": 1.5}, "probe_fraction"),
        ({"probe_iterations": 0}, "positive"),
        ({"probe_cap_ms": -1.0}, "negative"),
        ({"feature_tile": 32}, "feature_tile"),
        ({"warps_per_block": 3}, "warps_per_block"),
        ({"hub_threshold": 0}, "hub_threshold"),
    ],
)
def test_invalid_configuration_is_rejected(kwargs, message):
    with pytest.raises(ValueError, match=message):
        SchedulerConfig(**kwargs)


def test_bad_boolean_environment_value(monkeypatch):
    monkeypatch.setenv("AUTOSAGE_VEC4", "maybe")
    with pytest.raises(ValueError, match="AUTOSAGE_VEC4 must be a boolean value"):
        SchedulerConfig.from_env()


def test_candidate_order_closed_form():
    # degrees 1, 2, 0, 7: q90/q95/q99 (linear) = 5.5/6.25/6.85 -> 6, 6, 7;
    # F = 64 -> preferred tile 64 and 2 waves; preferred threshold 6.
    crow = torch.tensor([0, 1, 3, 3, 10], dtype=torch.long)
    assert _degree_quantiles(crow) == (6, 6, 7)
    got = _spmm_candidates(crow, 64, SchedulerConfig(candidate_count=18))
    want_tile, want_waves, want_thr = 64, 2, 6

    def dist(c):
        return abs(c[0] - want_tile) / 64 + abs(c[1] - want_waves) / 6 + abs(c[2] - want_thr) / want_thr

    brute = sorted(
        ((t, w, h) for t in (64, 128) for w in (2, 4, 8) for h in (6, 7)), key=lambda c: (dist(c), c)
    )
    assert got == brute
    assert got[0] == (64, 2, 6)
    wide = _spmm_candidates(crow, 256, SchedulerConfig(candidate_count=1))
    assert wide == [(128, 4, 6)]


def _golden():
    path = GOLDEN / "scheduler_golden.json"
    return json.loads(path.read_text())


def test_degree_quantiles_match_reference_golden():
    g = _golden()
    for case in g["quantiles"]:
        crow = torch.tensor(g["graphs"][case["graph"]]["crow"], dtype=torch.long)
        assert list(_degree_quantiles(crow)) == case["expected"], case["name"]


def test_candidates_match_reference_golden():
    """The candidate set equals the reference's; the ranking equals it
    whenever the reference's preferred warp count (8/4/2 by skew) equals the
    MI355X preferred wave count, and differs only through that term."""
    g = _golden()
    checked_order = 0
    for case in g["candidates"]:
        crow = torch.tensor(g["graphs"][case["graph"]]["crow"], dtype=torch.long)
        config = SchedulerConfig(candidate_count=case["k"])
        got = [list(c) for c in _spmm_candidates(crow, case["feature_width"], config)]
        full_got = sorted(map(tuple, _spmm_candidates(crow, case["feature_width"], SchedulerConfig(candidate_count=18))))
        if case["k"] >= 18:
            assert sorted(map(tuple, case["expected"])) == full_got, case["name"]
        deg = (crow[1:] - crow[:-1]).to(torch.float64)
        q50 = int(torch.quantile(deg, 0.5).round().item())
        q99 = _degree_quantiles(crow)[2]
        skew = q99 / max(q50, 1)
        reference_waves = 8 if skew >= 4 else 4 if skew >= 2 else 2
        if reference_waves == _preferred_waves(case["feature_width"]):
            assert got == case["expected"], case["name"]
            checked_order += 1
    assert checked_order >= 1


def test_induced_sample_matches_reference_golden():
    g = _golden()
    for case in g["samples"]:
        gr = g["graphs"][case["graph"]]
        crow = torch.tensor(gr["crow"], dtype=torch.long)
        col = torch.tensor(gr["col"], dtype=torch.long)
        val = torch.tensor(gr["val"], dtype=torch.float32)
        s_crow, s_col, s_val, sel = _induced_sample_csr(
            crow, col, val, fraction=case["fraction"], minimum_rows=case["minimum_rows"], seed=case["seed"]
        )
        exp = case["expected"]
        assert s_crow.tolist() == exp["crow"], case["name"]
        assert s_col.tolist() == exp["col"], case["name"]
        assert sel.tolist() == exp["selected"], case["name"]
        assert torch.equal(s_val, torch.tensor(exp["val"], dtype=torch.float32)), case["name"]


def test_edge_index_to_csr_matches_reference_golden():
    from autosage_amd.utils.csr import edge_index_to_csr

    for case in _golden()["csr"]:
        crow, col = edge_index_to_csr(torch.tensor(case["edge_index"]), case["num_nodes"], rows_by=case["rows_by"])
        assert crow.tolist() == case["expected"]["crow"], case["name"]
        assert col.tolist() == case["expected"]["col"], case["name"]


def test_cpu_row_softmax_matches_reference_golden_bits():
    """The CPU row softmax (torch ops, as the reference composes it) against
    the reference's own output bits.  Those bits depend on the host: torch's
    vectorised exp and reductions differ between CPUs (the GPU box's differ
    from this container's), so every probability must be within 2 units in
    the last place of the golden one."""
    import numpy as np

    from autosage_amd._auto import _csr_row_softmax

    g = _golden()
    for case in g["softmax"]:
        gr = g["graphs"][case["graph"]]
        crow = torch.tensor(gr["crow"], dtype=torch.long)
        scores = torch.tensor(gr["scores"], dtype=torch.float32)
        bits = _csr_row_softmax(crow, scores).numpy().view(np.uint32).astype(np.int64)
        want = np.asarray(case["expected_bits"], dtype=np.int64)
        # probabilities are non-negative, so bit patterns order like values
        assert np.max(np.abs(bits - want)) <= 2, case["name"]
