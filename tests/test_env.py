"""The per-call environment reader and the memoised scheduler configuration
keep the semantics of reading ``os.environ`` on every call."""

from __future__ import annotations

import os

import pytest

from autosage_amd import _env
from autosage_amd.config import SchedulerConfig


def test_get_follows_os_environ(monkeypatch):
    name = "AUTOSAGE_TEST_ENV_READER"
    monkeypatch.delenv(name, raising=False)
    assert _env.get(name) is None and _env.get(name, "d") == "d"
    for value in ("1", "", "  off ", "ünïcödé", "1"):
        monkeypatch.setenv(name, value)
        assert _env.get(name) == os.environ.get(name) == value
    monkeypatch.delenv(name)
    assert _env.get(name, "gone") == "gone"
    # raw values key memos: equal exactly when the values are
    monkeypatch.setenv(name, "a")
    first = _env.raw((name, "PATH"))
    assert first == _env.raw((name, "PATH"))
    monkeypatch.setenv(name, "b")
    assert _env.raw((name, "PATH")) != first
    monkeypatch.delenv(name)
    assert _env.raw((name,)) == (None,)


def test_from_env_sees_every_change(monkeypatch):
    for var in ("AUTOSAGE_PROBE_FRAC", "AUTOSAGE_HUB_MODE", "AUTOSAGE_COLUMN_SLICES", "AUTOSAGE_CACHE"):
        monkeypatch.delenv(var, raising=False)
    base = SchedulerConfig.from_env()
    assert base == SchedulerConfig()
    assert SchedulerConfig.from_env() is base  # memoised while the environment is unchanged
    monkeypatch.setenv("AUTOSAGE_PROBE_FRAC", "0.05")
    monkeypatch.setenv("AUTOSAGE_HUB_MODE", " Split64 ")
    monkeypatch.setenv("AUTOSAGE_COLUMN_SLICES", "off")
    changed = SchedulerConfig.from_env(guardrail=0.9, candidate_count=3)
    assert (changed.probe_fraction, changed.hub_mode, changed.column_slices) == (0.05, "split64", "off")
    assert (changed.guardrail, changed.candidate_count) == (0.9, 3)
    assert changed.tuning_signature() != base.tuning_signature()
    # invalid values raise on every call, not only the first
    monkeypatch.setenv("AUTOSAGE_CACHE", "maybe")
    for _ in range(2):
        with pytest.raises(ValueError, match="AUTOSAGE_CACHE must be a boolean value"):
            SchedulerConfig.from_env()
    monkeypatch.delenv("AUTOSAGE_CACHE")
    for var in ("AUTOSAGE_PROBE_FRAC", "AUTOSAGE_HUB_MODE", "AUTOSAGE_COLUMN_SLICES"):
        monkeypatch.delenv(var)
    assert SchedulerConfig.from_env() == base
