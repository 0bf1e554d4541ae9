"""Scheduler configuration (mirrors ``autosage/config.py:8-102``).

The fields, defaults, validation messages, environment variables and the
``tuning_signature`` of the reference are kept, because the signature is part
of cache validity (``_auto.py:219-224``).  One field is added: ``hub_mode``
(``AUTOSAGE_HUB_MODE`` = ``exact`` | ``split64``), the hub-row strategy of the
gfx950 split kernel, which changes results' rounding and therefore belongs in
the signature.  ``full_graph_check`` (``AUTOSAGE_FULL_CHECK``) makes a sampled
"autosage" decision confirm itself once on the full graph against the
PyTorch-ROCm baseline before it is cached.  ``column_slices``
(``AUTOSAGE_COLUMN_SLICES`` = ``auto`` | ``on`` | ``off``) controls the
column-sliced SpMM (one column slice per XCD, fp64 accumulation): ``auto``
times it on the full graph when the graph is large enough to profit, ``on``
times it on every graph with ascending columns, ``off`` never uses it, which
keeps SpMM results bit-identical to the sequential CSR product.
``feature_slices`` (``AUTOSAGE_FEATURE_SLICES`` = ``auto`` | ``on`` | ``off``)
controls the feature-sliced SpMM (32-feature slices of X per XCD, CSR-order
fp32 chains, bit-identical to the sequential CSR product): ``auto`` times it
on the full graph when the graph is large enough to profit, ``on`` on every
graph, ``off`` never.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from . import _env


def _optional_int(name: str) -> Optional[int]:
    raw = _env.get(name)
    return None if raw in (None, "") else int(raw)


def _boolean(name: str, default: bool) -> bool:
    raw = _env.get(name)
    if raw is None:
        return default
    word = raw.strip().lower()
    if word in ("1", "true", "yes", "on"):
        return True
    if word in ("0", "false", "no", "off"):
        return False
    raise ValueError(f"{name} must be a boolean value")


@dataclass(frozen=True)
class SchedulerConfig:
    guardrail: float = 0.95
    probe_fraction: float = 0.03
    probe_min_rows: int = 512
    probe_iterations: int = 7
    probe_cap_ms: float = 1.0
    minimum_probe_rows: int = 64
    minimum_probe_nonzeros: int = 512
    candidate_count: int = 6
    hub_split: bool = True
    vec4: bool = True
    cache: bool = True
    replay_only: bool = False
    feature_tile: Optional[int] = None
    warps_per_block: Optional[int] = None
    hub_threshold: Optional[int] = None
    hub_mode: str = "exact"
    full_graph_check: bool = True
    column_slices: str = "auto"
    feature_slices: str = "auto"

    def __post_init__(self) -> None:
        if not 0 < self.guardrail <= 1:
            raise ValueError("guardrail must be in (0, 1]")
        if not 0 < self.probe_fraction <= 1:
            raise ValueError("probe_fraction must be in (0, 1]")
        if min(self.probe_min_rows, self.probe_iterations, self.candidate_count) < 1:
            raise ValueError("probe row, iteration, and candidate counts must be positive")
        if self.probe_cap_ms < 0:
            raise ValueError("probe_cap_ms cannot be negative")
        if self.feature_tile not in (None, 64, 128):
            raise ValueError("feature_tile must be 64 or 128")
        if self.warps_per_block not in (None, 2, 4, 8):
            raise ValueError("warps_per_block must be 2, 4, or 8")
        if self.hub_threshold is not None and self.hub_threshold < 1:
            raise ValueError("hub_threshold must be positive")
        if self.hub_mode not in ("exact", "split64"):
            raise ValueError("hub_mode must be 'exact' or 'split64'")
        if self.column_slices not in ("auto", "on", "off"):
            raise ValueError("column_slices must be 'auto', 'on' or 'off'")
        if self.feature_slices not in ("auto", "on", "off"):
            raise ValueError("feature_slices must be 'auto', 'on' or 'off'")

    def tuning_signature(self) -> dict[str, object]:
        return {
            "guardrail": self.guardrail,
            "probe_fraction": self.probe_fraction,
            "probe_min_rows": self.probe_min_rows,
            "probe_iterations": self.probe_iterations,
            "probe_cap_ms": self.probe_cap_ms,
            "minimum_probe_rows": self.minimum_probe_rows,
            "minimum_probe_nonzeros": self.minimum_probe_nonzeros,
            "candidate_count": self.candidate_count,
            "hub_split": self.hub_split,
            "vec4": self.vec4,
            "feature_tile": self.feature_tile,
            "warps_per_block": self.warps_per_block,
            "hub_threshold": self.hub_threshold,
            "hub_mode": self.hub_mode,
            "full_graph_check": self.full_graph_check,
            "column_slices": self.column_slices,
            "feature_slices": self.feature_slices,
        }

    @classmethod
    def from_env(cls, *, guardrail: float = 0.95, candidate_count: int = 6) -> "SchedulerConfig":
        """The configuration the environment gives now (read on every call,
        as the reference does); the parsed value is memoised per set of raw
        environment values, so an unchanged environment costs twenty dict
        lookups.  Invalid values raise on every call."""
        key = (_env.raw(_ENV_NAMES), float(guardrail), int(candidate_count))
        config = _FROM_ENV_MEMO.get(key)
        if config is None:
            config = cls._parse_env(guardrail, candidate_count)
            if len(_FROM_ENV_MEMO) > 64:
                _FROM_ENV_MEMO.clear()
            _FROM_ENV_MEMO[key] = config
        return config

    @classmethod
    def _parse_env(cls, guardrail: float, candidate_count: int) -> "SchedulerConfig":
        env = _env.get
        return cls(
            guardrail=float(guardrail),
            probe_fraction=float(env("AUTOSAGE_PROBE_FRAC", "0.03")),
            probe_min_rows=int(env("AUTOSAGE_PROBE_MIN_ROWS", "512")),
            probe_iterations=int(env("AUTOSAGE_PROBE_ITERS", "7")),
            probe_cap_ms=float(env("AUTOSAGE_PROBE_CAP_MS", "1.0")),
            minimum_probe_rows=int(env("AUTOSAGE_MIN_PROBE_ROWS", "64")),
            minimum_probe_nonzeros=int(env("AUTOSAGE_MIN_PROBE_NNZ", "512")),
            candidate_count=int(candidate_count),
            hub_split=_boolean("AUTOSAGE_HUB_CTA", True),
            vec4=_boolean("AUTOSAGE_VEC4", True),
            cache=_boolean("AUTOSAGE_CACHE", True),
            replay_only=_boolean("AUTOSAGE_REPLAY_ONLY", False),
            feature_tile=_optional_int("AUTOSAGE_FTILE"),
            warps_per_block=_optional_int("AUTOSAGE_WPB"),
            hub_threshold=_optional_int("AUTOSAGE_HUB_T"),
            hub_mode=(env("AUTOSAGE_HUB_MODE") or "exact").strip().lower(),
            full_graph_check=_boolean("AUTOSAGE_FULL_CHECK", True),
            column_slices=(env("AUTOSAGE_COLUMN_SLICES") or "auto").strip().lower(),
            feature_slices=(env("AUTOSAGE_FEATURE_SLICES") or "auto").strip().lower(),
        )


# Every environment variable from_env reads.
_ENV_NAMES = (
    "AUTOSAGE_PROBE_FRAC", "AUTOSAGE_PROBE_MIN_ROWS", "AUTOSAGE_PROBE_ITERS", "AUTOSAGE_PROBE_CAP_MS",
    "AUTOSAGE_MIN_PROBE_ROWS", "AUTOSAGE_MIN_PROBE_NNZ", "AUTOSAGE_HUB_CTA", "AUTOSAGE_VEC4", "AUTOSAGE_CACHE",
    "AUTOSAGE_REPLAY_ONLY", "AUTOSAGE_FTILE", "AUTOSAGE_WPB", "AUTOSAGE_HUB_T", "AUTOSAGE_HUB_MODE",
    "AUTOSAGE_FULL_CHECK", "AUTOSAGE_COLUMN_SLICES", "AUTOSAGE_FEATURE_SLICES",
)
_FROM_ENV_MEMO: dict = {}
