"""Input-aware scheduling of the sparse kernels.

Behaviour follows ``autosage/_auto.py`` of the reference: the same public
functions and private helpers, the same sampling, shortlist, probing,
guardrail, cache replay and result dictionaries (``:266-441``, ``:544-741``),
so cached schedules and telemetry read the same.  The SpMM and SDDMM
schedulers share one probe engine here (``_probe_and_choose``).

gfx950 changes:
* candidates keep the reference's ``[tile, warps, threshold]`` shape; on
  MI355X ``tile`` is the light-row features per pass, ``warps`` the waves per
  hub workgroup and ``threshold`` the hub degree;
* a sampled "autosage" decision is confirmed once on the full graph against
  the PyTorch-ROCm baseline (``SchedulerConfig.full_graph_check``) before it is
  cached, so a replayed schedule is never slower than the baseline on the
  graph it was made for;
* the CSR row softmax and the attention pipeline run as native kernels on the
  GPU (``csr_attention_forward`` can fuse all three stages into one launch).
"""

from __future__ import annotations

import json
import os
import statistics
import time
from typing import Any, Callable, Optional

import torch

from . import _env
from ._cache import cached_result, ScheduleCache, device_signature, graph_signature_memo, log_probe
from .config import SchedulerConfig
from .ops import _normalize_csr, load_native, native_load_error, native_op, spmm_csr, validate_if_requested

AUTOTUNE_SCHEMA_VERSION = 3


def _time_cuda(
    function: Callable[[], torch.Tensor],
    *,
    warmup: int,
    iterations: int,
    cap_ms: Optional[float] = None,
) -> dict[str, Any]:
    """Event timing of ``_auto.py:18-54``: warmups, then per-iteration events
    with a sync, stopping early once ``cap_ms`` of kernel time is spent."""
    torch.cuda.synchronize()
    wall_start = time.perf_counter()
    for _ in range(max(0, warmup)):
        function()
    torch.cuda.synchronize()
    samples: list[float] = []
    output = None
    spent = 0.0
    for _ in range(max(1, iterations)):
        begin = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        begin.record()
        output = function()
        end.record()
        end.synchronize()
        elapsed = float(begin.elapsed_time(end))
        samples.append(elapsed)
        spent += elapsed
        if cap_ms is not None and spent >= max(0.0, cap_ms):
            break
    torch.cuda.synchronize()
    return {
        "best_ms": min(samples),
        "mean_ms": statistics.fmean(samples),
        "std_ms": statistics.pstdev(samples) if len(samples) > 1 else 0.0,
        "iterations": len(samples),
        "total_ms": spent,
        "wall_ms": (time.perf_counter() - wall_start) * 1000.0,
        "output": output,
    }


def _prepare_spmm_baseline(crow, col, val, x) -> tuple[Callable[[], torch.Tensor], str]:
    """PyTorch CSR SpMM (hipSPARSE on ROCm), ``_auto.py:57-76``.

    On PyTorch-ROCm, ``torch.sparse.mm`` on a bf16 CSR tensor on the GPU
    aborts the whole process inside the sparse library (no Python exception
    can be caught), and fp16 goes through the same library path.  For those
    feature types this raises ``RuntimeError`` before building the matrix;
    the schedulers time the native 16-bit kernels instead."""
    if x.is_cuda and x.dtype in _DTYPES_16:
        raise RuntimeError(
            f"torch.sparse.mm has no usable {x.dtype} CSR kernel on PyTorch-ROCm (the call aborts the process); "
            "use the native 16-bit SpMM (torch.ops.autosage.spmm_csr) instead"
        )
    weights = torch.ones(col.numel(), device=x.device, dtype=x.dtype) if val is None else val
    matrix = torch.sparse_csr_tensor(
        crow, col, weights.to(dtype=x.dtype), size=(crow.numel() - 1, x.size(0)), device=x.device, dtype=x.dtype
    )
    return (lambda: torch.sparse.mm(matrix, x)), "torch.sparse.mm(csr)"


def _edge_rows(crow: torch.Tensor) -> torch.Tensor:
    counts = (crow[1:] - crow[:-1]).to(torch.long)
    return torch.repeat_interleave(torch.arange(crow.numel() - 1, device=crow.device, dtype=torch.long), counts)


def _prepare_sddmm_baseline(crow, col, query, key) -> tuple[Callable[[], torch.Tensor], str]:
    """Gather-dot baseline, ``_auto.py:79-92``."""
    rows = _edge_rows(crow)
    return (lambda: (query.index_select(0, rows) * key.index_select(0, col)).sum(dim=1)), "gather-dot"


def _induced_sample_csr(crow, col, val, *, fraction: float, minimum_rows: int, seed: int):
    """Induced sub-graph on a seeded row sample (``_auto.py:95-154``): rows
    ``randperm(N)[:S]`` sorted, S = min(max(int(N·fraction), minimum_rows, 1), N);
    an edge survives when its column is also sampled; columns are renumbered.
    On the GPU the sub-graph comes from the native sampler; on the CPU from
    the reference's torch composition (same outputs)."""
    rows = crow.numel() - 1
    size = min(max(int(rows * fraction), minimum_rows, 1), rows)
    device = crow.device
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    selected = torch.randperm(rows, generator=generator, device=device)[:size].sort().values

    if crow.is_cuda and native_op("spmm_csr") is not None and (val is None or val.dtype == torch.float32):
        # the same sub-graph from two native passes (one host sync)
        from ._native import induced_sample

        new_crow, new_col, new_val = induced_sample(crow, col, val, selected)
        return new_crow, new_col, new_val, selected
    return (*_induced_subgraph_torch(crow, col, val, selected), selected)


def _induced_subgraph_torch(crow, col, val, selected):
    """The sub-graph induced by the sorted row sample ``selected``, as the
    reference's torch composition (``_auto.py:114-154``)."""
    rows = crow.numel() - 1
    size = selected.numel()
    device = crow.device
    remap = torch.full((rows,), -1, dtype=torch.long, device=device)
    remap[selected] = torch.arange(size, device=device)
    starts = crow.index_select(0, selected)
    counts = crow.index_select(0, selected + 1) - starts
    total = int(counts.sum().item())
    if total == 0:
        empty_val = None if val is None else torch.empty(0, dtype=val.dtype, device=val.device)
        return (
            torch.zeros(size + 1, dtype=torch.long, device=device),
            torch.empty(0, dtype=torch.long, device=col.device),
            empty_val,
        )
    owner = torch.repeat_interleave(torch.arange(size, device=device, dtype=torch.long), counts)
    first = torch.repeat_interleave(torch.cumsum(counts, dim=0) - counts, counts)
    positions = starts.index_select(0, owner) + torch.arange(total, device=device, dtype=torch.long) - first
    mapped = remap.index_select(0, col.index_select(0, positions))
    keep = mapped.ge(0)
    kept_counts = torch.bincount(owner[keep], minlength=size)
    new_crow = torch.cat((torch.zeros(1, dtype=torch.long, device=device), kept_counts.cumsum(0)))
    new_col = mapped[keep].contiguous()
    new_val = None if val is None else val.index_select(0, positions)[keep].contiguous()
    return new_crow, new_col, new_val


def _quantile_ints(degrees: torch.Tensor, points: list[float]) -> list[int]:
    q = torch.tensor(points, dtype=torch.float64, device=degrees.device)
    return torch.quantile(degrees.to(torch.float64), q).round().clamp_min(1).to(torch.long).cpu().tolist()


def _degree_quantiles(crow: torch.Tensor) -> tuple[int, int, int]:
    """Rounded q90/q95/q99 of the row degrees, at least 1 (``_auto.py:157-172``)."""
    degrees = crow[1:] - crow[:-1]
    if degrees.numel() == 0:
        return 1, 1, 1
    q90, q95, q99 = _quantile_ints(degrees, [0.9, 0.95, 0.99])
    return int(q90), int(q95), int(q99)


def _preferred_waves(feature_width: int) -> int:
    """Waves per hub workgroup to rank first.

    The reference prefers 8/4/2 warps for degree skew q99/q50 >= 4 / >= 2 /
    otherwise (``_auto.py:187-188``), because its warps split a hub row's
    edges.  Here the waves of a hub workgroup split the row's features (the
    sum keeps its order), and a slice narrower than 64 features leaves lanes
    idle: on the skewed 115M-nnz graph 2 waves beat 4 and 8 at F = 64, 128
    and 256 (6.29 / 8.19 / 13.7 ms at F = 128).  Two waves are preferred up
    to F = 128, four above."""
    return 2 if feature_width <= 128 else 4


def _spmm_candidates(crow: torch.Tensor, feature_width: int, config: SchedulerConfig) -> list[tuple[int, int, int]]:
    """Shortlist of ``(tile, waves, threshold)`` (``_auto.py:175-216``).

    The preferred point is tile 64 for F <= 64 else 128, the waves of
    ``_preferred_waves`` and threshold q95; candidates are ranked by
    |Δtile|/64 + |Δwaves|/6 + |Δthreshold|/threshold, ties broken by the
    tuple, and the first ``candidate_count`` are kept."""
    q90, q95, q99 = _degree_quantiles(crow)
    want_waves = _preferred_waves(feature_width)
    want_tile = 64 if feature_width <= 64 else 128
    want_threshold = q95

    tiles = [config.feature_tile] if config.feature_tile is not None else [64, 128]
    waves = [config.warps_per_block] if config.warps_per_block is not None else [2, 4, 8]
    thresholds = [config.hub_threshold] if config.hub_threshold is not None else list(dict.fromkeys((q95, q90, q99)))

    def rank(candidate: tuple[int, int, int]):
        tile, wave_count, threshold = candidate
        distance = abs(tile - want_tile) / 64 + abs(wave_count - want_waves) / 6
        distance += abs(threshold - want_threshold) / max(want_threshold, 1)
        return distance, candidate

    pool = {(int(t), int(w), max(1, int(h))) for t in tiles for w in waves for h in thresholds}
    return sorted(pool, key=rank)[: max(1, config.candidate_count)]


COLSLICE = "colslice"  # candidate value of the column-sliced SpMM
FSLICE = "fslice"  # candidate value of the feature-sliced SpMM (bit-exact)
# The column-sliced SpMM reassociates each row's sum (fp64 partials, one
# rounding); the other native schedules keep the reference's CSR-order fp32
# chain.  The full-graph decision takes the column-sliced one only when it
# beats the best bit-exact option by more than this fraction.
_INEXACT_MARGIN = 0.05
ROUNDED16 = "rounded16"  # candidate value of the bf16 / fp16 SpMM (column slices when the columns ascend)
ROUNDED16_EDGES = "rounded16:edges"  # the same product with edge slices
ROUNDED16_ROWS = "rounded16:rows"  # the same product, every row whole (one launch)
_ROUNDED16_ALL = (ROUNDED16, ROUNDED16_EDGES, ROUNDED16_ROWS)
_DTYPES_16 = (torch.bfloat16, torch.float16)
# Column slicing pays when X is beyond the 8 x 4 MB of L2 and rows are long
# enough that the per-(row, slice) fp64 partials (128·F bytes per row,
# written and read) stay small next to the gathers (4·F bytes per edge).
_COLSLICE_MIN_X_BYTES = 32 << 20
_COLSLICE_MIN_MEAN_DEGREE = 64
# It also pays on any graph with a row this long: the exact schedules walk a
# row's edges in order on one wave, the sliced one spreads them over 8 (on
# the reference's hub-sweep graph, one 12,000-edge row among 20,000 rows of
# 32, 0.18 ms against 0.45 ms for the best exact split at F = 128).
_COLSLICE_HUB_DEGREE = 2048


def _colslice_eligible(crow, col, x, config: SchedulerConfig) -> bool:
    """Whether the full-graph check should time the column-sliced SpMM."""
    if config.column_slices == "off" or not config.full_graph_check or native_op("spmm_csr_colslice") is None:
        return False
    n = crow.numel() - 1
    if n <= 0 or col.numel() == 0:
        return False
    from ._native import columns_ascending, row_counts

    if config.column_slices == "auto":
        large = x.numel() * x.element_size() >= _COLSLICE_MIN_X_BYTES and col.numel() >= _COLSLICE_MIN_MEAN_DEGREE * n
        if not large and row_counts(crow, _COLSLICE_HUB_DEGREE, 0)[0] == 0:
            return False

    # checks the graph once (a malformed one raises); a graph whose columns
    # do not ascend is eligible too: the op runs on its row-sorted copy
    columns_ascending(crow, col)
    return True


def _fslice_eligible(crow, col, x, config: SchedulerConfig) -> bool:
    """Whether the full-graph check should time the feature-sliced SpMM."""
    return config.full_graph_check and fslice_suits(crow, col, x, config.feature_slices)


def fslice_suits(crow, col, x, mode: str) -> bool:
    """Whether the feature-sliced SpMM is worth running for this graph and X:
    graphs whose X is beyond the L2s with long rows on average, or with a
    hub row (``auto``); every graph with edges (``on``); never (``off``)."""
    if mode == "off" or native_op("spmm_csr_fslice") is None:
        return False
    n = crow.numel() - 1
    if n <= 0 or col.numel() == 0 or x.size(1) == 0:
        return False
    if mode == "auto":
        from ._native import row_counts

        large = x.numel() * x.element_size() >= _COLSLICE_MIN_X_BYTES and col.numel() >= _COLSLICE_MIN_MEAN_DEGREE * n
        if not large and row_counts(crow, _COLSLICE_HUB_DEGREE, 0)[0] == 0:
            return False
    return True


def _require_native() -> None:
    """CUDA inputs run on the HIP library: without it the schedulers raise
    instead of quietly running the PyTorch baseline."""
    if not load_native():
        raise RuntimeError(f"AutoSAGE HIP library is unavailable: {native_load_error()}")


def _cache_hit_allowed(result: dict[str, Any], config: SchedulerConfig) -> bool:
    if result.get("schema_version") != AUTOTUNE_SCHEMA_VERSION:
        return False
    return True if config.replay_only else result.get("configuration") == config.tuning_signature()


def _cached_native_available(operation: str, choice: str, candidate) -> bool:
    if choice != "autosage":
        return True
    if candidate in _ROUNDED16_ALL:
        return native_op(operation) is not None
    if candidate == COLSLICE:
        return native_op(operation + "_colslice") is not None
    if candidate == FSLICE:
        return native_op(operation + "_fslice") is not None
    return native_op(operation + ("_split" if candidate is not None else "")) is not None


def _cached_record(crow, col, width: int, operation: str, config: SchedulerConfig, *, weighted: bool = False,
                   dtype=None) -> Optional[dict[str, Any]]:
    """The cached result for this device, graph, width, operation and
    configuration (``_auto.py:291-300`` of the reference: device and graph
    signatures, canonical-JSON key, schema and tuning-signature check), or
    None.  Memoised per live, unmodified (crow, col) pair while the schedule
    file is unchanged, so a repeated call skips the signatures and the key."""

    def lookup(cache: ScheduleCache) -> Optional[dict[str, Any]]:
        device = device_signature()
        graph = graph_signature_memo(crow, col, width, operation, weighted=weighted, dtype=dtype)
        record = cache.lookup(device, graph)
        if record is None or not _cache_hit_allowed(record.get("result", {}), config):
            return None
        return record["result"]

    extra = (operation, int(width), bool(weighted), str(dtype), config, torch.cuda.current_device())
    return cached_result(crow, col, extra, lookup)


def _cpu_info(operation: str) -> dict[str, Any]:
    return {
        "operation": operation,
        "schema_version": AUTOTUNE_SCHEMA_VERSION,
        "choice": "baseline",
        "baseline": "torch CPU",
        "from_cache": False,
        "reason": "AutoSAGE scheduling is CUDA-only",
    }


def _op_call(name: str, args: tuple, differentiable: tuple):
    """``torch.ops.autosage.<name>(*args)``, or None when the ops are not
    registered.  With nothing for autograd to record (grad mode off, or no
    tensor of ``differentiable`` requiring grad) the op's CUDA implementation
    is called directly: the function the op dispatches to, without the
    autograd wrapper and the dispatcher (~4 us a call)."""
    op = native_op(name)
    if op is None:
        return None
    if not torch.is_grad_enabled() or not any(t is not None and t.requires_grad for t in differentiable):
        from ._native import implementation

        return implementation(name)(*args)
    return op(*args)


def _run_spmm_choice(choice, candidate, crow, col, val, x) -> torch.Tensor:
    if choice == "autosage" and candidate in _ROUNDED16_ALL:
        from ._native import columns_ascending, spmm_rounded_16_impl, spmm_rows_16_impl

        if candidate == ROUNDED16_ROWS:
            return spmm_rows_16_impl(crow, col, val, x)
        # column slices need ascending columns (a cached choice may meet
        # another graph with the same key); every schedule gives the same bits
        columns = candidate == ROUNDED16 and columns_ascending(crow, col)
        return spmm_rounded_16_impl(crow, col, val, x, column_slices=columns)
    if choice == "autosage" and candidate == COLSLICE:
        # any column order: a graph whose columns do not ascend runs on its
        # row-sorted copy, made once per graph
        out = _op_call("spmm_csr_colslice", (crow, col, val, x), (val, x))
        if out is None:
            raise RuntimeError("native operator autosage::spmm_csr_colslice is not registered")
        return out
    if choice == "autosage" and candidate == FSLICE:
        out = _op_call("spmm_csr_fslice", (crow, col, val, x), (val, x))
        if out is None:
            raise RuntimeError("native operator autosage::spmm_csr_fslice is not registered")
        return out
    if choice == "autosage":
        out = None
        if candidate is not None:
            out = _op_call("spmm_csr_split", (crow, col, val, x, *map(int, candidate)), (val, x))
        if out is None:
            out = _op_call("spmm_csr", (crow, col, val, x), (val, x))
        if out is not None:
            return out
    baseline, _ = _prepare_spmm_baseline(crow, col, val, x)
    return baseline()


def _run_sddmm_choice(choice, candidate, crow, col, query, key) -> torch.Tensor:
    if choice == "autosage":
        out = None
        if candidate is not None:
            out = _op_call("sddmm_csr_split", (crow, col, query, key, *map(int, candidate)), (query, key))
        if out is None:
            out = _op_call("sddmm_csr", (crow, col, query, key), (query, key))
        if out is not None:
            return out
    baseline, _ = _prepare_sddmm_baseline(crow, col, query, key)
    return baseline()


def _strip_output(timing: dict[str, Any]) -> dict[str, Any]:
    return {k: v for k, v in timing.items() if k != "output"}


def _probe_and_choose(
    *,
    operation: str,
    config: SchedulerConfig,
    sampled_crow: torch.Tensor,
    sampled_col: torch.Tensor,
    baseline: Callable[[], torch.Tensor],
    split_calls: list[tuple[list[int], Callable[[], torch.Tensor]]],
    core_call: Optional[Callable[[], torch.Tensor]],
) -> dict[str, Any]:
    """Probe loop shared by SpMM and SDDMM (``_auto.py:338-401``, ``:632-704``):
    the baseline, then the shortlisted split candidates while the probe budget
    lasts (the first always runs), or the core kernel when no split op exists;
    the guardrail picks the native variant only with enough sampled work and
    ``best <= guardrail · baseline``."""
    baseline_timing = _time_cuda(baseline, warmup=1, iterations=config.probe_iterations)
    timings: list[dict[str, Any]] = []
    chosen: Optional[list[int]] = None
    best = float("inf")
    budget = config.probe_cap_ms
    if split_calls:
        for index, (candidate, call) in enumerate(split_calls):
            if index > 0 and budget <= 0.0:
                break
            timing = _time_cuda(call, warmup=1, iterations=config.probe_iterations, cap_ms=max(0.0, budget))
            budget = max(0.0, budget - timing["total_ms"])
            timings.append({"candidate": list(candidate), **_strip_output(timing)})
            if timing["best_ms"] < best:
                best = timing["best_ms"]
                chosen = list(candidate)
    elif core_call is not None:
        timing = _time_cuda(core_call, warmup=1, iterations=config.probe_iterations, cap_ms=config.probe_cap_ms)
        best = timing["best_ms"]
        timings.append({"candidate": None, **_strip_output(timing)})
    enough = (
        sampled_crow.numel() - 1 >= config.minimum_probe_rows and sampled_col.numel() >= config.minimum_probe_nonzeros
    )
    use_native = enough and best <= config.guardrail * baseline_timing["best_ms"]
    return {
        "baseline_timing": baseline_timing,
        "timings": timings,
        "chosen": chosen,
        "best": best,
        "use_native": use_native,
    }


def _result_dict(operation, config, probe, baseline_name, sampled_crow, sampled_col, sample_ms) -> dict[str, Any]:
    baseline_best = probe["baseline_timing"]["best_ms"]
    best = probe["best"]
    choice = "autosage" if probe["use_native"] else "baseline"
    return {
        "operation": operation,
        "schema_version": AUTOTUNE_SCHEMA_VERSION,
        "choice": choice,
        "candidate": probe["chosen"] if probe["use_native"] else None,
        "baseline": baseline_name,
        "guardrail": config.guardrail,
        "configuration": config.tuning_signature(),
        "probe_rows": int(sampled_crow.numel() - 1),
        "probe_nonzeros": int(sampled_col.numel()),
        "sampling_ms": sample_ms,
        "probe_ms": sample_ms
        + probe["baseline_timing"]["wall_ms"]
        + sum(entry["wall_ms"] for entry in probe["timings"]),
        "baseline_probe_ms": baseline_best,
        "autosage_probe_ms": None if best == float("inf") else best,
        "sampled_speedup": baseline_best / best if best not in (0.0, float("inf")) else None,
        "candidates": probe["timings"],
        "from_cache": False,
    }


def _replay_miss(operation: str, baseline_name: str) -> dict[str, Any]:
    return {
        "operation": operation,
        "schema_version": AUTOTUNE_SCHEMA_VERSION,
        "choice": "baseline",
        "baseline": baseline_name,
        "from_cache": False,
        "replay_only": True,
        "reason": "cache miss",
    }


def _verbose(tag: str, result: dict[str, Any], verbose: bool) -> None:
    if verbose or _env.get("AUTOSAGE_VERBOSE") == "1":
        print(
            f"[autosage:{tag}] rows={result['probe_rows']} nnz={result['probe_nonzeros']} "
            f"baseline={result['baseline_probe_ms']} ms auto={result['autosage_probe_ms']} "
            f"choice={result['choice']}"
        )


def spmm_csr_auto(
    crow: torch.Tensor,
    col: torch.Tensor,
    val: Optional[torch.Tensor],
    x: torch.Tensor,
    *,
    guardrail: float = 0.95,
    k: int = 6,
    seed: int = 0,
    verbose: bool = False,
) -> tuple[torch.Tensor, dict[str, Any]]:
    crow, col, val, x = _normalize_csr(crow, col, val, x)
    if not x.is_cuda:
        return spmm_csr(crow, col, val, x), _cpu_info("spmm")
    if x.dtype in _DTYPES_16:
        _require_native()
        return _spmm_auto_16(crow, col, val, x, SchedulerConfig.from_env(guardrail=guardrail, candidate_count=k),
                             verbose)
    if x.dtype != torch.float32:
        run, name = _prepare_spmm_baseline(crow, col, val, x)
        return run(), {**_cpu_info("spmm"), "baseline": name, "reason": "AutoSAGE CUDA kernels require float32 features"}

    _require_native()
    config = SchedulerConfig.from_env(guardrail=guardrail, candidate_count=k)
    if config.cache:
        result = _cached_record(crow, col, x.size(1), "spmm", config, weighted=val is not None, dtype=x.dtype)
        if result is not None:
            choice, candidate = result.get("choice", "baseline"), result.get("candidate")
            if _cached_native_available("spmm_csr", choice, candidate):
                return _run_spmm_choice(choice, candidate, crow, col, val, x), {**result, "from_cache": True}
    if config.replay_only:
        return _run_spmm_choice("baseline", None, crow, col, val, x), _replay_miss("spmm", "torch.sparse.mm(csr)")
    device = device_signature()
    graph = graph_signature_memo(crow, col, x.size(1), "spmm", weighted=val is not None, dtype=x.dtype)
    cache = ScheduleCache()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s_crow, s_col, s_val, selected = _induced_sample_csr(
        crow, col, val, fraction=config.probe_fraction, minimum_rows=config.probe_min_rows, seed=seed
    )
    s_x = x.index_select(0, selected).contiguous()
    torch.cuda.synchronize()
    sample_ms = (time.perf_counter() - t0) * 1000.0

    baseline, baseline_name = _prepare_spmm_baseline(s_crow, s_col, s_val, s_x)
    split = native_op("spmm_csr_split") if config.hub_split else None
    core = native_op("spmm_csr")
    split_calls = []
    if split is not None:
        for tile, waves, threshold in _spmm_candidates(s_crow, x.size(1), config):
            split_calls.append(
                ([tile, waves, threshold], lambda t=tile, w=waves, h=threshold: split(s_crow, s_col, s_val, s_x, t, w, h))
            )
    core_call = (lambda: core(s_crow, s_col, s_val, s_x)) if (split is None and core is not None) else None
    probe = _probe_and_choose(
        operation="spmm",
        config=config,
        sampled_crow=s_crow,
        sampled_col=s_col,
        baseline=baseline,
        split_calls=split_calls,
        core_call=core_call,
    )
    result = _result_dict("spmm", config, probe, baseline_name, s_crow, s_col, sample_ms)
    if config.full_graph_check:
        colslice = _colslice_eligible(crow, col, x, config)
        fslice = _fslice_eligible(crow, col, x, config)
        _confirm_spmm_on_full_graph(result, colslice, config, probe, crow, col, val, x, fslice=fslice)
    output = _run_spmm_choice(result["choice"], result["candidate"], crow, col, val, x)
    if config.cache:
        cache.store(device, graph, result)
    log_probe({"timestamp": time.time(), "device": device, "graph": graph, "result": result})
    _verbose("spmm", result, verbose)
    return output, result


# torch.sparse.mm on a bf16 CSR tensor aborts the process on PyTorch-ROCm
# 2.10 (inside the sparse library, uncatchable from Python); fp16 is not
# called for the same reason.  The 16-bit scheduler therefore never runs it.
_BASELINE_16_NOTE = "torch.sparse.mm on bf16/fp16 CSR is not run: it aborts the process on PyTorch-ROCm"


def _spmm_auto_16(crow, col, val, x, config: SchedulerConfig, verbose: bool) -> tuple[torch.Tensor, dict[str, Any]]:
    """bf16 / fp16 features (the reference runs torch.sparse.mm for them,
    ``_auto.py:281-287``).  Every output is the exactly rounded sum whatever
    the schedule, so there is no shortlist to probe and no accuracy trade:
    the schedules of the native SpMM (column slices, when the columns ascend,
    edge slices, and rows whole in one launch) are timed once on the full
    graph and the fastest is cached under the usual key, which includes the
    dtype.  The PyTorch
    baseline cannot be run for these types here (see _BASELINE_16_NOTE)."""
    if config.cache:
        result = _cached_record(crow, col, x.size(1), "spmm", config, weighted=val is not None, dtype=x.dtype)
        if result is not None and result.get("candidate") in _ROUNDED16_ALL:
            return (_run_spmm_choice("autosage", result["candidate"], crow, col, val, x),
                    {**result, "from_cache": True})
    device = device_signature()
    graph = graph_signature_memo(crow, col, x.size(1), "spmm", weighted=val is not None, dtype=x.dtype)
    cache = ScheduleCache()
    if config.replay_only:
        info = _replay_miss("spmm", "torch.sparse.mm(csr)")
        info.update(choice="autosage", candidate=ROUNDED16, reason="cache miss; " + _BASELINE_16_NOTE)
        return _run_spmm_choice("autosage", ROUNDED16, crow, col, val, x), info
    from ._native import columns_ascending

    wall_start = time.perf_counter()
    options = [ROUNDED16_EDGES] + ([ROUNDED16] if columns_ascending(crow, col) else []) + [ROUNDED16_ROWS]
    times = {
        o: _time_cuda(lambda o=o: _run_spmm_choice("autosage", o, crow, col, val, x), warmup=1, iterations=3)[
            "best_ms"]
        for o in options
    }
    best = min(options, key=lambda o: times[o])
    result: dict[str, Any] = {
        "operation": "spmm",
        "schema_version": AUTOTUNE_SCHEMA_VERSION,
        "choice": "autosage",
        "candidate": best,
        "baseline": "torch.sparse.mm(csr)",
        "guardrail": config.guardrail,
        "configuration": config.tuning_signature(),
        "probe_rows": int(crow.numel() - 1),
        "probe_nonzeros": int(col.numel()),
        "sampling_ms": 0.0,
        "probe_ms": (time.perf_counter() - wall_start) * 1000.0,
        "baseline_probe_ms": None,
        "autosage_probe_ms": times[best],
        "sampled_speedup": None,
        "candidates": [{"candidate": o, "best_ms": times[o]} for o in options],
        "from_cache": False,
        "reason": _BASELINE_16_NOTE,
    }
    output = _run_spmm_choice("autosage", best, crow, col, val, x)
    if config.cache:
        cache.store(device, graph, result)
    log_probe({"timestamp": time.time(), "device": device, "graph": graph, "result": result})
    _verbose("spmm", result, verbose)
    return output, result


_SDDMM_MIN_HUB_DEGREE = 1024


def _full_graph_candidate(crow: torch.Tensor, feature_width: int, config: SchedulerConfig) -> list[int]:
    """The shortlist's preferred point with the FULL graph's q95 as the hub
    threshold: the sample's quantiles are scaled down by the sampling
    fraction, so its thresholds can send every full-graph row to the hub
    path."""
    _, q95, _ = _degree_quantiles(crow)
    tile = config.feature_tile or (64 if feature_width <= 64 else 128)
    waves = config.warps_per_block or _preferred_waves(feature_width)
    return [int(tile), int(waves), int(config.hub_threshold or q95)]


def _prefer_exact(options: list[str], times: dict[str, float], inexact: tuple = ()) -> str:
    """The fastest option, except that an option of ``inexact`` (JSON keys)
    must beat the fastest of the others by more than ``_INEXACT_MARGIN``."""
    best_key = min(options, key=lambda k: times[k])
    exact = [k for k in options if k not in inexact]
    if best_key in inexact and exact:
        best_exact = min(exact, key=lambda k: times[k])
        if times[best_exact] <= times[best_key] * (1.0 + _INEXACT_MARGIN):
            return best_exact
    return best_key


def _decide_on_full_graph(result: dict[str, Any], options: list[Any], run_option, baseline,
                          inexact: tuple = ()) -> None:
    """Times each native option on the full graph (1 warmup, best of 3) and
    the baseline, keeps the fastest native option (a reassociating option of
    ``inexact`` only when it beats the best bit-exact one by more than
    ``_INEXACT_MARGIN``), and falls back to the baseline only when that is
    faster.  `result` gets a ``full_graph`` record; the sampled probe has
    only shortlisted."""
    wall_start = time.perf_counter()
    options = list(dict.fromkeys(json.dumps(o) for o in options))
    times = {
        key: _time_cuda(lambda o=json.loads(key): run_option(o), warmup=1, iterations=3)["best_ms"] for key in options
    }
    best_key = _prefer_exact(options, times, tuple(json.dumps(o) for o in inexact))
    best_ms = times[best_key]
    # One baseline call decides when it takes more than twice the best native
    # time; a closer race gets the full warm timing.  The sampled probe has
    # already run the baseline, so library set-up is not in this call, and on
    # large graphs one baseline call costs tens of native ones.
    baseline_ms = _time_cuda(baseline, warmup=0, iterations=1)["best_ms"]
    baseline_runs = 1
    if baseline_ms < 2.0 * best_ms:
        baseline_ms = _time_cuda(baseline, warmup=1, iterations=3)["best_ms"]
        baseline_runs = 5
    result["full_graph"] = {
        "autosage_ms": best_ms,
        "baseline_ms": baseline_ms,
        "baseline_runs": baseline_runs,
        "candidates": [{"candidate": json.loads(k), "best_ms": times[k]} for k in options],
        "sampled_choice": result.get("candidate"),
        "wall_ms": (time.perf_counter() - wall_start) * 1000.0,
    }
    if best_ms > baseline_ms:
        result["choice"] = "baseline"
        result["candidate"] = None
        result["reason"] = "slower than the baseline on the full graph"
    else:
        result["choice"] = "autosage"
        result["candidate"] = json.loads(best_key)
        result.pop("reason", None)


def _confirm_spmm_on_full_graph(result: dict[str, Any], colslice: bool, config: SchedulerConfig, probe,
                                crow, col, val, x, fslice: bool = False) -> None:
    """SpMM options on the full graph: the sampled probe's best split
    candidate, the preferred candidate at the full graph's q95, the
    whole-graph kernel (candidate None) and, when eligible, the
    feature-sliced and the column-sliced SpMM (the latter taken only when it
    beats the best bit-exact option by more than ``_INEXACT_MARGIN``)."""
    options: list[Any] = [probe["chosen"]] if probe["chosen"] is not None else []
    if native_op("spmm_csr_split") is not None and config.hub_split:
        options.append(_full_graph_candidate(crow, x.size(1), config))
    options.append(None)
    if fslice:
        options.append(FSLICE)
    if colslice:
        options.append(COLSLICE)
    full_baseline, _ = _prepare_spmm_baseline(crow, col, val, x)
    _decide_on_full_graph(result, options, lambda o: _run_spmm_choice("autosage", o, crow, col, val, x),
                          full_baseline, inexact=(COLSLICE,))


def calibrate_full(crow, col, val, x, guardrail: float = 0.95) -> tuple[str, dict[str, Any]]:
    """Full-graph calibration (``_auto.py:444-522``) of every shortlisted
    candidate, the whole-graph kernel and, when eligible, the feature-sliced
    and the column-sliced SpMM (the latter kept only when it beats the best
    bit-exact option by more than ``_INEXACT_MARGIN``)."""
    crow, col, val, x = _normalize_csr(crow, col, val, x)
    if not x.is_cuda:
        return "baseline", _cpu_info("spmm")
    if x.dtype != torch.float32:
        return "baseline", {
            **_cpu_info("spmm"),
            "baseline": "torch.sparse.mm(csr)",
            "reason": "AutoSAGE CUDA kernels require float32 features",
        }
    _require_native()
    config = SchedulerConfig.from_env(guardrail=guardrail, candidate_count=6)
    baseline, baseline_name = _prepare_spmm_baseline(crow, col, val, x)
    baseline_timing = _time_cuda(baseline, warmup=2, iterations=5)
    split = native_op("spmm_csr_split") if config.hub_split else None
    core = native_op("spmm_csr")
    best, selected = float("inf"), None
    timings: list[dict[str, Any]] = []
    if split is not None:
        for tile, waves, threshold in _spmm_candidates(crow, x.size(1), config):
            t = _time_cuda(lambda a=tile, b=waves, c=threshold: split(crow, col, val, x, a, b, c), warmup=2, iterations=5)
            timings.append({"candidate": [tile, waves, threshold], "best_ms": t["best_ms"]})
            if t["best_ms"] < best:
                best, selected = t["best_ms"], [tile, waves, threshold]
    if core is not None:
        # the whole-graph kernel (candidate None), as in the full-graph decision
        t = _time_cuda(lambda: core(crow, col, val, x), warmup=2, iterations=5)
        timings.append({"candidate": None, "best_ms": t["best_ms"]})
        if t["best_ms"] < best:
            best, selected = t["best_ms"], None
    if _fslice_eligible(crow, col, x, config):
        fslice_op = native_op("spmm_csr_fslice")
        t = _time_cuda(lambda: fslice_op(crow, col, val, x), warmup=2, iterations=5)
        timings.append({"candidate": FSLICE, "best_ms": t["best_ms"]})
        if t["best_ms"] < best:
            best, selected = t["best_ms"], FSLICE
    if _colslice_eligible(crow, col, x, config):
        colslice_op = native_op("spmm_csr_colslice")
        t = _time_cuda(lambda: colslice_op(crow, col, val, x), warmup=2, iterations=5)
        timings.append({"candidate": COLSLICE, "best_ms": t["best_ms"]})
        # the reassociating schedule only when it beats every bit-exact one by the margin
        if t["best_ms"] * (1.0 + _INEXACT_MARGIN) < best:
            best, selected = t["best_ms"], COLSLICE
    choice = "autosage" if best <= guardrail * baseline_timing["best_ms"] else "baseline"
    result = {
        "operation": "spmm",
        "schema_version": AUTOTUNE_SCHEMA_VERSION,
        "choice": choice,
        "candidate": selected if choice == "autosage" else None,
        "baseline": baseline_name,
        "guardrail": guardrail,
        "configuration": config.tuning_signature(),
        "calibration": "full_graph",
        "baseline_ms": baseline_timing["best_ms"],
        "autosage_ms": None if best == float("inf") else best,
        "speedup": baseline_timing["best_ms"] / best if best not in (0.0, float("inf")) else None,
        "candidates": timings,
        "from_cache": False,
    }
    device = device_signature()
    graph = graph_signature_memo(crow, col, x.size(1), "spmm", weighted=val is not None, dtype=x.dtype)
    if config.cache:
        ScheduleCache().store(device, graph, result)
    log_probe({"timestamp": time.time(), "device": device, "graph": graph, "result": result})
    return choice, result


def _normalize_sddmm(crow, col, query, key):
    """Checks of ``_auto.py:554-570``."""
    if crow.dtype not in (torch.int32, torch.int64) or col.dtype not in (torch.int32, torch.int64):
        raise TypeError("crow and col must use integer indices")
    crow = crow.to(dtype=torch.long).contiguous()
    col = col.to(dtype=torch.long).contiguous()
    query, key = query.contiguous(), key.contiguous()
    if query.shape != key.shape or query.ndim != 2:
        raise ValueError("query and key must have the same [N, F] shape")
    if not query.is_floating_point() or query.dtype != key.dtype:
        raise TypeError("query and key must use the same floating-point dtype")
    if crow.ndim != 1 or col.ndim != 1:
        raise ValueError("crow and col must be one-dimensional")
    if crow.numel() != query.size(0) + 1:
        raise ValueError("crow must contain N + 1 entries")
    if not (crow.device == col.device == query.device == key.device):
        raise ValueError("all SDDMM inputs must be on the same device")
    validate_if_requested(crow, col)
    return crow, col, query, key


def sddmm_csr_auto(
    crow: torch.Tensor,
    col: torch.Tensor,
    query: torch.Tensor,
    key: torch.Tensor,
    *,
    guardrail: float = 0.95,
    seed: int = 0,
    verbose: bool = False,
) -> tuple[torch.Tensor, dict[str, Any]]:
    crow, col, query, key = _normalize_sddmm(crow, col, query, key)
    if not query.is_cuda:
        run, name = _prepare_sddmm_baseline(crow, col, query, key)
        return run(), {**_cpu_info("sddmm"), "baseline": name}
    if query.dtype in _DTYPES_16:
        _require_native()
        return _sddmm_auto_16(crow, col, query, key, SchedulerConfig.from_env(guardrail=guardrail), verbose)
    if query.dtype != torch.float32:
        run, name = _prepare_sddmm_baseline(crow, col, query, key)
        return run(), {**_cpu_info("sddmm"), "baseline": name, "reason": "AutoSAGE CUDA kernels require float32 features"}

    _require_native()
    config = SchedulerConfig.from_env(guardrail=guardrail, candidate_count=6)
    if config.cache:
        result = _cached_record(crow, col, query.size(1), "sddmm", config, dtype=query.dtype)
        if result is not None:
            choice, candidate = result.get("choice", "baseline"), result.get("candidate")
            if _cached_native_available("sddmm_csr", choice, candidate):
                return _run_sddmm_choice(choice, candidate, crow, col, query, key), {**result, "from_cache": True}
    if config.replay_only:
        return _run_sddmm_choice("baseline", None, crow, col, query, key), _replay_miss("sddmm", "gather-dot")
    device = device_signature()
    graph = graph_signature_memo(crow, col, query.size(1), "sddmm", dtype=query.dtype)
    cache = ScheduleCache()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s_crow, s_col, _, selected = _induced_sample_csr(
        crow, col, None, fraction=config.probe_fraction, minimum_rows=config.probe_min_rows, seed=seed
    )
    s_q = query.index_select(0, selected).contiguous()
    s_k = key.index_select(0, selected).contiguous()
    torch.cuda.synchronize()
    sample_ms = (time.perf_counter() - t0) * 1000.0

    baseline, baseline_name = _prepare_sddmm_baseline(s_crow, s_col, s_q, s_k)
    split = native_op("sddmm_csr_split") if config.hub_split else None
    core = native_op("sddmm_csr")
    split_calls = []
    if split is not None:
        pairs = dict.fromkeys((w, h) for _, w, h in _spmm_candidates(s_crow, query.size(1), config))
        for waves, threshold in pairs:
            split_calls.append(([waves, threshold], lambda w=waves, h=threshold: split(s_crow, s_col, s_q, s_k, w, h)))
    core_call = (lambda: core(s_crow, s_col, s_q, s_k)) if (split is None and core is not None) else None
    probe = _probe_and_choose(
        operation="sddmm",
        config=config,
        sampled_crow=s_crow,
        sampled_col=s_col,
        baseline=baseline,
        split_calls=split_calls,
        core_call=core_call,
    )
    result = _result_dict("sddmm", config, probe, baseline_name, s_crow, s_col, sample_ms)
    if config.full_graph_check and split is not None:
        # the sampled best pair and the pair of the full graph's preferred
        # candidate, on the full graph
        # (the SDDMM hub path cuts rows into 2048-edge chunks; below ~1024
        # edges the one-wave-per-row path is faster: on cfg4, where 101k rows
        # have degree 197-198 = q95, threshold 197 costs 2.45 ms, 256 or
        # 1024 cost 1.82 ms)
        _, waves, threshold = _full_graph_candidate(crow, query.size(1), config)
        if config.hub_threshold is None:
            threshold = max(threshold, _SDDMM_MIN_HUB_DEGREE)
        options = ([probe["chosen"]] if probe["chosen"] is not None else []) + [[waves, threshold]]
        full_baseline, _ = _prepare_sddmm_baseline(crow, col, query, key)
        _decide_on_full_graph(result, options, lambda o: _run_sddmm_choice("autosage", o, crow, col, query, key),
                              full_baseline)
    output = _run_sddmm_choice(result["choice"], result["candidate"], crow, col, query, key)
    if config.cache:
        cache.store(device, graph, result)
    log_probe({"timestamp": time.time(), "device": device, "graph": graph, "result": result})
    _verbose("sddmm", result, verbose)
    return output, result


# Split points timed for 16-bit SDDMM: (waves per block, hub threshold).
# None: sddmm_csr's own schedule (blocks of 64 edges in CSR order)
_SDDMM_16_OPTIONS = (None, [4, 1024], [8, 4096])
_SDDMM_16_NOTE = ("bf16/fp16 SDDMM is native (fp64 sums of exact products, rounded); the gather-dot baseline "
                  "rounds every product to the 16-bit type and is not a candidate")


def _sddmm_auto_16(crow, col, query, key, config: SchedulerConfig, verbose: bool) -> tuple[torch.Tensor, dict]:
    """bf16 / fp16 query and key (the reference runs its gather-dot baseline
    for them, ``_auto.py:575-581``).  Every output is the rounded fp64 sum
    whatever the schedule, so the schedules of ``_SDDMM_16_OPTIONS`` (edge
    blocks, and two degree splits) are timed once on the full graph and the
    fastest is cached under the usual key (which includes the dtype)."""
    options = [None if o is None else list(o) for o in _SDDMM_16_OPTIONS]
    if config.cache:
        result = _cached_record(crow, col, query.size(1), "sddmm", config, dtype=query.dtype)
        if result is not None and result.get("choice") == "autosage" and result.get("candidate") in options:
            return (_run_sddmm_choice("autosage", result["candidate"], crow, col, query, key),
                    {**result, "from_cache": True})
    device = device_signature()
    graph = graph_signature_memo(crow, col, query.size(1), "sddmm", dtype=query.dtype)
    cache = ScheduleCache()
    if config.replay_only:
        info = _replay_miss("sddmm", "gather-dot")
        info.update(choice="autosage", candidate=options[0], reason="cache miss; " + _SDDMM_16_NOTE)
        return _run_sddmm_choice("autosage", options[0], crow, col, query, key), info
    wall_start = time.perf_counter()
    times = [
        _time_cuda(lambda o=o: _run_sddmm_choice("autosage", o, crow, col, query, key), warmup=1, iterations=3)[
            "best_ms"]
        for o in options
    ]
    best = min(range(len(options)), key=lambda i: times[i])
    result: dict[str, Any] = {
        "operation": "sddmm",
        "schema_version": AUTOTUNE_SCHEMA_VERSION,
        "choice": "autosage",
        "candidate": options[best],
        "baseline": "gather-dot",
        "guardrail": config.guardrail,
        "configuration": config.tuning_signature(),
        "probe_rows": int(crow.numel() - 1),
        "probe_nonzeros": int(col.numel()),
        "sampling_ms": 0.0,
        "probe_ms": (time.perf_counter() - wall_start) * 1000.0,
        "baseline_probe_ms": None,
        "autosage_probe_ms": times[best],
        "sampled_speedup": None,
        "candidates": [{"candidate": o, "best_ms": t} for o, t in zip(options, times)],
        "from_cache": False,
        "reason": _SDDMM_16_NOTE,
    }
    output = _run_sddmm_choice("autosage", options[best], crow, col, query, key)
    if config.cache:
        cache.store(device, graph, result)
    log_probe({"timestamp": time.time(), "device": device, "graph": graph, "result": result})
    _verbose("sddmm", result, verbose)
    return output, result


def _torch_row_softmax(crow: torch.Tensor, scores: torch.Tensor) -> torch.Tensor:
    """The reference composition (``_auto.py:744-759``): per-row amax,
    exp(s - max), scatter_add denominators, divide."""
    rows = _edge_rows(crow)
    if scores.numel() == 0:
        return scores.clone()
    maxima = torch.full((crow.numel() - 1,), -torch.inf, dtype=scores.dtype, device=scores.device)
    maxima.scatter_reduce_(0, rows, scores, reduce="amax", include_self=True)
    exps = (scores - maxima.index_select(0, rows)).exp()
    sums = torch.zeros_like(maxima)
    sums.scatter_add_(0, rows, exps)
    return exps / sums.index_select(0, rows)


def _csr_row_softmax(crow: torch.Tensor, scores: torch.Tensor) -> torch.Tensor:
    """CSR row softmax: the native kernel on the GPU (float32, and bf16 /
    fp16 computed in fp32 and rounded once), the reference torch composition
    on the CPU."""
    if scores.is_cuda and scores.dtype in (torch.float32, torch.bfloat16, torch.float16):
        if not load_native() or native_op("csr_row_softmax") is None:
            raise RuntimeError("AutoSAGE native csr_row_softmax is unavailable")
        return native_op("csr_row_softmax")(crow.to(torch.long).contiguous(), scores.contiguous())
    return _torch_row_softmax(crow, scores)


def _attention_colslice_eligible(crow, col, query, value, config: SchedulerConfig) -> bool:
    """Whether the fused path should time the column-sliced attention."""
    if config.column_slices == "off" or not config.full_graph_check:
        return False
    if native_op("csr_attention_colslice") is None or crow.numel() <= 1 or col.numel() == 0:
        return False
    from ._native import attention_colslice_supported, columns_ascending, row_counts

    if not attention_colslice_supported(query, value):
        return False
    gathered = (query.size(1) + value.size(1)) * 4 * (crow.numel() - 1)
    if (config.column_slices == "auto" and gathered < _COLSLICE_MIN_X_BYTES
            and row_counts(crow, _COLSLICE_HUB_DEGREE, 0)[0] == 0):
        return False
    columns_ascending(crow, col)  # a malformed graph raises; any column order is eligible
    return True


def _attention_variant(crow, col, q, k, v, scale: float) -> tuple[str, dict[str, Any]]:
    """"fused" (the exact fused kernel) or "colslice" for this graph: the
    column-sliced attention is timed against the fused kernel once per graph
    on the full graph when eligible, and the faster one is cached."""
    config = SchedulerConfig.from_env()
    if not _attention_colslice_eligible(crow, col, q, v, config):
        return "fused", {"variant": "fused", "from_cache": False}
    operation = f"attention:fv={v.size(1)}"
    if config.cache:
        result = _cached_record(crow, col, q.size(1), operation, config, dtype=q.dtype)
        if result is not None and result.get("variant") in ("fused", "colslice"):
            return result["variant"], {**result, "from_cache": True}
    device = device_signature()
    graph = graph_signature_memo(crow, col, q.size(1), operation, dtype=q.dtype)
    cache = ScheduleCache()
    times = {}
    for name, op in (("fused", native_op("csr_attention")), ("colslice", native_op("csr_attention_colslice"))):
        times[name] = _time_cuda(lambda o=op: o(crow, col, q, k, v, scale), warmup=1, iterations=3)["best_ms"]
    variant = min(times, key=times.get)
    result = {
        "operation": "attention",
        "schema_version": AUTOTUNE_SCHEMA_VERSION,
        "variant": variant,
        "configuration": config.tuning_signature(),
        "full_graph": {"fused_ms": times["fused"], "colslice_ms": times["colslice"]},
        "from_cache": False,
    }
    if config.cache:
        cache.store(device, graph, result)
    return variant, result


def _fused_default() -> bool:
    return _env.get("AUTOSAGE_FUSED_ATTENTION", "1") == "1"


def csr_attention_forward(
    crow: torch.Tensor,
    col: torch.Tensor,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    guardrail: float = 0.95,
    seed: int = 0,
    verbose: bool = False,
    scale: float = 1.0,
    fused: Optional[bool] = None,
) -> tuple[torch.Tensor, dict[str, Any]]:
    """softmax_row(scale · SDDMM(query, key)) · value (``_auto.py:762-780``;
    the reference has no scale, i.e. scale = 1).

    On the GPU with ``fused`` (default: the ``AUTOSAGE_FUSED_ATTENTION``
    switch, on) the three stages run as one native kernel: for float32 the
    exact fused kernel or the column-sliced one, whichever a full-graph
    timing picks; for bf16 / fp16 the column-sliced kernel in fp32 arithmetic
    with each output rounded once (when its widths fit: multiples of 8 up to
    512).  Otherwise the stages run as the scheduled SDDMM, the row softmax
    and the scheduled SpMM, as in the reference."""
    use_fused = _fused_default() if fused is None else bool(fused)
    if (use_fused and query.is_cuda and query.dtype in _DTYPES_16 and value.dtype == query.dtype
            and key.dtype == query.dtype):
        crow_n, col_n, q, k = _normalize_sddmm(crow, col, query, key)
        from ._native import attention_colslice_supported

        v = value.contiguous()
        if attention_colslice_supported(q, v) and k.data_ptr() % 16 == 0:
            _require_native()
            out = native_op("csr_attention_colslice")(crow_n, col_n, q, k, v, float(scale))
            info = {"operation": "attention", "schema_version": AUTOTUNE_SCHEMA_VERSION, "choice": "fused",
                    "from_cache": False}
            return out, {"sddmm": {**info, "operation": "sddmm"}, "spmm": {**info, "operation": "spmm"},
                         "fused": True, "variant": "colslice16", "attention": {"variant": "colslice16"}}
    if use_fused and query.is_cuda and query.dtype == torch.float32 and value.dtype == torch.float32:
        crow_n, col_n, q, k = _normalize_sddmm(crow, col, query, key)
        if not load_native() or native_op("csr_attention") is None:
            raise RuntimeError("AutoSAGE native csr_attention is unavailable")
        v = value.contiguous()
        variant, decision = _attention_variant(crow_n, col_n, q, k, v, float(scale))
        out = native_op("csr_attention" if variant == "fused" else "csr_attention_colslice")(
            crow_n, col_n, q, k, v, float(scale))
        info = {"operation": "attention", "schema_version": AUTOTUNE_SCHEMA_VERSION, "choice": "fused",
                "from_cache": decision.get("from_cache", False)}
        return out, {"sddmm": {**info, "operation": "sddmm"}, "spmm": {**info, "operation": "spmm"}, "fused": True,
                     "variant": variant, "attention": decision}
    scores, sddmm_info = sddmm_csr_auto(crow, col, query, key, guardrail=guardrail, seed=seed, verbose=verbose)
    scores = scores.to(query.dtype)
    if scale != 1.0:
        scores = scores * scale
    probabilities = _csr_row_softmax(crow, scores)
    output, spmm_info = spmm_csr_auto(crow, col, probabilities, value, guardrail=guardrail, seed=seed, verbose=verbose)
    return output, {"sddmm": sddmm_info, "spmm": spmm_info}


__all__ = [
    "AUTOTUNE_SCHEMA_VERSION",
    "calibrate_full",
    "csr_attention_forward",
    "sddmm_csr_auto",
    "spmm_csr_auto",
]
