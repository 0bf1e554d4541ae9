"""Schedule keys and the on-disk schedule cache.

Follows ``autosage/_cache.py`` of the reference so that keys and files are
interchangeable: the device dictionary (``:24-37``), the graph dictionary with
rounded linear degree quantiles (``:57-93``), the 24-hex-digit structure hash
over the raw little-endian bytes of at most the first and last 1024 entries of
``crow`` and ``col`` (``:40-54``), the key as canonical JSON of
``{"device", "graph"}`` (``:103-107``), the schema-1 JSON file replaced
atomically (``:126-148``) and the JSONL probe log (``:151-157``).
"""

from __future__ import annotations

import collections
import hashlib
import json
import os
import tempfile
import threading
import time
import weakref
from pathlib import Path
from typing import Any, Optional

import torch

from . import _env
from ._memo import GraphMemo

CACHE_SCHEMA_VERSION = 1
_HASH_EDGE = 1024  # entries hashed from each end of a long index vector

# Steady-state memos that keep the per-call host work of the schedulers small
# (no quantile sort, hash, device->host sync or JSON parse on a repeated
# call).  Both cache values the functions below would recompute identically.
_MEMO_LOCK = threading.Lock()
_SIGNATURE_MEMO: "collections.OrderedDict[tuple, tuple]" = collections.OrderedDict()
_SIGNATURE_MEMO_SIZE = 64
_FILE_MEMO: dict[str, tuple[int, int, dict]] = {}


_DIRECTORY_MEMO: dict[Optional[str], Path] = {}


def cache_directory() -> Path:
    configured = _env.get("AUTOSAGE_CACHE_DIR")
    path = _DIRECTORY_MEMO.get(configured)
    if path is None:
        path = Path(configured).expanduser() if configured else Path.home() / ".cache" / "autosage"
        _DIRECTORY_MEMO[configured] = path
    return path


_FILE_PATH_MEMO: dict[Path, Path] = {}


def schedule_file() -> Path:
    """The schedule cache file of the current ``AUTOSAGE_CACHE_DIR``."""
    directory = cache_directory()
    path = _FILE_PATH_MEMO.get(directory)
    if path is None:
        path = directory / "schedules.json"
        _FILE_PATH_MEMO[directory] = path
    return path


_DEVICE_MEMO: dict[int, dict[str, Any]] = {}


def device_signature(device: Optional[int] = None) -> dict[str, Any]:
    if not torch.cuda.is_available():
        return {"type": "cpu", "torch": torch.__version__}
    index = torch.cuda.current_device() if device is None else device
    signature = _DEVICE_MEMO.get(index)
    if signature is None:
        # a device's properties do not change while the process runs
        props = torch.cuda.get_device_properties(index)
        signature = {
            "type": "cuda",
            "name": props.name,
            "compute_capability": [props.major, props.minor],
            "multiprocessors": props.multi_processor_count,
            "total_memory": int(props.total_memory),
            "cuda": torch.version.cuda,
            "torch": torch.__version__,
        }
        _DEVICE_MEMO[index] = signature
    return {**signature, "compute_capability": list(signature["compute_capability"])}


def _hash_slice(tensor: torch.Tensor) -> torch.Tensor:
    count = tensor.numel()
    if count <= 2 * _HASH_EDGE:
        return tensor
    return torch.cat((tensor[:_HASH_EDGE], tensor[-_HASH_EDGE:]))


def _sample_hash(crow: torch.Tensor, col: torch.Tensor) -> str:
    digest = hashlib.sha256()
    for tensor in (crow, col):
        if tensor.numel() == 0:
            continue
        raw = _hash_slice(tensor).detach().contiguous().cpu()
        digest.update(raw.numpy().tobytes())
    return digest.hexdigest()[:24]


def _rounded_quantiles(degrees: torch.Tensor, qs: list[float]) -> list[int]:
    points = torch.tensor(qs, dtype=torch.float64, device=degrees.device)
    values = torch.quantile(degrees.to(torch.float64), points).round().to(torch.long)
    return [int(v) for v in values.cpu().tolist()]


def graph_signature(
    crow: torch.Tensor,
    col: torch.Tensor,
    feature_width: int,
    operation: str,
    *,
    weighted: bool = False,
    dtype: Optional[torch.dtype] = None,
) -> dict[str, Any]:
    degrees = crow[1:] - crow[:-1]
    q50, q90, q99 = _rounded_quantiles(degrees, [0.5, 0.9, 0.99]) if degrees.numel() else (0, 0, 0)
    return {
        "operation": operation,
        "feature_width": int(feature_width),
        "dtype": None if dtype is None else str(dtype),
        "weighted": bool(weighted),
        "rows": int(crow.numel() - 1),
        "nonzeros": int(col.numel()),
        "degree_q50": q50,
        "degree_q90": q90,
        "degree_q99": q99,
        "structure_hash": _sample_hash(crow, col),
    }


def graph_signature_memo(
    crow: torch.Tensor,
    col: torch.Tensor,
    feature_width: int,
    operation: str,
    *,
    weighted: bool = False,
    dtype: Optional[torch.dtype] = None,
) -> dict[str, Any]:
    """``graph_signature`` memoised per live (crow, col) tensor pair.

    The memo holds weak references to the two tensor objects and their
    in-place version counters: a hit needs the very same objects, still
    alive and unmodified, so the signature cannot be stale.  Saves the two
    device->host syncs, the quantile sort and the hash on repeated calls."""
    key = (id(crow), crow._version, id(col), col._version, int(feature_width), operation, bool(weighted), str(dtype))
    with _MEMO_LOCK:
        entry = _SIGNATURE_MEMO.get(key)
        if entry is not None and entry[0]() is crow and entry[1]() is col:
            _SIGNATURE_MEMO.move_to_end(key)
            return dict(entry[2])
    signature = graph_signature(crow, col, feature_width, operation, weighted=weighted, dtype=dtype)
    try:
        refs = (weakref.ref(crow), weakref.ref(col))
    except TypeError:
        return signature
    with _MEMO_LOCK:
        _SIGNATURE_MEMO[key] = (*refs, dict(signature))
        while len(_SIGNATURE_MEMO) > _SIGNATURE_MEMO_SIZE:
            _SIGNATURE_MEMO.popitem(last=False)
    return signature


def _file_stamp(path: Path) -> Optional[tuple[int, int]]:
    try:
        st = path.stat()
    except OSError:
        return None
    return st.st_mtime_ns, st.st_size


class ScheduleCache:
    def __init__(self, path: Optional[os.PathLike[str] | str] = None):
        self.path = Path(path) if path is not None else schedule_file()
        self._records = self._load_memo()

    def _load_memo(self) -> dict[str, dict[str, Any]]:
        """``_load`` unless the file is unchanged (same mtime and size) since
        this process last parsed or wrote it.  The records are shared with
        the memo and copied before ``store`` changes them."""
        stamp = _file_stamp(self.path)
        key = str(self.path)
        with _MEMO_LOCK:
            memo = _FILE_MEMO.get(key)
            if stamp is not None and memo is not None and memo[:2] == stamp:
                return memo[2]
        records = self._load()
        if stamp is not None:
            with _MEMO_LOCK:
                _FILE_MEMO[key] = (*stamp, records)
        return records

    @staticmethod
    def _key(device: dict[str, Any], graph: dict[str, Any]) -> str:
        return json.dumps({"device": device, "graph": graph}, sort_keys=True, separators=(",", ":"))

    def _load(self) -> dict[str, dict[str, Any]]:
        try:
            payload = json.loads(self.path.read_text(encoding="utf-8"))
        except FileNotFoundError:
            return {}
        except (OSError, json.JSONDecodeError):
            return {}
        if not isinstance(payload, dict) or payload.get("schema_version") != CACHE_SCHEMA_VERSION:
            return {}
        records = payload.get("records", {})
        return records if isinstance(records, dict) else {}

    def lookup(self, device: dict[str, Any], graph: dict[str, Any]) -> Optional[dict[str, Any]]:
        return self._records.get(self._key(device, graph))

    def store(self, device: dict[str, Any], graph: dict[str, Any], result: dict[str, Any]) -> None:
        self.path.parent.mkdir(parents=True, exist_ok=True)
        records = dict(self._records)  # the loaded records may be shared with the memo
        records[self._key(device, graph)] = {
            "timestamp": int(time.time()),
            "device": device,
            "graph": graph,
            "result": result,
        }
        self._records = records
        payload = {"schema_version": CACHE_SCHEMA_VERSION, "records": self._records}
        fd, temporary = tempfile.mkstemp(prefix="schedules-", suffix=".json", dir=self.path.parent)
        try:
            with os.fdopen(fd, "w", encoding="utf-8") as stream:
                json.dump(payload, stream, indent=2, sort_keys=True)
                stream.write("\n")
            os.replace(temporary, self.path)
        finally:
            if os.path.exists(temporary):
                os.unlink(temporary)
        stamp = _file_stamp(self.path)
        if stamp is not None:
            with _MEMO_LOCK:
                _FILE_MEMO[str(self.path)] = (*stamp, self._records)


# The cache record a repeated call replays, per live (crow, col) pair and the
# call's settings, so that a steady-state call skips the device and graph
# signatures, the canonical-JSON key and the record lookup.  The schedule
# file's stamp (mtime, size) is part of the key: a file written since (by this
# or another process) is looked up again.
_DECISION_MEMO = GraphMemo("cached_decision", max_entries=64)


def cached_result(crow: torch.Tensor, col: torch.Tensor, extra: tuple,
                  lookup) -> Optional[dict[str, Any]]:
    """``lookup(cache)`` (the cached result or None) memoised per live,
    unmodified (crow, col), ``extra`` (the caller's settings) and the current
    schedule file and its stamp."""
    path = schedule_file()
    stamp = _file_stamp(path)
    if stamp is None:
        return lookup(ScheduleCache(path))
    return _DECISION_MEMO.get((crow, col), (extra, str(path), stamp), lambda: lookup(ScheduleCache(path)))


def log_probe(event: dict[str, Any]) -> None:
    if _env.get("AUTOSAGE_LOG_PROBES", "1") != "1":
        return
    path = cache_directory() / "probe_logs.jsonl"
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("a", encoding="utf-8") as stream:
        stream.write(json.dumps(event, sort_keys=True) + "\n")


__all__ = [
    "CACHE_SCHEMA_VERSION",
    "ScheduleCache",
    "cache_directory",
    "device_signature",
    "graph_signature",
    "graph_signature_memo",
    "log_probe",
]
