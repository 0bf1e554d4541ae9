"""Values derived once per graph and kept while the graph's tensors live.

The schedulers and operators derive per-graph data from the CSR tensors:
whether the columns ascend, how many rows are long enough to slice, the
transposed CSR of the backward, the row-sorted copy of a graph whose columns
do not ascend.  Recomputing them on every call costs host syncs and
nnz-sized passes, so they are memoised per live, unmodified tensor tuple:

* the key is the tensors' identities and version counters plus any extra
  hashable argument, so an in-place change of a tensor misses;
* an entry is dropped as soon as one of its tensors is garbage-collected
  (``weakref.finalize``), so a dead graph never keeps its derived device
  buffers alive, and the entries of older versions of the same tensors are
  dropped when a new version is stored;
* the memo is capped by entry count and by the bytes of the device tensors
  its values hold (least recently used first).

Thread-safe; the derived values must not hold references to the key tensors
(that would keep them alive and the entry with them).
"""

from __future__ import annotations

import collections
import threading
import weakref
from typing import Any, Callable, Hashable, Sequence

import torch


def _value_bytes(value: Any) -> int:
    if isinstance(value, torch.Tensor):
        return value.numel() * value.element_size()
    if isinstance(value, (tuple, list)):
        return sum(_value_bytes(v) for v in value)
    if isinstance(value, dict):
        return sum(_value_bytes(v) for v in value.values())
    return 0


class GraphMemo:
    """LRU memo keyed by live tensors (see the module docstring)."""

    def __init__(self, name: str, max_entries: int = 64, max_bytes: int | None = None) -> None:
        self.name = name
        self.max_entries = max_entries
        self.max_bytes = max_bytes
        self._lock = threading.Lock()
        # key -> (weak refs, value, bytes)
        self._entries: "collections.OrderedDict[tuple, tuple]" = collections.OrderedDict()
        self._bytes = 0

    @staticmethod
    def _key(tensors: Sequence[torch.Tensor], extra: Hashable) -> tuple:
        return (tuple((id(t), t._version) for t in tensors), extra)

    def get(self, tensors: Sequence[torch.Tensor], extra: Hashable, compute: Callable[[], Any]) -> Any:
        """The memoised value for (tensors, extra), computed on a miss."""
        key = self._key(tensors, extra)
        with self._lock:
            hit = self._entries.get(key)
            if hit is not None and all(ref() is t for ref, t in zip(hit[0], tensors)):
                self._entries.move_to_end(key)
                return hit[1]
        value = compute()
        self.put(tensors, extra, value, key=key)
        return value

    def put(self, tensors: Sequence[torch.Tensor], extra: Hashable, value: Any, *, key: tuple | None = None) -> None:
        key = key if key is not None else self._key(tensors, extra)
        try:
            refs = tuple(weakref.ref(t) for t in tensors)
        except TypeError:
            return
        size = _value_bytes(value)
        ids = tuple(i for i, _ in key[0])
        with self._lock:
            # entries of older versions of these same tensors can never hit again
            stale = [k for k in self._entries if k[1] == extra and tuple(i for i, _ in k[0]) == ids and k != key]
            for k in stale:
                self._drop_locked(k)
            if key in self._entries:
                self._drop_locked(key)
            self._entries[key] = (refs, value, size)
            self._bytes += size
            self._evict_locked()
        for t in tensors:
            weakref.finalize(t, self._discard, key)

    def _drop_locked(self, key: tuple) -> None:
        entry = self._entries.pop(key, None)
        if entry is not None:
            self._bytes -= entry[2]

    def _evict_locked(self) -> None:
        while self._entries and (
            len(self._entries) > self.max_entries or (self.max_bytes is not None and self._bytes > self.max_bytes)
        ):
            if len(self._entries) == 1:
                break  # keep the newest entry even when it alone exceeds the byte cap
            self._drop_locked(next(iter(self._entries)))

    def _discard(self, key: tuple) -> None:
        with self._lock:
            self._drop_locked(key)

    def __len__(self) -> int:
        with self._lock:
            return len(self._entries)

    def nbytes(self) -> int:
        with self._lock:
            return self._bytes

    def clear(self) -> None:
        with self._lock:
            self._entries.clear()
            self._bytes = 0


__all__ = ["GraphMemo"]
