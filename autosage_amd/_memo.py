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
  its values hold (least recently used first);
* a value's device tensors come from PyTorch's caching allocator on the
  stream that was current when they were built; when a later call uses them
  on another stream, ``get`` records them on that stream
  (``Tensor.record_stream``), so that a dropped entry's blocks are not
  handed to a new allocation while a kernel there still reads them.

Thread-safe; the derived values must not hold references to the key tensors
(that would keep them alive and the entry with them).  One finalizer is
registered per live key tensor, whatever the number of entries it keys.
"""

from __future__ import annotations

import collections
import threading
import weakref
from typing import Any, Callable, Hashable, Sequence

import torch


def _device_tensors(value: Any) -> list:
    if isinstance(value, torch.Tensor):
        return [value] if value.is_cuda else []
    if isinstance(value, (tuple, list)):
        return [t for v in value for t in _device_tensors(v)]
    if isinstance(value, dict):
        return [t for v in value.values() for t in _device_tensors(v)]
    return []


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
        # reentrant: a key tensor can die (and its finalizer run) while this
        # thread holds the lock, when dropping an entry frees the last
        # reference to it
        self._lock = threading.RLock()
        # key -> (weak refs, value, bytes, streams the value is recorded on)
        self._entries: "collections.OrderedDict[tuple, tuple]" = collections.OrderedDict()
        self._bytes = 0
        # id of a live key tensor -> (its finalizer, the keys it is part of)
        self._finalizers: dict[int, tuple] = {}

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
                self._record_stream_locked(hit)
                return hit[1]
        value = compute()
        self.put(tensors, extra, value, key=key)
        return value

    @staticmethod
    def _current_stream(device: torch.device):
        return torch.cuda.current_stream(device)

    def _record_stream_locked(self, entry: tuple) -> None:
        """Records the value's device tensors on the current stream of their
        device when it is not one they are already recorded on."""
        device_tensors, streams = entry[3]
        if not device_tensors:
            return
        stream = self._current_stream(device_tensors[0].device)
        if stream in streams:
            return
        for t in device_tensors:
            t.record_stream(stream)
        streams.add(stream)

    def put(self, tensors: Sequence[torch.Tensor], extra: Hashable, value: Any, *, key: tuple | None = None) -> None:
        key = key if key is not None else self._key(tensors, extra)
        try:
            refs = tuple(weakref.ref(t) for t in tensors)
        except TypeError:
            return
        size = _value_bytes(value)
        device_tensors = _device_tensors(value)
        # the stream the value was built on: its blocks belong to it already
        streams = {self._current_stream(device_tensors[0].device)} if device_tensors else set()
        ids = tuple(i for i, _ in key[0])
        with self._lock:
            # entries of older versions of these same tensors can never hit again
            stale = [k for k in self._entries if k[1] == extra and tuple(i for i, _ in k[0]) == ids and k != key]
            for k in stale:
                self._drop_locked(k)
            if key in self._entries:
                self._drop_locked(key)
            self._entries[key] = (refs, value, size, (device_tensors, streams))
            self._bytes += size
            for t in tensors:
                handle = self._finalizers.get(id(t))
                if handle is None or not handle[0].alive:
                    handle = (weakref.finalize(t, self._discard_tensor, id(t)), set())
                    self._finalizers[id(t)] = handle
                handle[1].add(key)
            self._evict_locked()

    def _drop_locked(self, key: tuple) -> None:
        entry = self._entries.pop(key, None)
        if entry is None:
            return
        self._bytes -= entry[2]
        # a key tensor that keys no entry any more needs no finalizer
        for tid in {i for i, _ in key[0]}:
            handle = self._finalizers.get(tid)
            if handle is not None:
                handle[1].discard(key)
                if not handle[1]:
                    handle[0].detach()
                    del self._finalizers[tid]

    def _evict_locked(self) -> None:
        while self._entries and (
            len(self._entries) > self.max_entries or (self.max_bytes is not None and self._bytes > self.max_bytes)
        ):
            if len(self._entries) == 1:
                break  # keep the newest entry even when it alone exceeds the byte cap
            self._drop_locked(next(iter(self._entries)))

    def _discard_tensor(self, tid: int) -> None:
        """A key tensor died: every entry it keys goes."""
        with self._lock:
            handle = self._finalizers.pop(tid, None)
            if handle is None:
                return
            for key in list(handle[1]):
                self._drop_locked(key)

    def __len__(self) -> int:
        with self._lock:
            return len(self._entries)

    def nbytes(self) -> int:
        with self._lock:
            return self._bytes

    def finalizer_count(self) -> int:
        with self._lock:
            return len(self._finalizers)

    def clear(self) -> None:
        with self._lock:
            for handle, _ in self._finalizers.values():
                handle.detach()
            self._finalizers.clear()
            self._entries.clear()
            self._bytes = 0


__all__ = ["GraphMemo"]
