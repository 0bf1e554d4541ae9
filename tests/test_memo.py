"""The per-graph memo: hits only for the same live, unmodified tensors, drops
entries when a key tensor dies or a newer version is stored, and is capped by
entries and by the bytes of the tensors it holds."""

from __future__ import annotations

import gc

import pytest
import torch

from autosage_amd._memo import GraphMemo


def test_hits_and_misses_follow_identity_and_version():
    memo = GraphMemo("t", max_entries=8)
    a, b = torch.arange(5), torch.arange(5)
    calls = []

    def compute():
        calls.append(1)
        return torch.zeros(3)

    first = memo.get((a,), None, compute)
    assert memo.get((a,), None, compute) is first and len(calls) == 1
    memo.get((b,), None, compute)  # equal values, another tensor: a miss
    assert len(calls) == 2
    memo.get((a,), "other", compute)  # another extra key: a miss
    assert len(calls) == 3
    a.add_(1)  # new version: a miss, and the old versions' entries go
    memo.get((a,), None, compute)
    assert len(calls) == 4
    # (a, None) of the old version is replaced; (b, None) and (a, "other")
    # stay until their tensors die or the cap evicts them
    assert len(memo) == 3


def test_entries_die_with_their_tensors():
    memo = GraphMemo("t", max_entries=8)
    crow, col = torch.arange(4), torch.arange(9)
    memo.get((crow, col), None, lambda: torch.ones(1000))
    assert len(memo) == 1 and memo.nbytes() == 4000
    del col
    gc.collect()
    assert len(memo) == 0 and memo.nbytes() == 0


def test_caps_by_count_and_bytes():
    memo = GraphMemo("t", max_entries=3, max_bytes=10_000)
    keep = [torch.arange(2) for _ in range(6)]
    for t in keep[:4]:
        memo.get((t,), None, lambda: torch.ones(10))
    assert len(memo) == 3  # oldest evicted
    for t in keep[4:]:
        memo.get((t,), None, lambda: torch.ones(2000))  # 8000 bytes each
    assert len(memo) == 1 and memo.nbytes() == 8000  # the newest stays even alone


def test_one_finalizer_per_live_key_tensor():
    """A long-lived key tensor whose version keeps changing (an edge-weight
    parameter updated in place by an optimizer) keeps one finalizer, not one
    per store."""
    memo = GraphMemo("t", max_entries=8)
    weights, cols = torch.ones(10), torch.arange(10)
    for step in range(200):
        weights.add_(1.0)
        memo.get((cols, weights), None, lambda: torch.zeros(4))
    assert len(memo) == 1
    assert memo.finalizer_count() == 2
    # evicted and replaced entries release their finalizers too
    others = [torch.arange(3) for _ in range(20)]
    for t in others:
        memo.get((t,), None, lambda: torch.zeros(1))
    assert len(memo) == 8 and memo.finalizer_count() == 8
    del others
    gc.collect()
    assert memo.finalizer_count() == len(memo) <= 2


def test_entries_keyed_by_a_value_of_another_memo_die_with_it():
    """Derived tensors of one memo (a transposed CSR) key entries of another
    (its plan): dropping the first releases the second, without deadlock."""
    first, second = GraphMemo("a", max_entries=1), GraphMemo("b", max_entries=8)
    k1, k2 = torch.arange(5), torch.arange(6)
    derived = first.get((k1,), None, lambda: torch.arange(7))
    second.get((derived,), None, lambda: torch.zeros(2))
    del derived
    first.get((k2,), None, lambda: torch.arange(8))  # evicts k1's entry, freeing its value
    gc.collect()
    assert len(first) == 1 and len(second) == 0


@pytest.mark.gpu
def test_values_used_on_another_stream_are_recorded_on_it():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    memo = GraphMemo("t")
    key = torch.arange(4, device="cuda")
    memo.get((key,), None, lambda: (torch.ones(1000, device="cuda"), 3))
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        memo.get((key,), None, lambda: pytest.fail("recomputed"))
    streams = next(iter(memo._entries.values()))[3][1]
    assert side in streams and torch.cuda.current_stream() in streams
