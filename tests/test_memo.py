"""The per-graph memo: hits only for the same live, unmodified tensors, drops
entries when a key tensor dies or a newer version is stored, and is capped by
entries and by the bytes of the tensors it holds."""

from __future__ import annotations

import gc

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
