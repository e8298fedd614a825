"""Paged-KV block allocator: produces the block tables the HIP kernels index.

Same semantics as the reference's ``BlockManager`` (reference
``serve/block_manager.py:32-143``), which is what makes its block tables valid kernel
inputs: ids are handed out smallest-first (deterministic tables for tests and the
capacity simulation), ``reserve(n)`` is all-or-nothing, ``free`` validates the whole call
before changing anything, and ``blocks_for(prompt, budget)`` reserves
``max(1, ceil((prompt + budget) / block_size))`` blocks up front so decode never needs a
mid-request allocation. Blocks are opaque integers here; ``PagedPool`` maps them to bytes.
"""

from __future__ import annotations

import heapq
from typing import Sequence

__all__ = ["BlockManager"]


def _nonneg_int(name: str, value) -> int:
    if not isinstance(value, int) or isinstance(value, bool) or value < 0:
        raise ValueError(f"{name} must be a non-negative int, got {value!r}")
    return value


class BlockManager:
    """Deterministic free list of ``n_blocks`` physical blocks of ``block_size`` tokens."""

    def __init__(self, n_blocks: int, block_size: int) -> None:
        for name, value in (("n_blocks", n_blocks), ("block_size", block_size)):
            if not isinstance(value, int) or isinstance(value, bool) or value < 1:
                raise ValueError(f"{name} must be a positive int, got {value!r}")
        self.n_blocks = n_blocks
        self.block_size = block_size
        self._heap = list(range(n_blocks))  # already a valid min-heap
        self._held: set[int] = set()
        self._peak = 0
        self._alloc_calls = 0
        self._free_calls = 0

    def reserve(self, n: int) -> list[int] | None:
        """``n`` distinct ids, smallest first, or ``None`` with nothing consumed."""
        n = _nonneg_int("n", n)
        if n > len(self._heap):
            return None
        if n == 0:
            return []
        ids = [heapq.heappop(self._heap) for _ in range(n)]
        self._held.update(ids)
        self._alloc_calls += 1
        self._peak = max(self._peak, len(self._held))
        return ids

    def free(self, ids: Sequence[int]) -> None:
        """Return ids; the whole call is validated first (no partial frees)."""
        batch: set[int] = set()
        for block_id in ids:
            if not isinstance(block_id, int) or isinstance(block_id, bool):
                raise ValueError(f"block ids must be ints, got {block_id!r}")
            if block_id in batch:
                raise ValueError(f"duplicate block id {block_id} in one free call")
            if block_id not in self._held:
                raise ValueError(f"block {block_id} is not allocated")
            batch.add(block_id)
        if not batch:
            return
        self._held -= batch
        for block_id in batch:
            heapq.heappush(self._heap, block_id)
        self._free_calls += 1

    @property
    def in_use(self) -> int:
        return len(self._held)

    @property
    def peak(self) -> int:
        return self._peak

    def stats(self) -> dict:
        in_use = len(self._held)
        return {
            "n_blocks": self.n_blocks, "block_size": self.block_size, "in_use": in_use,
            "free": len(self._heap), "reserved": in_use, "peak": self._peak,
            "alloc_calls": self._alloc_calls, "free_calls": self._free_calls,
        }

    def blocks_for(self, prompt_len: int, budget: int) -> int:
        prompt_len = _nonneg_int("prompt_len", prompt_len)
        budget = _nonneg_int("budget", budget)
        return max(1, -(-(prompt_len + budget) // self.block_size))
