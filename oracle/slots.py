"""Slot mapping and KV slot-write oracles (numpy, CPU). Test infrastructure only.

Pinned by: the reference tests' known-answer slots (``tests/golden/slot_kats.json``:
reference ``tests/unit/test_paged_kv.py:150-158,464-478``), by the agreement of three
independent formulations below (closed form, per-token loop, per-block slice loop), and by
the invariant that a copy through distinct slots is a bijection (every written row reads
back bit-identical, untouched rows stay unchanged).
"""

from __future__ import annotations

import numpy as np

__all__ = ["slot_ids", "write_tokens", "write_blocks", "gather_tokens"]


def slot_ids(block_table, start: int, length: int, block_size: int) -> np.ndarray:
    """Closed form ``slot(t) = table[t // bs] * bs + t % bs``, t in [start, start+length).

    Follows reference ``model/paged.py:150-168`` (prefill map) and ``:499-501`` (decode map,
    one position per row).
    """
    table = np.asarray(block_table, dtype=np.int64)
    t = np.arange(start, start + length, dtype=np.int64)
    if length and (t[-1] // block_size) >= table.size:
        raise IndexError(f"block table has {table.size} blocks, needs {t[-1] // block_size + 1}")
    return table[t // block_size] * block_size + t % block_size


def write_tokens(pool: np.ndarray, block_table, positions, rows: np.ndarray) -> None:
    """Per-token write: token i goes to ``pool[table[p // bs], p % bs]`` (reference
    ``tests/reference/paged.py:93-124``, the pre-slot-map decode write).

    ``pool`` is ``(n_blocks, bs, H_kv, D)``; ``rows`` is ``(n, H_kv, D)``; a Python loop
    over tokens, for small cases.
    """
    bs = pool.shape[1]
    for i, p in enumerate(positions):
        p = int(p)
        blk = int(block_table[p // bs])
        if not 0 <= blk < pool.shape[0]:
            raise IndexError(f"block id {blk} outside the pool's {pool.shape[0]} blocks")
        pool[blk, p % bs] = rows[i]


def write_blocks(pool: np.ndarray, block_table, start: int, rows: np.ndarray) -> None:
    """Per-block slice write of ``rows`` as logical tokens ``[start, start + n)``
    (reference ``tests/unit/test_paged_kv.py:63-80``)."""
    bs = pool.shape[1]
    written, n = 0, rows.shape[0]
    while written < n:
        p = start + written
        blk = int(block_table[p // bs])
        off = p % bs
        take = min(bs - off, n - written)
        pool[blk, off: off + take] = rows[written: written + take]
        written += take


def gather_tokens(pool: np.ndarray, block_table, length: int) -> np.ndarray:
    """Logical ``(length, H_kv, D)`` view of a request, one token at a time
    (reference ``tests/reference/paged.py:40-90`` minus the zero padding)."""
    bs = pool.shape[1]
    out = np.empty((length,) + pool.shape[2:], dtype=pool.dtype)
    for t in range(length):
        out[t] = pool[int(block_table[t // bs]), t % bs]
    return out
