"""Pin the slot-map / slot-write oracle against the reference tests' known answers.

The closed form, the per-token loop and the per-block slice loop are three formulations;
each is checked against the transcribed known-answer values and against the others, and
a planted index mistake in the closed form must fail the known answers.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import slots as S

KATS = json.loads((Path(__file__).parent / "golden" / "slot_kats.json").read_text())
H_KV, D = 2, 4


def _rows(n, seed):
    return np.random.default_rng(seed).standard_normal((n, H_KV, D)).astype(np.float32)


def test_prefill_shuffled_table_known_answers():
    case = KATS["prefill_shuffled_table"]
    bs, table = case["block_size"], case["block_table"]
    slots = S.slot_ids(table, case["start"], case["length"], bs)
    for token, block, offset in case["token_to_block_offset"]:
        assert slots[token] == block * bs + offset
    pool = np.zeros((8, bs, H_KV, D), np.float32)
    rows = _rows(case["length"], 1)
    S.write_tokens(pool, table, range(case["length"]), rows)
    for token, block, offset in case["token_to_block_offset"]:
        assert np.array_equal(pool[block, offset], rows[token])
    for block in case["untouched_blocks"]:
        assert not pool[block].any()


def test_decode_boundary_and_rebuilt_container_slots():
    case = KATS["decode_block_boundary"]
    assert S.slot_ids(case["block_table"], case["position"], 1, case["block_size"])[0] == case["slot"]
    rebuilt = KATS["rebuilt_container"]
    for table, position, slot in rebuilt["cases"]:
        assert S.slot_ids(table, position, 1, rebuilt["block_size"])[0] == slot


def test_three_formulations_agree_on_chunked_append():
    case = KATS["chunked_append"]
    bs, table = case["block_size"], case["block_table"]
    a = np.zeros((8, bs, H_KV, D), np.float32)
    b = np.zeros_like(a)
    c = np.zeros_like(a).reshape(-1, H_KV, D)
    chunks = [_rows(n, 10 + i) for i, (_, n) in enumerate(case["chunks"])]
    for (start, n), rows in zip(case["chunks"], chunks):
        S.write_blocks(a, table, start, rows)
        S.write_tokens(b, table, range(start, start + n), rows)
        c[S.slot_ids(table, start, n, bs)] = rows
    assert np.array_equal(a, b) and np.array_equal(a.reshape(-1, H_KV, D), c)
    total = sum(n for _, n in case["chunks"])
    assert np.array_equal(S.gather_tokens(a, table, total), np.concatenate(chunks))


def test_block_size_does_not_change_the_logical_sequence():
    case = KATS["block_size_invariance"]
    rows = _rows(case["length"], 3)
    small = np.zeros((8, 16, H_KV, D), np.float32)
    large = np.zeros((8, 32, H_KV, D), np.float32)
    S.write_blocks(small, case["bs16_table"], 0, rows)
    S.write_blocks(large, case["bs32_table"], 0, rows)
    assert np.array_equal(S.gather_tokens(small, case["bs16_table"], case["length"]),
                          S.gather_tokens(large, case["bs32_table"], case["length"]))


def test_decode_rows_match_the_per_row_reference_write():
    case = KATS["decode_rows"]
    bs = case["block_size"]
    rows = _rows(2, 5)
    by_slot = np.zeros((8 * bs, H_KV, D), np.float32)
    by_row = np.zeros((8, bs, H_KV, D), np.float32)
    for r, (table, pos) in enumerate(zip(case["block_tables"], case["positions"])):
        by_slot[S.slot_ids(table, pos, 1, bs)[0]] = rows[r]
        S.write_tokens(by_row, table, [pos], rows[r:r + 1])
    assert np.array_equal(by_slot, by_row.reshape(-1, H_KV, D))


def test_a_planted_index_mistake_fails_the_known_answers():
    """Swapping // and % (a plausible slip) must not satisfy the transcribed values."""
    case = KATS["prefill_shuffled_table"]
    bs, table = case["block_size"], np.asarray(case["block_table"])
    t = np.arange(case["length"])
    wrong = table[np.minimum(t % len(table), len(table) - 1)] * bs + t // bs
    assert any(wrong[tok] != blk * bs + off for tok, blk, off in case["token_to_block_offset"])


def test_table_too_short_raises():
    with pytest.raises(IndexError):
        S.slot_ids([0], 0, 17, 16)
