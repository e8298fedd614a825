"""Host pieces of the continuous-batching loop (miattn/serve.py): the seeded trace follows the
reference's conventions (reference bench/loadgen.py:201-295: gamma gaps of shape
``burstiness`` and mean 1/rate rescaled to span exactly n/rate seconds from t=0; uniform
ids, reference :87-92), the block free list is all-or-nothing, and the percentile rule is
nearest-rank (reference bench/metrics.py:209-228)."""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from miattn.serve import BlockFreeList, RequestRecord, _nearest_rank, latency_summary, poisson_trace


def test_trace_spans_n_over_rate_from_zero_and_is_seeded():
    t = poisson_trace(50, rate=4.0, vocab=1000, seed=3)
    a = [r.arrival_s for r in t]
    assert a[0] == 0.0 and all(x < y for x, y in zip(a, a[1:]))
    # the last gap ends exactly at n / rate: arrivals[-1] + gap_n == 12.5
    assert a[-1] < 50 / 4.0
    assert [r.prompt for r in poisson_trace(50, rate=4.0, vocab=1000, seed=3)] == [r.prompt for r in t]
    assert [r.prompt for r in poisson_trace(50, rate=4.0, vocab=1000, seed=4)] != [r.prompt for r in t]
    assert all(32 <= len(r.prompt) <= 2048 and max(r.prompt) < 1000 and min(r.prompt) >= 0 for r in t)


def test_trace_gap_and_length_statistics():
    """Poisson (shape 1): gap coefficient of variation 1; shape 4: 1/2; prompt lengths
    lognormal around the median, clipped."""
    for shape, cv in ((1.0, 1.0), (4.0, 0.5)):
        t = poisson_trace(20000, rate=4.0, vocab=10, seed=1, burstiness=shape, median=256)
        a = np.array([r.arrival_s for r in t])
        gaps = np.diff(a)
        assert abs(gaps.std() / gaps.mean() - cv) < 0.03
        assert abs(gaps.mean() - 0.25) < 0.01
        lengths = np.array([len(r.prompt) for r in t])
        assert abs(np.median(lengths) - 256) <= 6 and lengths.min() >= 32 and lengths.max() <= 2048
        assert abs(np.log(lengths).std() - 0.6) < 0.02


def test_gate_fixture_trace_is_this_generator():
    fix = json.loads((Path(__file__).parent / "golden" / "greedy_gate_seed0.json").read_text())["trace"]
    t = poisson_trace(8, rate=fix["rate"], vocab=151936, max_new=fix["max_new"], seed=fix["seed"])
    assert [list(r.prompt) for r in t] == fix["prompts"]
    assert np.allclose([r.arrival_s for r in t], fix["arrivals"], rtol=0, atol=1e-12)


def test_block_free_list_is_all_or_nothing():
    blocks = BlockFreeList(6, 16)
    assert blocks.blocks_for(0) == 1 and blocks.blocks_for(16) == 1 and blocks.blocks_for(17) == 2
    a = blocks.take(4)
    assert a == [0, 1, 2, 3] and blocks.n_free == 2
    assert blocks.take(3) is None and blocks.n_free == 2
    blocks.give_back(a[:2])
    assert blocks.take(3) == [0, 1, 4]


def test_nearest_rank_percentiles_and_summary():
    assert _nearest_rank([5, 1, 3, 2, 4], 0.5) == 3
    assert _nearest_rank([5, 1, 3, 2, 4], 0.95) == 5
    assert _nearest_rank([], 0.5) is None
    rec = RequestRecord(0, 1.0, 10, admitted_s=1.1, first_token_s=1.2, finish_s=2.2, tokens=list(range(11)))
    assert math.isclose(rec.ttft_ms, 200.0) and math.isclose(rec.tpot_ms, 100.0)
    s = latency_summary([rec], 2.0)
    assert s["output_tokens"] == 11 and s["tpot_p50_ms"] == pytest.approx(100.0)
