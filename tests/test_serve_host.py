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
import torch

from miattn.serve import BlockFreeList, RequestRecord, TraceRequest, _nearest_rank, latency_summary, poisson_trace


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
    n = len(fix["prompts"])
    t = poisson_trace(n, rate=fix["rate"], vocab=151936, seed=fix["seed"])
    assert [list(r.prompt) for r in t] == fix["prompts"]
    assert np.allclose([r.arrival_s for r in t], fix["arrivals"], rtol=0, atol=1e-12)
    assert fix["max_new"] == [(128, 32, 48)[i % 3] for i in range(n)]
    assert [len(x) for x in fix["tokens"]] == fix["max_new"]


# ---- the serving loop's scheduling on the host: a stand-in model and seat decoder that
# compute nothing (a request's next token is a fixed function of the previous one)

VOCAB = 97


def _next(tok: int) -> int:
    return (tok * 31 + 7) % VOCAB


class _FakeModel:
    def new_pool(self, n_blocks, block_size):
        return None

    def prefill(self, prompts, pool, tables):
        for p, t in zip(prompts, tables):
            assert len(t) >= -(-len(p) // 16)
        logits = torch.zeros(len(prompts), VOCAB)
        for i, p in enumerate(prompts):
            logits[i, sum(p) % VOCAB] = 1.0
        return logits


class _FakeSeats:
    """The SeatDecoder interface over host lists: step() advances every admitted seat."""

    instances: list = []

    def __init__(self, model, pool, max_batch, max_blocks, max_new):
        self.table = torch.full((max_batch, max_blocks), -1, dtype=torch.int32)
        self.tok = [None] * max_batch
        self.hist = [[] for _ in range(max_batch)]
        self.active_per_step = []
        _FakeSeats.instances.append(self)

    def capture(self, stream=None):
        pass

    def step(self):
        live = [s for s, t in enumerate(self.tok) if t is not None]
        self.active_per_step.append(len(live))
        for s in live:
            self.tok[s] = _next(self.tok[s])
            self.hist[s].append(self.tok[s])

    def admit(self, seat, blocks, prompt_len, first_token):
        assert self.tok[seat] is None
        self.tok[seat], self.hist[seat] = first_token, []

    def force(self, seats, tokens):
        for s, t in zip(seats, tokens):
            self.tok[s] = t

    def retire(self, seat, n):
        out = self.hist[seat][:n]
        self.tok[seat] = None
        return out

    def check(self):
        pass


@pytest.fixture
def fake_server(monkeypatch):
    from miattn import serve
    monkeypatch.setattr(serve, "SeatDecoder", _FakeSeats)
    monkeypatch.setattr(serve.torch.cuda, "synchronize", lambda *a, **k: None)

    def make(**kw):
        return serve.ContinuousServer(_FakeModel(), **kw)

    return make


def _gate_trace():
    fix = json.loads((Path(__file__).parent / "golden" / "greedy_gate_seed0.json").read_text())["trace"]
    return fix, [TraceRequest(i, a, tuple(p), m)
                 for i, (a, p, m) in enumerate(zip(fix["arrivals"], fix["prompts"], fix["max_new"]))]


def test_gate_trace_schedule_reaches_config5_concurrency(fake_server):
    """The GPU gate's schedule, replayed on the host: on the synthetic clock the fixture's
    16 requests are admitted in small groups while others decode, at least 8 seats decode
    together, short requests retire while long ones go on, and every request gets exactly
    its token budget (free-running: the fake model's own chain of tokens)."""
    fix, trace = _gate_trace()
    server = fake_server(max_batch=32, n_blocks=4096, max_new=128)
    records, wall = server.run(trace, realtime=False, step_s=fix["step_s"])
    assert server.max_active >= 8 and server.admitted_mid_decode >= 8 and server.retired_mid_decode >= 8
    for rec, req in zip(records, trace):
        first = sum(req.prompt) % VOCAB
        chain = [first]
        while len(chain) < req.max_new:
            chain.append(_next(chain[-1]))
        assert rec.tokens == chain
        assert rec.first_token_s >= rec.arrival_s and rec.finish_s > rec.first_token_s
    # deterministic: the same schedule again
    again = fake_server(max_batch=32, n_blocks=4096, max_new=128)
    records2, wall2 = again.run(trace, realtime=False, step_s=fix["step_s"])
    assert wall2 == wall and [r.first_token_s for r in records2] == [r.first_token_s for r in records]
    assert _FakeSeats.instances[-1].active_per_step == _FakeSeats.instances[-2].active_per_step


def test_teacher_forcing_feeds_the_given_tokens_and_records_the_picks(fake_server):
    """Forced: each step's input is the given token, each record holds what the model
    picked from it -- here _next(forced[s - 1]) at step s, the prefill's own pick at 0."""
    fix, trace = _gate_trace()
    forced = {r.idx: [(r.idx * 13 + s * 5) % VOCAB for s in range(r.max_new)] for r in trace}
    server = fake_server(max_batch=32, n_blocks=4096, max_new=128)
    records, _ = server.run(trace, realtime=False, step_s=fix["step_s"], forced=forced)
    for rec, req in zip(records, trace):
        want = [sum(req.prompt) % VOCAB] + [_next(t) for t in forced[req.idx][:req.max_new - 1]]
        assert rec.tokens == want


def test_requests_that_can_never_be_admitted_raise_up_front(fake_server):
    """A request needing more blocks than the whole pool would wait at the queue head
    forever; it (and one beyond the budgets) is refused before anything runs."""
    server = fake_server(max_batch=4, n_blocks=8, max_new=32, max_prompt=512)
    with pytest.raises(ValueError, match="blocks; the pool has 8"):
        server.run([TraceRequest(0, 0.0, tuple(range(200)), 16)], realtime=False)
    with pytest.raises(ValueError, match="max_new 64"):
        server.run([TraceRequest(0, 0.0, (1, 2), 64)], realtime=False)
    with pytest.raises(ValueError, match="exceed a seat"):
        server.run([TraceRequest(0, 0.0, tuple(range(600)), 16)], realtime=False)
    with pytest.raises(ValueError, match="forced tokens"):
        server.run([TraceRequest(0, 0.0, (1, 2), 8)], realtime=False, forced={0: [1, 2]})
    with pytest.raises(ValueError, match="step_s"):
        server.run([TraceRequest(0, 0.0, (1, 2), 8)], step_s=0.01)
    # a pool that fits one request at a time: the second waits for the first's blocks
    records, _ = server.run([TraceRequest(0, 0.0, tuple(range(90)), 20), TraceRequest(1, 0.0, tuple(range(90)), 20)],
                            realtime=False, step_s=0.001)
    assert [len(r.tokens) for r in records] == [20, 20] and records[1].admitted_s >= records[0].finish_s


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
