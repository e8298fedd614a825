"""Continuous-batching serving loop over the HIP attention path (benchmark config 5).

A minimal engine + scheduler, enough to run the reference's online workload end to end:
Poisson arrivals, FIFO packed-group admission, one batched greedy decode step at a time,
retirement at the token budget, blocks returned to the pool. The reference splits this
over ``bench/loadgen.py`` (traces), ``serve/scheduler.py`` (admission, ``step``),
``serve/engine.py`` (``prefill_group``, ``_decode_paged``, ``_sync_paged_cache``) and
``serve/block_manager.py`` (blocks); here it is one loop because only its use of the
attention path is being exercised.

Trace (reference conventions, ``bench/loadgen.py:87-92, 201-295``): ``n`` requests, gamma
inter-arrival gaps of shape ``burstiness`` (1 = Poisson) and mean ``1/rate``, rescaled so
the trace spans exactly ``n/rate`` seconds with the first arrival at 0; prompt lengths
lognormal around a median, rounded and clipped; token ids uniform over the vocabulary.

Admission (reference ``serve/scheduler.py:445-540``, "continuous" policy): before every
decode step, the queue head and the requests behind it that have arrived are admitted in
FIFO order while a seat is free, the group's prompts fit ``max_prefill_tokens`` (a single
longer prompt still forms a group of its own) and the pool holds every member's blocks
(``ceil((prompt + budget) / block_size)`` each); the head is never skipped. The admitted
group runs one packed prefill (``Qwen3.prefill``: ``PackedPrefill`` over the HIP varlen
kernel, one group K/V write per layer); its last-token argmax is each request's first
token. When nothing is active the loop waits for the next arrival.

Decode, MI355X-first: the batch is a fixed set of ``max_batch`` seats and one greedy step of
all of them is captured once in a HIP graph (:class:`SeatDecoder`) and replayed every step.
An idle seat has position -1, which every launch of the step treats as "nothing to do"
(no K/V write, zero-length attention, no token advance); admitting or retiring a request
only rewrites that seat's table row, position and token on the device between replays. The
reference instead rebuilds its ``PagedKV`` whenever the active set changes (``serve/engine.py
:1076-1100``); here nothing is rebuilt or recaptured for the whole trace, and attention cost
follows the active rows' lengths (an idle seat's decode reads nothing).

Timing follows the reference's per-request metrics: TTFT = first token - arrival, TPOT =
(last token - first token) / (tokens - 1); each step ends with one device synchronisation
(as the reference's engine does, ``serve/engine.py:1049-1058``), and its host clock stamps
the tokens it produced.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import numpy as np
import torch

from .decode import paged_decode_plan
from .paged import PagedPool
from .qwen3 import Qwen3, decode_step_begin, greedy_advance, greedy_advance_tiles
from .rows import rows_supported, rows_tile_best

__all__ = ["TraceRequest", "poisson_trace", "BlockFreeList", "SeatDecoder", "ContinuousServer", "RequestRecord",
           "latency_summary"]


@dataclass(frozen=True)
class TraceRequest:
    idx: int
    arrival_s: float
    prompt: tuple
    max_new: int


def poisson_trace(n: int, *, rate: float, vocab: int, median: float = 256, sigma: float = 0.6, lo: int = 32,
                  hi: int = 2048, max_new: int = 128, seed: int = 0, burstiness: float = 1.0) -> list[TraceRequest]:
    """A seeded open-loop trace (see the module docstring for the conventions)."""
    if rate <= 0 or burstiness <= 0 or n < 0:
        raise ValueError("rate and burstiness must be > 0 and n >= 0")
    rng = np.random.default_rng(seed)
    gaps = rng.gamma(burstiness, 1.0 / (rate * burstiness), size=n)
    arrivals = np.concatenate([[0.0], np.cumsum(gaps)[:-1]]) * ((n / rate) / gaps.sum()) if n else np.zeros(0)
    lengths = np.clip(np.rint(rng.lognormal(math.log(median), sigma, size=n)), lo, hi).astype(int)
    prompts = [tuple(int(t) for t in rng.integers(0, vocab, size=int(m))) for m in lengths]
    return [TraceRequest(i, float(arrivals[i]), prompts[i], int(max_new)) for i in range(n)]


class BlockFreeList:
    """Physical block ids of one pool: a request takes all its blocks or none; freed ids go
    back to the front, so a pool that cycles through short requests keeps reusing the
    same low blocks."""

    def __init__(self, n_blocks: int, block_size: int) -> None:
        self.block_size = int(block_size)
        self._free = list(range(n_blocks - 1, -1, -1))  # pop() hands out 0, 1, 2, ...

    @property
    def n_free(self) -> int:
        return len(self._free)

    def blocks_for(self, tokens: int) -> int:
        return max(1, -(-int(tokens) // self.block_size))

    def take(self, count: int) -> list[int] | None:
        if count > len(self._free):
            return None
        return [self._free.pop() for _ in range(count)]

    def give_back(self, blocks: list[int]) -> None:
        self._free.extend(reversed(blocks))


class SeatDecoder:
    """One greedy decode step of ``max_batch`` seats, captured once as a HIP graph.

    Per seat on the device: block-table row (int32, -1 past the seat's blocks), position
    (int64, -1 when idle), next input token, step count and the tokens produced. The step's
    launches are those of :class:`~miattn.qwen3.GraphDecoder` (step begin, 28 layers of HIP
    projections, fused epilogue and paged decode, lm_head with per-tile picks, greedy
    advance), each of which leaves idle seats untouched.
    """

    def __init__(self, model: Qwen3, pool: PagedPool, max_batch: int, max_blocks: int, max_new: int) -> None:
        c, dev = model.cfg, model.device
        self.model, self.pool = model, pool
        self.S = int(max_batch)
        self.table = torch.full((self.S, max_blocks), -1, dtype=torch.int32, device=dev)
        self.pos = torch.full((self.S,), -1, dtype=torch.long, device=dev)
        self.tokens = torch.zeros(self.S, dtype=torch.long, device=dev)
        self.steps = torch.zeros(self.S, dtype=torch.long, device=dev)
        self.history = torch.zeros(self.S, max_new, dtype=torch.long, device=dev)
        self.seqlen = torch.zeros(self.S, dtype=torch.int32, device=dev)
        self.slots = torch.full((self.S,), -1, dtype=torch.long, device=dev)
        self.error = torch.zeros(1, dtype=torch.int32, device=dev)
        self.x = torch.empty(self.S, c.hidden, dtype=model.dtype, device=dev)
        self.h0 = torch.empty_like(self.x)
        q0 = torch.zeros(self.S, c.n_head, c.head_dim, dtype=model.dtype, device=dev)
        self.plan = paged_decode_plan(q0, pool.keys, pool.values, self.table, self.seqlen,
                                      scale=1.0 / math.sqrt(c.head_dim))
        # q/k norm + RoPE + K/V write fused into the decode launch where the shape allows
        self.fused = self.plan.fused_supported(model.dtype, 2 * int(model.cos.shape[-1]))
        self.graph = None

    def _step(self) -> None:
        m, c = self.model, self.model.cfg
        decode_step_begin(self.tokens, self.pos, self.table, self.pool.block_size, m.w["embed"], m.w["l0.ln1"],
                          c.eps, self.seqlen, self.slots, self.x, self.h0, self.error)

        def attend(i: int, qkv) -> torch.Tensor:
            p = f"l{i}."
            # idle seats: slot -1 and seqlen 0, nothing written or attended
            if self.fused:
                return self.plan.run_fused(i, qkv, m.w[p + "qn"], m.w[p + "kn"], m.cos, m.sin, self.pos, self.slots,
                                           c.eps, error_word=self.pool.write_error_word).view(self.S, -1)
            q = self.pool.write_qk_norm_rope(i, self.slots, qkv, m.w[p + "qn"], m.w[p + "kn"], m.cos, m.sin,
                                             self.pos, c.eps)
            return self.plan.run(i, q).view(self.S, -1)

        h = m._decode_stack(self.x, attend, self.h0)
        w = m.w["embed"]
        if rows_supported(h, w) and h.shape[1] <= 1024:
            greedy_advance_tiles(rows_tile_best(h, w), self.tokens, self.pos, self.history, self.steps)
        else:
            greedy_advance(m._lm_head(h), self.tokens, self.pos, self.history, self.steps)

    def capture(self, stream=None) -> None:
        """Record the step; run once first (all seats idle) so lazily built state exists."""
        self._step()
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self._step()
        torch.cuda.synchronize()

    def step(self) -> None:
        self._step() if self.graph is None else self.graph.replay()

    def admit(self, seat: int, blocks: list[int], prompt_len: int, first_token: int) -> None:
        row = torch.full((self.table.shape[1],), -1, dtype=torch.int32)
        row[: len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
        self.table[seat].copy_(row)
        self.pos[seat] = prompt_len
        self.tokens[seat] = first_token
        self.steps[seat] = 0

    def force(self, seats: list[int], tokens: list[int]) -> None:
        """Replace the named seats' next input tokens (teacher forcing); the picks already
        recorded in the history stay as the step produced them."""
        idx = torch.tensor(seats, dtype=torch.long)
        self.tokens.index_put_((idx.to(self.tokens.device),),
                               torch.tensor(tokens, dtype=torch.long).to(self.tokens.device))

    def retire(self, seat: int, n_tokens: int) -> list[int]:
        """The seat's decode tokens (one device read) and the seat made idle."""
        out = self.history[seat, :n_tokens].tolist()
        self.pos[seat] = -1
        self.table[seat].fill_(-1)
        return out

    def check(self) -> None:
        bad = int(self.error.item())
        if bad:
            self.error.zero_()
            raise IndexError(f"seat {bad - 1}: token or position out of range in a decode step")
        self.pool.check_writes()


@dataclass
class RequestRecord:
    idx: int
    arrival_s: float
    prompt_len: int
    admitted_s: float = float("nan")
    first_token_s: float = float("nan")
    finish_s: float = float("nan")
    tokens: list = field(default_factory=list)

    @property
    def ttft_ms(self) -> float:
        return (self.first_token_s - self.arrival_s) * 1e3

    @property
    def tpot_ms(self) -> float:
        n = len(self.tokens)
        return (self.finish_s - self.first_token_s) * 1e3 / (n - 1) if n > 1 else float("nan")


def _nearest_rank(values, q: float):
    """Nearest-rank percentile (the reference's rule, ``bench/metrics.py:209-228``)."""
    vals = sorted(v for v in values if v == v)
    if not vals:
        return None
    return vals[min(len(vals) - 1, max(0, math.ceil(q * len(vals)) - 1))]


def latency_summary(records: list[RequestRecord], wall_s: float) -> dict:
    tokens = sum(len(r.tokens) for r in records)
    ttft = [r.ttft_ms for r in records]
    tpot = [r.tpot_ms for r in records]
    return {
        "requests": len(records),
        "output_tokens": tokens,
        "wall_s": wall_s,
        "output_tokens_per_s": tokens / wall_s if wall_s > 0 else None,
        "ttft_p50_ms": _nearest_rank(ttft, 0.5), "ttft_p95_ms": _nearest_rank(ttft, 0.95),
        "tpot_p50_ms": _nearest_rank(tpot, 0.5), "tpot_p95_ms": _nearest_rank(tpot, 0.95),
    }


class ContinuousServer:
    """The loop of the module docstring over one model, pool and seat decoder."""

    def __init__(self, model: Qwen3, *, max_batch: int = 32, n_blocks: int = 8192, block_size: int = 16,
                 max_prompt: int = 2048, max_new: int = 128, max_prefill_tokens: int = 8192, stream=None) -> None:
        self.model = model
        self.pool = model.new_pool(n_blocks, block_size)
        self.blocks = BlockFreeList(n_blocks, block_size)
        self.max_batch = int(max_batch)
        self.max_new = int(max_new)
        self.max_prefill_tokens = int(max_prefill_tokens)
        self.seats = SeatDecoder(model, self.pool, max_batch, self.blocks.blocks_for(max_prompt + max_new), max_new)
        self.stream = stream
        self.n_blocks = int(n_blocks)
        self.steps_run = 0
        # concurrency seen by the last run(): the most seats active in one decode step,
        # admissions made while other requests were decoding, and retirements that left
        # other requests decoding
        self.max_active = 0
        self.admitted_mid_decode = 0
        self.retired_mid_decode = 0

    def warm(self) -> None:
        """Capture the step graph and run one throwaway prefill (GEMM algorithm choice,
        allocator growth) so the first real request does not pay for them."""
        self.seats.capture(self.stream)
        blocks = self.blocks.take(self.blocks.blocks_for(64))
        self.model.prefill([[1] * 64], self.pool, [blocks])
        self.blocks.give_back(blocks)
        torch.cuda.synchronize()

    def run(self, trace: list[TraceRequest], *, realtime: bool = True, step_s: float | None = None,
            forced: dict | None = None) -> tuple[list[RequestRecord], float]:
        """Serve ``trace``; returns the per-request records and the wall time.

        ``realtime=False`` replays the same schedule on a virtual clock: instead of
        sleeping until the next arrival when nothing is active, the clock jumps to it (the
        GPU work and its timing are unchanged; tests use this). ``step_s`` (virtual clock
        only) makes the clock fully synthetic: each prefill group and each decode step
        advances it by ``step_s`` seconds, so admissions and retirements follow the trace
        deterministically, whatever the GPU's speed.

        ``forced`` (request idx -> tokens, at least ``max_new`` of them) runs the requests
        teacher-forced: every step's input token is the given one rather than the previous
        pick, while each record still holds the picks the GPU made. A token-by-token
        comparison against another implementation's greedy tokens then compares every
        step on the same context, not just the prefix before a first divergence.

        A request that could never be admitted -- more blocks than the whole pool, or past
        the prompt / token budget the seats were sized for -- raises ``ValueError`` before
        anything runs."""
        if step_s is not None and (realtime or step_s <= 0):
            raise ValueError("step_s needs realtime=False and a positive step")
        for r in trace:
            if r.max_new < 1 or r.max_new > self.max_new:
                raise ValueError(f"request {r.idx}: max_new {r.max_new} outside [1, {self.max_new}]")
            if len(r.prompt) + r.max_new > self.seats.table.shape[1] * self.blocks.block_size:
                raise ValueError(f"request {r.idx}: {len(r.prompt)} + {r.max_new} tokens exceed a seat's "
                                 f"{self.seats.table.shape[1] * self.blocks.block_size} positions")
            if self.blocks.blocks_for(len(r.prompt) + r.max_new) > self.n_blocks:
                raise ValueError(f"request {r.idx} needs {self.blocks.blocks_for(len(r.prompt) + r.max_new)} "
                                 f"blocks; the pool has {self.n_blocks}")
            if forced is not None and len(forced.get(r.idx, ())) < r.max_new:
                raise ValueError(f"request {r.idx}: forced tokens must cover its {r.max_new} tokens")
        records = {r.idx: RequestRecord(r.idx, r.arrival_s, len(r.prompt)) for r in trace}
        queue = sorted(trace, key=lambda r: (r.arrival_s, r.idx))
        free_seats = list(range(self.max_batch - 1, -1, -1))
        active: dict[int, tuple[TraceRequest, list[int], int]] = {}  # seat -> (request, blocks, tokens so far)
        skew = 0.0  # virtual-clock offset (the whole clock when step_s is given)
        t0 = time.perf_counter()
        self.max_active = self.admitted_mid_decode = self.retired_mid_decode = 0

        def now() -> float:
            return skew if step_s is not None else time.perf_counter() - t0 + skew

        head = 0
        while head < len(queue) or active:
            # ---- admission: one FIFO group, before the step
            group = []
            tokens = 0
            while head < len(queue) and len(active) + len(group) < self.max_batch:
                req = queue[head]
                if req.arrival_s > now():
                    if active or group:
                        break
                    wait = req.arrival_s - now()
                    if realtime:
                        time.sleep(max(0.0, wait))
                    else:
                        skew += max(0.0, wait)
                    continue
                if group and tokens + len(req.prompt) > self.max_prefill_tokens:
                    break
                blocks = self.blocks.take(self.blocks.blocks_for(len(req.prompt) + req.max_new))
                if blocks is None:
                    break  # the head waits for blocks; it is never skipped
                group.append((req, blocks))
                tokens += len(req.prompt)
                head += 1
            if group:
                if active:
                    self.admitted_mid_decode += len(group)
                t_admit = now()
                logits = self.model.prefill([list(r.prompt) for r, _ in group], self.pool, [b for _, b in group])
                first = logits.argmax(-1)
                torch.cuda.synchronize()
                if step_s is not None:
                    skew += step_s
                t_first = now()
                first_host = first.tolist()
                for (req, blocks), tok in zip(group, first_host):
                    seat = free_seats.pop()
                    self.seats.admit(seat, blocks, len(req.prompt), tok if forced is None else forced[req.idx][0])
                    rec = records[req.idx]
                    rec.admitted_s, rec.first_token_s, rec.tokens = t_admit, t_first, [tok]
                    active[seat] = (req, blocks, 1)
                    if req.max_new == 1:
                        self._finish(seat, active, free_seats, records, t_first)
            if not active:
                continue
            # ---- one decode step of every seat
            self.max_active = max(self.max_active, len(active))
            self.seats.step()
            torch.cuda.synchronize()
            if step_s is not None:
                skew += step_s
            t_step = now()
            self.steps_run += 1
            force_seats, force_tokens = [], []
            for seat in list(active):
                req, blocks, n = active[seat]
                active[seat] = (req, blocks, n + 1)
                if n + 1 == req.max_new:
                    self._finish(seat, active, free_seats, records, t_step)
                    if active:
                        self.retired_mid_decode += 1
                elif forced is not None:
                    force_seats.append(seat)
                    force_tokens.append(forced[req.idx][n])
            if force_seats:
                self.seats.force(force_seats, force_tokens)
        self.seats.check()
        wall = skew if step_s is not None else time.perf_counter() - t0 + skew
        return [records[r.idx] for r in trace], wall

    def _finish(self, seat, active, free_seats, records, t) -> None:
        req, blocks, n = active.pop(seat)
        rec = records[req.idx]
        rec.tokens = rec.tokens[:1] + self.seats.retire(seat, n - 1)
        rec.finish_s = t
        self.blocks.give_back(blocks)
        free_seats.append(seat)
