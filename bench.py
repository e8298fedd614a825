#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path; prints ONE JSON line.

Headline (``value``): paged-decode attention HBM throughput on config 2 -- Qwen3-0.6B
attention shape (16/8 heads, D=128, bf16, block size 16), B=32 rows with context lengths
uniform in [128, 2048], an 8192-block pool per layer, 28 layers run back to back. One
step = the 28 layers' ``PagedDecodePlan.run`` calls (the engine's per-layer decode
launch), captured once in a HIP graph and replayed, so the number is GPU time rather
than Python launch overhead; the eager (un-captured) step time is reported beside it.
Algorithmic bytes per layer = sum(seqlen) * 2 * H_kv * D * 2 B (K and V read once per KV
head) + q and out (2 * B * H * D * 2 B) + seqlen + block table.

Extra fields: packed prefill (config 3) TFLOP/s against bf16 MFMA peak, also at the
Qwen3.5 attention shape (H 8 / H_kv 2 / head_dim 256) and for one 8192-token segment
(``prefill_long``, the default kernel there), the packed KV slot write (config 3) GB/s,
long-context split-K decode (config 4), decode at the Qwen3.5 shape on the config-2 lengths
(``decode_qwen35``), and the CPU baseline:
the reference's seat path (contiguous slab + baddbmm decode, bf16 softmax) timed on this
host's cores on one layer of the same config-2 inputs, after checking the GPU output
against it.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "llm-serving_amd"))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
METRIC = "paged-decode attn HBM GB/s (% peak) + TPOT ms, Qwen3-0.6B B=32 ctx2048"
N_LAYER = 28
WARM_MS = 300.0  # untimed replays before each timed graph block


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def percentile(values, q):
    vals = sorted(values)
    if not vals:
        return None
    return vals[min(len(vals) - 1, max(0, math.ceil(q * len(vals)) - 1))]


class EventTimer:
    """HIP events on the stream the kernels run on (torch's current stream)."""

    def __init__(self, stream):
        self.stream = stream
        self.start = torch.cuda.Event(enable_timing=True)
        self.end = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.start.record(self.stream)
        return self

    def __exit__(self, *exc):
        self.end.record(self.stream)

    def ms(self) -> float:
        self.end.synchronize()
        return self.start.elapsed_time(self.end)


def time_graph(step, stream, steps: int, warmup: int):
    """Capture ``step`` (a Python function that launches one step's kernels) into a HIP
    graph on ``stream`` and time ``steps`` replays with events on that stream.

    Returns (ms per step over the timed block, per-replay samples in ms)."""
    with torch.cuda.stream(stream):
        step()  # warm caches (schedules, workspaces) outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    samples = []
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            graph.replay()
        # then at least WARM_MS of untimed replays: a short graph (one prefill step is under
        # a millisecond) would otherwise be timed while the clocks are still ramping
        with EventTimer(stream) as one:
            graph.replay()
        for _ in range(int(WARM_MS / max(one.ms(), 1e-3))):
            graph.replay()
        torch.cuda.synchronize()
        with EventTimer(stream) as total:
            for _ in range(steps):
                graph.replay()
        total_ms = total.ms()
        for _ in range(min(steps, 50)):
            with EventTimer(stream) as t:
                graph.replay()
            samples.append(t.ms())
    torch.cuda.synchronize()
    return total_ms / steps, samples


def decode_bytes(lengths, B, H, H_kv, D, max_blocks, esize=2) -> int:
    kv = sum(lengths) * 2 * H_kv * D * esize
    qo = 2 * B * H * D * esize
    meta = B * 4 + B * max_blocks * 4
    return kv + qo + meta


def bench_decode(inp, steps: int, warmup: int, stream, eager: bool = False, check_rows=None):
    """Time 28-layer decode steps; layer 0's output rows ``check_rows`` (default: all) are
    checked against the fp32 oracle after the warm-up and before the timed region."""
    from miattn import paged_decode_plan

    B, H, D = inp.q[0].shape
    H_kv = inp.k_caches[0].shape[2]
    plan = paged_decode_plan(inp.q[0], inp.k_caches, inp.v_caches, inp.block_table, inp.seqlen)
    outs = [None] * N_LAYER

    def step():
        for layer in range(N_LAYER):
            outs[layer] = plan.run(layer, inp.q[layer])

    # eager step (Python launch path), for reference
    with torch.cuda.stream(stream):
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(10 if not eager else steps):
            step()
        torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / (10 if not eager else steps)
    checked = check_decode_rows(inp, outs[0], list(range(B)) if check_rows is None else check_rows)
    nbytes = decode_bytes(inp.lengths, B, H, H_kv, D, inp.block_table.shape[1])
    if eager:
        ms_per_step, per_step = eager_ms, [eager_ms]
    else:
        ms_per_step, per_step = time_graph(step, stream, steps, warmup)
    return {
        "ms_per_step": ms_per_step,
        "eager_ms_per_step": eager_ms,
        "p50_ms": percentile(per_step, 0.5),
        "p95_ms": percentile(per_step, 0.95),
        "bytes_per_layer": nbytes,
        "us_per_layer": ms_per_step * 1e3 / N_LAYER,
        "gbs": nbytes * N_LAYER / (ms_per_step * 1e-3) / 1e9,
        "out0": outs[0],
        "checked_max_abs_diff": checked,
    }


def bench_prefill(stream, steps: int = 20, eager: bool = False):
    """Config 3: packed varlen prefill (28 layer calls on one packed group) and the packed
    group's KV slot write (28 layers), each captured in a HIP graph and replayed."""
    from miattn import HipVarlen, PackedPrefill, PagedPool, PagedWriteSink
    from miattn import workloads as W

    from oracle.varlen import longhand_varlen

    inp = W.prefill_config3(device="cuda")
    backend = HipVarlen()
    H, D = inp.q.shape[1], inp.q.shape[2]
    flop = 4 * H * D * sum(n * (n + 1) // 2 for n in inp.lengths)  # causal pairs incl. diagonal
    ms = max(inp.lengths)
    # checked against the fp32 longhand oracle before it is timed
    got = backend.prefill_varlen(inp.q, inp.k, inp.v, cu_seqlens=inp.cu_seqlens, max_seqlen=ms).cpu().float()
    prefill_diff = (got - longhand_varlen(inp.q.cpu(), inp.k.cpu(), inp.v.cpu(), inp.cu_seqlens)).abs().max().item()
    if not prefill_diff <= 2e-2:
        raise SystemExit(f"packed prefill disagrees with the oracle: max|delta|={prefill_diff}")

    def prefill_step():
        for _ in range(N_LAYER):
            backend.prefill_varlen(inp.q, inp.k, inp.v, cu_seqlens=inp.cu_seqlens, max_seqlen=ms)

    if eager:  # plain dispatches, for counter collection
        with torch.cuda.stream(stream):
            for _ in range(2):
                prefill_step()
            torch.cuda.synchronize()
            with EventTimer(stream) as t:
                prefill_step()
            prefill_step_ms = t.ms()
    else:
        prefill_step_ms, _ = time_graph(prefill_step, stream, steps, 3)
    prefill_ms = prefill_step_ms / N_LAYER
    tflops = flop / (prefill_ms * 1e-3) / 1e12

    pool = PagedPool(N_LAYER, inp.n_blocks, inp.block_size, inp.k.shape[1], D, dtype=torch.bfloat16,
                     device="cuda", n_head=H)
    positions = torch.cat([torch.arange(n) for n in inp.lengths]).cuda()
    sinks = [PagedWriteSink(pool, t_, n) for t_, n in zip(inp.tables, inp.lengths)]
    packed = PackedPrefill(cu_seqlens=inp.cu_seqlens, positions=positions, sinks=sinks, backend=backend)
    slots = packed.group_slots
    # distinct K/V sources per layer, so no layer's write reads what the previous one cached
    ks = [torch.randn_like(inp.k) for _ in range(N_LAYER)]
    vs = [torch.randn_like(inp.v) for _ in range(N_LAYER)]

    def write_step():
        for layer in range(N_LAYER):
            pool.write_prefill_slots(layer, slots, ks[layer], vs[layer])

    # bit-exact before it is timed: every written slot row equals its source row
    write_step()
    pool.check_writes()
    for layer in (0, N_LAYER - 1):
        flat_k = pool.keys[layer].view(-1, *ks[layer].shape[1:])
        flat_v = pool.values[layer].view(-1, *vs[layer].shape[1:])
        if not (torch.equal(flat_k[slots], ks[layer]) and torch.equal(flat_v[slots], vs[layer])):
            raise SystemExit(f"packed slot write is not bit-exact on layer {layer}")

    if eager:
        with torch.cuda.stream(stream):
            write_step()
            torch.cuda.synchronize()
            with EventTimer(stream) as t:
                write_step()
            write_step_ms = t.ms()
    else:
        # a write step is ~0.25 ms: at least 100 replays, so the figure is not a few ms of
        # samples
        write_step_ms, _ = time_graph(write_step, stream, max(steps, 100), 3)
    pool.check_writes()
    write_ms = write_step_ms / N_LAYER
    write_bytes = 2 * 2 * sum(inp.lengths) * inp.k.shape[1] * D * 2 + sum(inp.lengths) * 8
    return {
        "workload": "config3: 8 prompts lognormal(median 512, sigma 0.6) clip [64,2048], H16/8 D128 bf16",
        "lengths": inp.lengths,
        "prefill_us_per_layer": prefill_ms * 1e3,
        "prefill_tflops": tflops,
        "prefill_frac_mfma_peak": tflops / BF16_MFMA_PEAK_TFLOPS,
        # tokens through one forward's attention (28 layer calls), not one layer call
        "prefill_attention_tokens_per_s_per_forward": sum(inp.lengths) / (N_LAYER * prefill_ms * 1e-3),
        "flop_per_layer": flop,
        "slot_write_us_per_layer": write_ms * 1e3,
        "slot_write_gbs": write_bytes / (write_ms * 1e-3) / 1e9,
        "slot_write_frac_hbm_peak": write_bytes / (write_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "slot_write_bytes_per_layer": write_bytes,
        "checked": {"prefill_max_abs_diff_vs_fp32_oracle": prefill_diff, "slot_write_bit_exact": True},
    }


def bench_tpot(stream, prompt_len: int = 1920, new_tokens: int = 128, B: int = 32, seed: int = 0) -> dict:
    """Config 5 shape, closed batch: random-init Qwen3-0.6B, B rows of ``prompt_len`` random
    tokens prefilled in one packed group, then ``new_tokens`` greedy decode steps (context
    ``prompt_len`` -> ``prompt_len + new_tokens``). TPOT = GPU time of one whole decode step
    (step start: slots, seqlen, embedding, layer-0 norm; 28 layers: rows-GEMM projections, the
    q/k-norm + RoPE + K/V write epilogue, paged decode + merge, residual add + RMSNorm,
    gate/up + SiLU * up; lm_head with per-tile greedy picks; the pick and position advance --
    all HIP launches), replayed from one HIP graph; the eager (Python-launched) step is
    reported too."""
    from miattn import PagedKV
    from miattn.qwen3 import GraphDecoder, Qwen3, Qwen3Config, random_weights

    cfg = Qwen3Config()
    model = Qwen3(cfg, random_weights(cfg, seed), "cuda")
    gen = torch.Generator().manual_seed(seed + 1)
    prompts = [torch.randint(0, cfg.vocab, (prompt_len,), generator=gen).tolist() for _ in range(B)]
    bs = 16
    per = (prompt_len + new_tokens + 1 + bs - 1) // bs
    n_blocks = max(8192, B * per)
    perm = torch.randperm(n_blocks, generator=torch.Generator().manual_seed(seed + 2)).tolist()
    tables = [perm[r * per:(r + 1) * per] for r in range(B)]
    pool = model.new_pool(n_blocks, bs)
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        # the first prefill pays one-time costs (GEMM algorithm selection, the prefill
        # schedule, allocator growth); the second, into the same slots, is the TTFT figure
        with EventTimer(stream) as t:
            model.prefill(prompts, pool, tables)
        prefill_cold_ms = t.ms()
        with EventTimer(stream) as t:
            logits = model.prefill(prompts, pool, tables)
        prefill_ms = t.ms()
        first = logits.argmax(-1)
        # eager steps on a copy of the state (PagedKV, Python launch path)
        paged = PagedKV(pool, tables, [prompt_len] * B, rope_len=prompt_len + new_tokens + 1, n_head=cfg.n_head)
        tok = first
        for _ in range(2):
            tok = model.decode(paged, tok).argmax(-1)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(8):
            tok = model.decode(paged, tok).argmax(-1)
        torch.cuda.synchronize()
        eager_ms = (time.perf_counter() - t0) * 1e3 / 8
    dec = GraphDecoder(model, pool, tables, [prompt_len] * B, first, new_tokens)
    dec.capture(stream)
    samples = []
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        with EventTimer(stream) as total:
            for _ in range(new_tokens):
                dec.step()
        total_ms = total.ms()
    # second pass over the same positions, one event pair per step, for percentiles
    dec.pos.fill_(prompt_len)
    dec.tokens.copy_(first)
    dec.step_idx.zero_()
    with torch.cuda.stream(stream):
        for _ in range(new_tokens):
            with EventTimer(stream) as t:
                dec.step()
            samples.append(t.ms())
    torch.cuda.synchronize()
    return {
        "workload": f"config5 shape (closed batch): random-init Qwen3-0.6B bf16, B={B}, prompt {prompt_len} "
                    f"random tokens, {new_tokens} greedy steps (context {prompt_len}->{prompt_len + new_tokens}), "
                    "block 16, decode step replayed from one HIP graph",
        "tpot_ms": total_ms / new_tokens,
        "tpot_p50_ms": percentile(samples, 0.5),
        "tpot_p95_ms": percentile(samples, 0.95),
        "decode_tokens_per_s": B * new_tokens / (total_ms * 1e-3),
        "eager_step_ms": eager_ms,
        "prefill_ms": prefill_ms,
        "prefill_cold_ms": prefill_cold_ms,
        "prefill_tokens": B * prompt_len,
    }


def bench_config5(stream, n_requests: int = 64, rate: float = 4.0, seed: int = 0) -> dict:
    """Config 5 as specified: random-init Qwen3-0.6B served under a seeded Poisson trace (4
    req/s, prompts lognormal(median 256, sigma 0.6) clipped to [32, 2048], uniform ids, 128
    new tokens, greedy, max batch 32) by the continuous-batching loop (miattn.serve: FIFO
    packed-group admission, one captured HIP graph over 32 seats, retirement at 128 tokens),
    in real time. Reports TTFT and TPOT p50/p95 (nearest rank) over the requests."""
    from miattn.qwen3 import Qwen3, Qwen3Config, random_weights
    from miattn.serve import ContinuousServer, latency_summary, poisson_trace

    cfg = Qwen3Config()
    model = Qwen3(cfg, random_weights(cfg, seed), "cuda")
    trace = poisson_trace(n_requests, rate=rate, vocab=cfg.vocab, max_new=128, seed=seed)
    server = ContinuousServer(model, max_batch=32, n_blocks=8192, max_new=128, stream=None)
    server.warm()
    records, wall = server.run(trace, realtime=True)
    out = latency_summary(records, wall)
    out.update({
        "workload": f"config5: {n_requests} requests, Poisson {rate} req/s (gamma shape 1, seed {seed}), prompts "
                    "lognormal(median 256, sigma 0.6) clip [32,2048], 128 new tokens, greedy, max batch 32, "
                    "block 16, continuous batching (one HIP graph over 32 seats), real time",
        "decode_steps": server.steps_run,
        "mean_prompt_tokens": sum(len(r.prompt) for r in trace) / max(1, len(trace)),
    })
    del server, model
    torch.cuda.empty_cache()
    return out


def profiled_traffic() -> float | None:
    """HBM bytes per layer (split + merge launch) from the committed PMC summary
    (``profiles/paged_decode_config2_counters.json``): FETCH_SIZE and WRITE_SIZE per
    dispatch, each scaled by what the counter reads for a plain 1 GiB device copy."""
    path = ROOT / "profiles" / "paged_decode_config2_counters.json"
    try:
        c = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    fetch = c["fetch_kib_per_dispatch"] * (1048576.0 / c["copy_fetch_kib_for_1gib"])
    write = c["write_kib_per_dispatch"] * (1048576.0 / c["copy_write_kib_for_1gib"])
    return (fetch + write) * 1024.0


def copy_calibration(mib: int, reps: int) -> dict:
    """A plain device copy of a known size, run under the same PMC counters as the decode
    kernel: FETCH_SIZE / WRITE_SIZE of this launch over its known bytes is the counters'
    scale factor."""
    n = mib * 2**20 // 2
    src = torch.randn(n, device="cuda").to(torch.bfloat16)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    return {"copy_mib": mib, "bytes_read": n * 2, "bytes_written": n * 2,
            "gbs_read_plus_write": 2 * n * 2 / dt / 1e9}


def bench_prefill_qwen35(stream, steps: int = 20, eager: bool = False) -> dict:
    """Config 3's lengths at the Qwen3.5 attention shape (H 8 / H_kv 2 / head_dim 256): the
    packed prefill (28 layer calls on one packed group, HIP-graph replay), checked against
    the fp32 longhand oracle before it is timed."""
    from miattn import HipVarlen
    from miattn import workloads as W

    from oracle.varlen import longhand_varlen

    inp = W.prefill_config3(device="cuda", H=8, H_kv=2, D=256)
    backend = HipVarlen()
    H, D = inp.q.shape[1], inp.q.shape[2]
    flop = 4 * H * D * sum(n * (n + 1) // 2 for n in inp.lengths)
    ms = max(inp.lengths)
    got = backend.prefill_varlen(inp.q, inp.k, inp.v, cu_seqlens=inp.cu_seqlens, max_seqlen=ms).cpu().float()
    diff = (got - longhand_varlen(inp.q.cpu(), inp.k.cpu(), inp.v.cpu(), inp.cu_seqlens)).abs().max().item()
    if not diff <= 2e-2:
        raise SystemExit(f"Qwen3.5-shape prefill disagrees with the oracle: max|delta|={diff}")

    def prefill_step():
        for _ in range(N_LAYER):
            backend.prefill_varlen(inp.q, inp.k, inp.v, cu_seqlens=inp.cu_seqlens, max_seqlen=ms)

    if eager:  # plain dispatches, for counter collection
        with torch.cuda.stream(stream):
            for _ in range(2):
                prefill_step()
            torch.cuda.synchronize()
            with EventTimer(stream) as t:
                prefill_step()
            step_ms = t.ms()
    else:
        step_ms, _ = time_graph(prefill_step, stream, steps, 3)
    us = step_ms / N_LAYER * 1e3
    tflops = flop / (us * 1e-6) / 1e12
    return {
        "workload": "config3 lengths at H8/H_kv2/D256 bf16 (Qwen3.5 attention), 28 layer calls, HIP-graph replay",
        "prefill_us_per_layer": us,
        "prefill_tflops": tflops,
        "prefill_frac_mfma_peak": tflops / BF16_MFMA_PEAK_TFLOPS,
        "flop_per_layer": flop,
        "checked": {"max_abs_diff_vs_fp32_oracle": diff},
    }


def bench_prefill_long(stream, steps: int = 5, eager: bool = False, L: int = 8192) -> dict:
    """One ``L``-token segment at the Qwen3 attention shape (H16/H_kv8/D128 bf16), the
    library's default kernel (the tall kernel at this length): 28 layer calls per step,
    HIP-graph replay. Checked before it is timed on sampled query rows (the last 64 and 64
    spread over the segment, 4 heads) against an fp32 softmax of those rows over their
    whole causal key range, which the CPU computes in a second (the whole segment's fp32
    oracle would take minutes)."""
    from miattn import HipVarlen, _lib
    from miattn import workloads as W

    inp = W.prefill_config3(device="cuda", lengths=[L])
    backend = HipVarlen()
    H, D = inp.q.shape[1], inp.q.shape[2]
    G = H // inp.k.shape[1]
    # the kernel the library's default schedule names (header word 3, bits 20 and up)
    cu = (ctypes.c_int32 * 2)(0, L)
    n_words = _lib.lib.mi_varlen_schedule_for(cu, 1, H, inp.k.shape[1], D, 1, -1, None, 0)
    words = (ctypes.c_int32 * n_words)()
    _lib.lib.mi_varlen_schedule_for(cu, 1, H, inp.k.shape[1], D, 1, -1, words, n_words)
    kernel = {0: "staged", 1: "ring", 3: "duo", 4: "tall"}[words[3] >> 20]
    flop = 4 * H * D * L * (L + 1) // 2
    got = backend.prefill_varlen(inp.q, inp.k, inp.v, cu_seqlens=inp.cu_seqlens, max_seqlen=L).float().cpu()
    qc, kc, vc = inp.q.float().cpu(), inp.k.float().cpu(), inp.v.float().cpu()
    rows = sorted(set(range(L - 64, L)) | set(range(0, L, L // 64)))
    diff = 0.0
    for h in (0, 5, 10, 15):
        s = qc[rows, h] @ kc[:, h // G].T / D ** 0.5
        s = s.masked_fill(torch.arange(L)[None, :] > torch.tensor(rows)[:, None], float("-inf"))
        ref = torch.softmax(s, -1) @ vc[:, h // G]
        diff = max(diff, (got[rows, h] - ref).abs().max().item())
    if not diff <= 2e-2:
        raise SystemExit(f"long-segment prefill disagrees with the fp32 rows: max|delta|={diff}")

    def prefill_step():
        for _ in range(N_LAYER):
            backend.prefill_varlen(inp.q, inp.k, inp.v, cu_seqlens=inp.cu_seqlens, max_seqlen=L)

    if eager:
        with torch.cuda.stream(stream):
            prefill_step()
            torch.cuda.synchronize()
            with EventTimer(stream) as t:
                prefill_step()
            step_ms = t.ms()
    else:
        step_ms, _ = time_graph(prefill_step, stream, steps, 1)
    us = step_ms / N_LAYER * 1e3
    tflops = flop / (us * 1e-6) / 1e12
    return {
        "workload": f"one {L}-token segment, H16/H_kv8/D128 bf16, default kernel, 28 layer calls, HIP-graph replay",
        "kernel": kernel,
        "prefill_us_per_layer": us,
        "prefill_tflops": tflops,
        "prefill_frac_mfma_peak": tflops / BF16_MFMA_PEAK_TFLOPS,
        "flop_per_layer": flop,
        "checked": {"max_abs_diff_vs_fp32_rows": diff, "rows": len(rows), "heads": 4},
    }


def bench_block32(stream, steps: int = 50) -> dict:
    """Config 2 with 32-token blocks (the reference's other contract block size): the same
    lengths and the same bytes in 4096 blocks of 32 per layer, checked then timed like the
    headline leg."""
    from miattn import workloads as W

    inp = W.paged_decode_config(device="cuda", block_size=32, n_blocks=4096)
    res = bench_decode(inp, steps, 5, stream)
    res.pop("out0")
    del inp
    torch.cuda.empty_cache()
    return {"workload": "config2 lengths, block size 32 (4096 blocks/layer), 28 layers, HIP-graph replay", **res,
            "frac_hbm_peak": res["gbs"] / HBM_PEAK_GBS}


def bench_decode_config1(stream, steps: int = 50) -> dict:
    """Config 1's shape on the GPU kernel (the CPU seat path's workload in `cpu_baseline`):
    B=8 rows of 512 tokens (511 cached + 1), H16/8/D128 bf16, block size 16, 28 layers of
    512-block pools with permuted tables; checked then timed like the headline leg. (The
    config-1 inputs themselves, RoPE pre-applied, are checked against the seat path in
    tests/test_gpu_decode.py.)"""
    from miattn import workloads as W

    inp = W.paged_decode_config(device="cuda", B=8, lengths=[512] * 8, n_blocks=512)
    res = bench_decode(inp, steps, 5, stream)
    res.pop("out0")
    del inp
    torch.cuda.empty_cache()
    return {"workload": "config1 shape: B=8 x 512 tokens, H16/H_kv8/D128 bf16, block 16, 28 layers, HIP-graph replay",
            **res, "frac_hbm_peak": res["gbs"] / HBM_PEAK_GBS}


def bench_decode_qwen35(stream, steps: int = 50) -> dict:
    """Config 2's lengths at the Qwen3.5 attention shape (H 8 / H_kv 2 / head_dim 256,
    block size 16, 8192 blocks per layer, 28 layers): checked then timed like the
    headline leg."""
    from miattn import workloads as W

    inp = W.paged_decode_config(device="cuda", H=8, H_kv=2, D=256)
    res = bench_decode(inp, steps, 5, stream)
    res.pop("out0")
    del inp
    torch.cuda.empty_cache()
    return {"workload": "config2 lengths at H8/H_kv2/D256 bf16 (Qwen3.5 attention), 28 layers, HIP-graph replay",
            **res, "frac_hbm_peak": res["gbs"] / HBM_PEAK_GBS}


def bench_head_major(stream, steps: int = 50) -> dict:
    """Config 2 with head-major pools: each layer's K and V stored as (n_blocks, H_kv, 16,
    128), so a block holds each KV head's 16 tokens contiguously, and passed as the
    (n_blocks, 16, H_kv, 128) view with those strides; the same lengths, tables and bytes,
    checked then timed like the headline leg."""
    from miattn import workloads as W

    inp = W.paged_decode_config(device="cuda", head_major=True)
    res = bench_decode(inp, steps, 5, stream)
    res.pop("out0")
    del inp
    torch.cuda.empty_cache()
    return {"workload": "config2 lengths, head-major pools (n_blocks, H_kv, 16, D), 28 layers, HIP-graph replay",
            **res, "frac_hbm_peak": res["gbs"] / HBM_PEAK_GBS}


def check_decode_rows(inp, out0, rows) -> float:
    """Layer 0's output rows ``rows`` against the fp32 gather oracle (oracle.decode), before
    anything is timed; returns max|delta| and exits when it is outside the bf16 bar."""
    from oracle.decode import reference_paged_decode

    idx = torch.tensor(rows)
    got = out0.index_select(0, idx.to(out0.device)).cpu().float()
    table = inp.block_table.cpu()[idx]
    width = int(((inp.seqlen.cpu()[idx].max() + inp.block_size - 1) // inp.block_size).item())
    expected = reference_paged_decode(inp.q[0].cpu()[idx], inp.k_caches[0].cpu(), inp.v_caches[0].cpu(),
                                      table[:, :max(width, 1)], inp.seqlen.cpu()[idx], out_dtype=torch.float32)
    diff = (got - expected).abs().max().item()
    if not diff <= 2e-2:
        raise SystemExit(f"paged decode disagrees with the oracle on rows {rows}: max|delta|={diff}")
    return diff


def bench_long_context(stream, steps: int = 10):
    from miattn import workloads as W

    inp = W.paged_decode_config(B=32, lengths=[8192] * 32, n_blocks=16384, n_layer=N_LAYER, device="cuda",
                                max_blocks=512, seed=4)
    res = bench_decode(inp, steps, 3, stream, check_rows=[0, 13, 31])
    res.pop("out0")
    del inp
    torch.cuda.empty_cache()
    return {"workload": "config4: B=32 x 8192 tokens, 16384 blocks/layer, 28 layers", **res,
            "frac_hbm_peak": res["gbs"] / HBM_PEAK_GBS}


def cpu_baseline(inp, gpu_out0, budget_s: float = 10.0):
    """The reference's CPU seat path on layer 0 of the config-2 inputs (oracle.seat).

    Checks the GPU layer-0 output against it first, then times as many seat decodes as fit
    in ``budget_s`` on all host cores.
    """
    from oracle.seat import SeatSlab

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    B, H, D = inp.q[0].shape
    H_kv = inp.k_caches[0].shape[2]
    max_len = inp.block_table.shape[1] * inp.block_size
    kc = inp.k_caches[0].cpu()
    vc = inp.v_caches[0].cpu()
    slab = SeatSlab(1, B, H_kv, D, max_len, dtype=torch.bfloat16, n_head=H)
    bs = inp.block_size
    for b, (table, n) in enumerate(zip(inp.tables, inp.lengths)):
        t = torch.arange(n)
        blocks = torch.tensor(table)[t // bs]
        slab.keys[0][b, :, :n] = kc[blocks, t % bs].permute(1, 0, 2)
        slab.values[0][b, :, :n] = vc[blocks, t % bs].permute(1, 0, 2)
        slab.activate(b, n)
    slab.build_mask(next_token=False)
    q = inp.q[0].cpu().unsqueeze(2)
    seat = slab.attend(0, q)[:, :, 0]
    max_diff = (gpu_out0.cpu().float() - seat.float()).abs().max().item()
    if not max_diff <= 2e-2:
        raise SystemExit(f"GPU decode disagrees with the CPU seat path: max|delta|={max_diff}")
    times = []
    deadline = time.perf_counter() + budget_s
    while time.perf_counter() < deadline or len(times) < 3:
        t0 = time.perf_counter()
        slab.attend(0, q)
        times.append(time.perf_counter() - t0)
    p50 = percentile(times, 0.5)
    nbytes = decode_bytes(inp.lengths, B, H, H_kv, D, inp.block_table.shape[1])
    c1 = cpu_config1(budget_s / 2)
    c5 = cpu_config5_step()
    cpu_model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": nbytes / p50 / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{len(times)} seat-path decodes of config-2 layer 0 (B=32, slab width {max_len}), "
                  f"p50 {p50 * 1e3:.2f} ms per layer; same algorithmic bytes as the GPU line",
        "ms_per_layer_p50": p50 * 1e3,
        "cpu_model": cpu_model,
        "gpu_vs_seat_max_abs_diff": max_diff,
        "config1": c1,
        "config5_decode_step": c5,
    }


def cpu_config1(budget_s: float) -> dict:
    """Config 1 on the CPU seat path: one layer of B=8 rows, 511 cached + 1 new token, RoPE
    pre-applied (miattn.workloads.seat_decode_config1), timed on all host threads;
    algorithmic bytes B * 512 * 2 * H_kv * D * 2 = 16.8 MB."""
    from miattn import workloads as W
    from oracle.seat import SeatSlab

    q, k, v = W.seat_decode_config1()
    B, H_kv, L, D = k.shape
    slab = SeatSlab(1, B, H_kv, D, L, dtype=k.dtype, n_head=q.shape[1])
    slab.keys[0].copy_(k)
    slab.values[0].copy_(v)
    for b in range(B):
        slab.activate(b, L)
    slab.build_mask(next_token=False)
    times = []
    deadline = time.perf_counter() + budget_s
    while time.perf_counter() < deadline or len(times) < 20:
        t0 = time.perf_counter()
        slab.attend(0, q)
        times.append(time.perf_counter() - t0)
    p50 = percentile(times, 0.5)
    nbytes = B * L * 2 * H_kv * D * k.element_size()
    return {"us_per_step_p50": p50 * 1e6, "us_per_step_p95": percentile(times, 0.95) * 1e6,
            "gbs": nbytes / p50 / 1e9, "bytes": nbytes, "samples": len(times),
            "sample": "config1: one seat-path decode layer, B=8 x 512 tokens, H16/8 D128 bf16"}


def cpu_config5_step(B: int = 32, prompt: int = 128, steps: int = 3) -> dict:
    """A few B=32 greedy decode steps of the random-init Qwen3-0.6B on the CPU seat path
    (oracle.qwen3_seat: slab KV, SDPA prefill, bf16 softmax decode), prompts of ``prompt``
    uniform tokens; ms per whole decode step (28 layers + lm_head)."""
    from miattn.qwen3 import Qwen3Config, random_weights
    from oracle.qwen3_seat import SeatQwen3

    cfg = Qwen3Config()
    model = SeatQwen3(cfg, random_weights(cfg, 0), B, prompt + steps + 2)
    gen = torch.Generator().manual_seed(1)
    t0 = time.perf_counter()
    first = torch.stack([model.prefill(r, torch.randint(0, cfg.vocab, (prompt,), generator=gen).tolist())
                         for r in range(B)])
    prefill_s = time.perf_counter() - t0
    tok = first.argmax(-1)
    times = []
    for _ in range(steps + 1):
        t0 = time.perf_counter()
        tok = model.decode(tok).argmax(-1)
        times.append(time.perf_counter() - t0)
    times = times[1:]  # the first step warms the host allocator
    return {"ms_per_step_p50": percentile(times, 0.5) * 1e3, "steps": len(times), "prefill_s": prefill_s,
            "sample": f"config5 shape on the CPU: B={B} rows, {prompt}-token prompts (context {prompt}->"
                      f"{prompt + steps + 1}), bf16 seat path, {steps} timed steps after one warm step"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--decode-only", action="store_true", help="only the headline decode leg (for profiling)")
    ap.add_argument("--e2e-only", action="store_true", help="only the end-to-end legs (TPOT and the config-5 trace)")
    ap.add_argument("--tpot-only", action="store_true", help="only the end-to-end TPOT leg (for profiling)")
    ap.add_argument("--qwen35-decode-only", action="store_true",
                    help="only the Qwen3.5-shape decode leg (for profiling)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the config-3 prefill and slot-write legs (for profiling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true", help="time the decode leg without graph capture "
                    "(for counter collection, which needs plain kernel dispatches)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (counter scale calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        return 2
    import miattn
    from miattn import workloads as W

    if not miattn.HIP_AVAILABLE:
        raise RuntimeError(f"libmiattn.so is not loadable: {miattn.LOAD_ERROR}")
    torch.cuda.set_device(0)
    if args.copy_calibration:
        print(json.dumps(copy_calibration(args.copy_calibration, 5)), flush=True)
        return 0
    stream = torch.cuda.Stream()
    if args.e2e_only:
        print(json.dumps({"e2e": bench_tpot(stream), "config5_trace": bench_config5(stream)}), flush=True)
        return 0
    if args.tpot_only:
        print(json.dumps({"e2e": bench_tpot(stream)}), flush=True)
        return 0
    if args.qwen35_decode_only:
        print(json.dumps({"decode_qwen35": bench_decode_qwen35(stream)}), flush=True)
        return 0
    if args.prefill_only:
        print(json.dumps({"prefill": bench_prefill(stream, args.steps, eager=args.eager),
                          "prefill_qwen35": bench_prefill_qwen35(stream, args.steps, eager=args.eager),
                          "prefill_long": bench_prefill_long(stream, eager=args.eager)}),
              flush=True)
        return 0
    log("building config-2 inputs (28 layers, 8192 blocks each)")
    inp = W.paged_decode_config(device="cuda", max_blocks=128)
    log(f"decode: sum(seqlen)={inp.tokens}, B={len(inp.lengths)}")
    dec = bench_decode(inp, args.steps, args.warmup, stream, eager=args.eager)
    log(f"decode: {dec['us_per_layer']:.2f} us/layer, {dec['gbs']:.1f} GB/s")
    B, H, D = inp.q[0].shape
    H_kv = inp.k_caches[0].shape[2]
    line = {
        "metric": METRIC,
        "value": round(dec["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V, seeded uniform seqlen, permuted block tables)",
        "config": {
            "workload": "config2: paged decode, B=32, seqlen~U[128,2048], block 16, 8192 blocks/layer, "
                        "H16/H_kv8/D128, 28 layers per step (HIP-graph replay)",
            "B": B, "H": H, "H_kv": H_kv, "D": D, "block_size": inp.block_size, "layers": N_LAYER,
            "sum_seqlen": inp.tokens,
        },
        "pct_hbm_peak": round(100 * dec["gbs"] / HBM_PEAK_GBS, 2),
        "decode_us_per_layer": round(dec["us_per_layer"], 3),
        "decode_p50_ms_per_step": dec["p50_ms"],
        "decode_p95_ms_per_step": dec["p95_ms"],
        "eager_ms_per_step": round(dec["eager_ms_per_step"], 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "paged decode (split-K kernel + LSE merge kernel) per layer",
            "achieved": round(dec["bytes_per_layer"] / (dec["us_per_layer"] * 1e-6) / 1e9, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["bytes_per_layer"] / (dec["us_per_layer"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(),
            "algorithmic_bytes_per_launch": dec["bytes_per_layer"],
        },
        "tpot_ms": None,
    }
    if not args.decode_only:
        log("prefill + slot write (config 3)")
        line["prefill"] = bench_prefill(stream)
        log(f"prefill: {line['prefill']['prefill_tflops']:.1f} TFLOP/s, "
            f"slot write {line['prefill']['slot_write_gbs']:.1f} GB/s")
        line["prefill_qwen35"] = bench_prefill_qwen35(stream)
        log(f"prefill (Qwen3.5 shape, D256): {line['prefill_qwen35']['prefill_tflops']:.1f} TFLOP/s")
        line["prefill_long"] = bench_prefill_long(stream)
        log(f"prefill (one 8192-token segment, {line['prefill_long']['kernel']} kernel): "
            f"{line['prefill_long']['prefill_tflops']:.1f} TFLOP/s")
        log("end-to-end TPOT (config 5 shape, B=32 ctx 2048)")
        line["e2e"] = bench_tpot(stream)
        line["tpot_ms"] = round(line["e2e"]["tpot_ms"], 4)
        log(f"TPOT {line['tpot_ms']:.3f} ms (eager step {line['e2e']['eager_step_ms']:.2f} ms)")
        torch.cuda.empty_cache()
        log("config 5: continuous batching under a Poisson trace (real time)")
        line["config5_trace"] = bench_config5(stream)
        log(f"config5: TTFT p50 {line['config5_trace']['ttft_p50_ms']:.1f} ms, "
            f"TPOT p50 {line['config5_trace']['tpot_p50_ms']:.3f} ms")
        log("block size 32 (config 2 lengths)")
        line["decode_block32"] = bench_block32(stream)
        log(f"bs32: {line['decode_block32']['us_per_layer']:.2f} us/layer")
        line["decode_head_major"] = bench_head_major(stream)
        log(f"head-major pools: {line['decode_head_major']['us_per_layer']:.2f} us/layer")
        line["decode_qwen35"] = bench_decode_qwen35(stream)
        log(f"decode (Qwen3.5 shape, D256): {line['decode_qwen35']['us_per_layer']:.2f} us/layer")
        line["decode_config1"] = bench_decode_config1(stream)
        log(f"decode (config 1 shape, B=8 x 512): {line['decode_config1']['us_per_layer']:.2f} us/layer, "
            f"{line['decode_config1']['gbs']:.1f} GB/s")
        log("long-context decode (config 4)")
        line["long_context"] = bench_long_context(stream)
        log(f"config4: {line['long_context']['gbs']:.1f} GB/s")
    if not args.no_cpu_baseline:
        log("cpu baseline (seat path, config 2 layer 0)")
        line["cpu_baseline"] = cpu_baseline(inp, dec["out0"], args.cpu_budget)
    line["host"] = {"cpu_count": os.cpu_count(), "platform": platform.platform(),
                    "device": torch.cuda.get_device_name(0)}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
