"""Write ``greedy_gate_seed0.json``: the CPU seat path's greedy tokens for a random-init
Qwen3-0.6B, with an fp32 recomputation of every step, for the end-to-end greedy gate.

Two cases, same weights (``miattn.qwen3.random_weights(Qwen3Config(), seed=0)``, bf16
N(0, 0.02)):

* ``closed``: 4 prompts of 37/64/100/128 uniform ids (torch.Generator seed 1), the prefill
  token and 64 decode steps each (65 greedy tokens per request);
* ``trace``: config 5 at its concurrency, time-compressed -- 16 requests of
  ``miattn.serve.poisson_trace`` (prompts lognormal(median 256, sigma 0.6) clipped to
  [32, 2048], seed 5) at 400 req/s instead of 4 (the arrivals x 1/100), with 128 new tokens
  for every third request and 32 or 48 for the others. Served on the synthetic clock of
  ``ContinuousServer.run(step_s=TRACE_STEP_S)``, one arrival lands about every decode step:
  the requests are admitted in small groups while earlier ones decode, up to 16 seats
  decode together, and the short requests retire while the long ones go on.

The reference's gate is exact greedy agreement, with every miss first checked as a
near-tie against an fp32 oracle (reference
``results/W45/0001-paged-packed-numeric-gate/config.toml:9``). So for every step this
records, besides the bf16 seat path's token (``tokens``): the same model in fp32 (weights,
RoPE tables and KV upcast) run teacher-forced on the bf16 path's tokens, its logits at the
union of the bf16 top-8 and fp32 top-8 ids (``cand_ids``/``cand_fp32``), and ``bf16_err``,
the largest |bf16 - fp32| logit difference over those ids -- how far the bf16 computation
itself strays from fp32 at that step. The closed case indexes these ``[step][row]``, the
trace case ``[request][step]`` (its requests have different lengths). Runs in about two
minutes on 8 cores:

    python tests/golden/make_greedy_gate.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "llm-serving_amd")]

from miattn.qwen3 import Qwen3Config, random_weights  # noqa: E402
from miattn.serve import poisson_trace  # noqa: E402
from oracle.qwen3_seat import SeatQwen3  # noqa: E402

SEED, TOP = 0, 8
TRACE_N, TRACE_RATE, TRACE_SEED, TRACE_STEP_S = 16, 400.0, 5, 0.0025


def trace_max_new(i: int) -> int:
    return (128, 32, 48)[i % 3]


def greedy(cfg, weights, prompts, steps, forced=None):
    """Per-step logits ``[(rows, vocab)]`` of greedy decoding (or of decoding fed ``forced``
    tokens, ``forced[r][s]`` being the token after step s) on the CPU seat path."""
    model = SeatQwen3(cfg, weights, len(prompts), max(len(p) for p in prompts) + steps + 1)
    out = [torch.stack([model.prefill(r, p) for r, p in enumerate(prompts)]).float()]
    for s in range(steps):
        tok = out[-1].argmax(-1) if forced is None else torch.tensor([f[s] for f in forced])
        out.append(model.decode(tok).float())
    return out


def per_request(cfg, w16, w32, prompts, max_new) -> dict:
    """The trace case: requests grouped by token budget, each group through :func:`case`,
    the results re-indexed ``[request][step]``."""
    out = {"lengths": [len(p) for p in prompts], "prompts": [list(p) for p in prompts], "tokens": [None] * len(prompts),
           "cand_ids": [None] * len(prompts), "cand_fp32": [None] * len(prompts), "bf16_err": [None] * len(prompts)}
    for budget in sorted(set(max_new)):
        rows = [i for i, m in enumerate(max_new) if m == budget]
        rec = case(cfg, w16, w32, [prompts[i] for i in rows], budget - 1)
        for j, i in enumerate(rows):
            out["tokens"][i] = rec["tokens"][j]
            for key in ("cand_ids", "cand_fp32", "bf16_err"):
                out[key][i] = [step[j] for step in rec[key]]
    return out


def case(cfg, w16, w32, prompts, steps) -> dict:
    logits16 = greedy(cfg, w16, prompts, steps)
    tokens = [[int(step[r].argmax()) for step in logits16] for r in range(len(prompts))]
    logits32 = greedy(cfg, w32, prompts, steps, forced=tokens)
    rec = {"lengths": [len(p) for p in prompts], "prompts": [list(p) for p in prompts], "tokens": tokens,
           "cand_ids": [], "cand_fp32": [], "bf16_err": []}
    for l16, l32 in zip(logits16, logits32):
        ids_s, vals_s, err_s = [], [], []
        for r in range(len(prompts)):
            ids = sorted(set(l16[r].topk(TOP).indices.tolist()) | set(l32[r].topk(TOP).indices.tolist()))
            idx = torch.tensor(ids)
            ids_s.append(ids)
            vals_s.append([round(v, 5) for v in l32[r, idx].tolist()])
            err_s.append(round(float((l16[r, idx] - l32[r, idx]).abs().max()), 5))
        rec["cand_ids"].append(ids_s)
        rec["cand_fp32"].append(vals_s)
        rec["bf16_err"].append(err_s)
    return rec


def main() -> None:
    torch.set_num_threads(min(16, torch.get_num_threads()))
    cfg = Qwen3Config()
    w16 = random_weights(cfg, SEED)
    w32 = {k: v.float() for k, v in w16.items()}
    gen = torch.Generator().manual_seed(1)
    closed = [torch.randint(0, cfg.vocab, (n,), generator=gen).tolist() for n in (37, 64, 100, 128)]
    trace = poisson_trace(TRACE_N, rate=TRACE_RATE, vocab=cfg.vocab, seed=TRACE_SEED)
    max_new = [trace_max_new(i) for i in range(TRACE_N)]
    out = {
        "weights_seed": SEED,
        "closed": {"steps": 64, **case(cfg, w16, w32, closed, 64)},
        "trace": {"rate": TRACE_RATE, "seed": TRACE_SEED, "step_s": TRACE_STEP_S, "max_new": max_new,
                  "arrivals": [r.arrival_s for r in trace],
                  **per_request(cfg, w16, w32, [list(r.prompt) for r in trace], max_new)},
        "note": "tokens[r][s] is the bf16 seat path's greedy token s of request r (s=0 from the prefill); "
                "cand_ids/cand_fp32/bf16_err are indexed [s][r] in the closed case and [r][s] in the trace case",
    }
    path = Path(__file__).with_name("greedy_gate_seed0.json")
    path.write_text(json.dumps(out, separators=(",", ":")))
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
