"""Write ``greedy_gate_seed0.json``: the CPU seat path's greedy tokens for a random-init
Qwen3-0.6B, with an fp32 recomputation of every step, for the end-to-end greedy gate.

Two cases, same weights (``miattn.qwen3.random_weights(Qwen3Config(), seed=0)``, bf16
N(0, 0.02)):

* ``closed``: 4 prompts of 37/64/100/128 uniform ids (torch.Generator seed 1), the prefill
  token and 64 decode steps each (65 greedy tokens per request);
* ``trace``: a sized-down config 5 -- 8 requests of ``miattn.serve.poisson_trace`` (4 req/s,
  prompts lognormal(median 256, sigma 0.6) clipped to [32, 2048], seed 5) with 32 new tokens
  each instead of 128.

The reference's gate is exact greedy agreement, with every miss first checked as a
near-tie against an fp32 oracle (reference
``results/W45/0001-paged-packed-numeric-gate/config.toml:9``). So for every step this
records, besides the bf16 seat path's token (``tokens``): the same model in fp32 (weights,
RoPE tables and KV upcast) run teacher-forced on the bf16 path's tokens, its logits at the
union of the bf16 top-8 and fp32 top-8 ids (``cand_ids``/``cand_fp32``), and ``bf16_err``,
the largest |bf16 - fp32| logit difference over those ids -- how far the bf16 computation
itself strays from fp32 at that step. Runs in well under a minute on 8 cores:

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


def greedy(cfg, weights, prompts, steps, forced=None):
    """Per-step logits ``[(rows, vocab)]`` of greedy decoding (or of decoding fed ``forced``
    tokens, ``forced[r][s]`` being the token after step s) on the CPU seat path."""
    model = SeatQwen3(cfg, weights, len(prompts), max(len(p) for p in prompts) + steps + 1)
    out = [torch.stack([model.prefill(r, p) for r, p in enumerate(prompts)]).float()]
    for s in range(steps):
        tok = out[-1].argmax(-1) if forced is None else torch.tensor([f[s] for f in forced])
        out.append(model.decode(tok).float())
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
    trace = poisson_trace(8, rate=4.0, vocab=cfg.vocab, max_new=32, seed=5)
    out = {
        "weights_seed": SEED,
        "closed": {"steps": 64, **case(cfg, w16, w32, closed, 64)},
        "trace": {"rate": 4.0, "seed": 5, "max_new": 32, "arrivals": [r.arrival_s for r in trace],
                  **case(cfg, w16, w32, [list(r.prompt) for r in trace], 31)},
        "note": "per case: tokens[r][s] is the bf16 seat path's greedy token s of request r (s=0 from the "
                "prefill); cand_ids/cand_fp32/bf16_err are indexed [s][r]",
    }
    path = Path(__file__).with_name("greedy_gate_seed0.json")
    path.write_text(json.dumps(out, separators=(",", ":")))
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
