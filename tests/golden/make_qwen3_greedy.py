"""Write ``qwen3_greedy_seed0.json``: the CPU seat path's greedy decode of a random-init
Qwen3-0.6B (the end-to-end fixture the GPU path is checked against).

Weights: ``miattn.qwen3.random_weights(Qwen3Config(), seed=0)`` (bf16, N(0, 0.02)).
Prompts: 4 requests of 37/64/100/128 uniform token ids (torch.Generator seed 1).
Recorded per request: the greedy tokens of the prefill step and 64 decode steps, and at
every step the 16 largest logits (ids and values) so a checker can tell a genuine
disagreement from a near-tie. Runs in about 10 s on 8 cores:

    python tests/golden/make_qwen3_greedy.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "llm-serving_amd")]

from miattn.qwen3 import Qwen3Config, random_weights  # noqa: E402
from oracle.qwen3_seat import SeatQwen3  # noqa: E402

SEED, PROMPT_SEED, LENGTHS, STEPS, TOPK = 0, 1, (37, 64, 100, 128), 64, 16


def main() -> None:
    torch.set_num_threads(min(16, torch.get_num_threads()))
    cfg = Qwen3Config()
    model = SeatQwen3(cfg, random_weights(cfg, SEED), len(LENGTHS), max(LENGTHS) + STEPS + 1)
    gen = torch.Generator().manual_seed(PROMPT_SEED)
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen).tolist() for n in LENGTHS]
    steps = []

    def record(logits):
        top = logits.float().topk(TOPK, dim=-1)
        steps.append({"ids": top.indices.tolist(), "logits": top.values.tolist(),
                      "argmax": logits.argmax(-1).tolist()})
        return logits.argmax(-1)

    tok = record(torch.stack([model.prefill(r, p) for r, p in enumerate(prompts)]))
    for _ in range(STEPS):
        tok = record(model.decode(tok))
    out = {"weights_seed": SEED, "prompt_seed": PROMPT_SEED, "lengths": list(LENGTHS),
           "prompts": prompts, "steps": steps,
           "tokens": [[s["argmax"][r] for s in steps] for r in range(len(LENGTHS))],
           "note": "steps[0] is the prefill's last-token logits; steps[1..64] the decode steps"}
    path = Path(__file__).with_name("qwen3_greedy_seed0.json")
    path.write_text(json.dumps(out))
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
