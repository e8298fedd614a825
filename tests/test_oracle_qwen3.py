"""Pins the CPU seat-path model (``oracle.qwen3_seat``) used as the end-to-end oracle.

* Library pin: on a tiny Qwen3 configuration, in float64, the seat model's prefill and
  decode logits equal Hugging Face ``Qwen3ForCausalLM`` (an independent implementation of
  the same architecture) given the same weights, to 1e-6 (HF's RMSNorm and RoPE tables
  compute in float32 even in a float64 model; that rounding is the whole difference).
* Cache pin: a decode step after prefill equals a fresh prefill of the extended prompt.
* A planted mistake (RoPE pairing (2k, 2k+1) instead of the NeoX halves) fails the
  library pin.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

from miattn.qwen3 import Qwen3Config, random_weights
import oracle.qwen3_seat as seat_mod
from oracle.qwen3_seat import SeatQwen3

transformers = pytest.importorskip("transformers")

TINY = Qwen3Config(vocab=97, hidden=64, inter=96, n_layer=2, n_head=4, n_kv_head=2, head_dim=16)


def _weights(seed=3):
    w = {k: v.to(torch.float64) for k, v in random_weights(TINY, seed, dtype=torch.float32).items()}
    gen = torch.Generator().manual_seed(seed + 100)
    for k in w:  # non-unit norm weights so the norms are exercised
        if w[k].dim() == 1:
            w[k] = 1.0 + 0.3 * torch.randn(w[k].shape, generator=gen, dtype=torch.float64)
    return w


def _hf(w):
    c = TINY
    cfg = transformers.Qwen3Config(
        vocab_size=c.vocab, hidden_size=c.hidden, intermediate_size=c.inter, num_hidden_layers=c.n_layer,
        num_attention_heads=c.n_head, num_key_value_heads=c.n_kv_head, head_dim=c.head_dim,
        rms_norm_eps=c.eps, rope_theta=c.rope_theta, tie_word_embeddings=True, max_position_embeddings=512,
        attention_bias=False,
    )
    m = transformers.Qwen3ForCausalLM(cfg).to(torch.float64).eval()
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm"], "lm_head.weight": w["embed"]}
    names = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj", "wo": "self_attn.o_proj",
             "wg": "mlp.gate_proj", "wu": "mlp.up_proj", "wd": "mlp.down_proj", "qn": "self_attn.q_norm",
             "kn": "self_attn.k_norm", "ln1": "input_layernorm", "ln2": "post_attention_layernorm"}
    for i in range(c.n_layer):
        for short, long in names.items():
            sd[f"model.layers.{i}.{long}.weight"] = w[f"l{i}.{short}"]
    m.load_state_dict(sd, strict=True)
    return m


def _run_seat(w, prompts, steps):
    m = SeatQwen3(TINY, w, len(prompts), max(map(len, prompts)) + steps + 1)
    logits = [torch.stack([m.prefill(r, p) for r, p in enumerate(prompts)])]
    tok = logits[0].argmax(-1)
    toks = [tok]
    for _ in range(steps):
        logits.append(m.decode(tok))
        tok = logits[-1].argmax(-1)
        toks.append(tok)
    return logits, toks


def _hf_logits(hf, prompts, toks):
    """Full-prefix HF logits for every step the seat model took (teacher forced)."""
    out = []
    for s in range(len(toks)):
        rows = []
        for r, p in enumerate(prompts):
            seq = p + [int(t[r]) for t in toks[:s]]
            with torch.no_grad():
                rows.append(hf(torch.tensor([seq])).logits[0, -1])
        out.append(torch.stack(rows))
    return out


def test_seat_model_matches_hugging_face_qwen3_in_float64():
    w = _weights()
    gen = torch.Generator().manual_seed(5)
    prompts = [torch.randint(0, TINY.vocab, (n,), generator=gen).tolist() for n in (5, 11, 1)]
    seat_logits, toks = _run_seat(w, prompts, steps=6)
    hf_logits = _hf_logits(_hf(w), prompts, toks)
    for s, (a, b) in enumerate(zip(seat_logits, hf_logits)):
        assert torch.allclose(a, b, rtol=0, atol=1e-6), f"step {s}: max|delta| {(a - b).abs().max().item()}"


def test_decode_step_equals_prefill_of_the_extended_prompt():
    w = _weights(seed=7)
    prompt = list(range(3, 12))
    logits, toks = _run_seat(w, [prompt], steps=3)
    m = SeatQwen3(TINY, w, 1, 64)
    ext = prompt + [int(t[0]) for t in toks[:3]]
    assert torch.allclose(m.prefill(0, ext), logits[3][0], rtol=0, atol=1e-9)


def test_planted_rope_pairing_mistake_fails_the_library_pin(monkeypatch):
    def interleaved(x, cos, sin):
        x1, x2 = x[..., 0::2], x[..., 1::2]
        return torch.stack([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1).flatten(-2)

    monkeypatch.setattr(seat_mod, "_rotate", interleaved)
    w = _weights()
    prompts = [[1, 2, 3, 4, 5, 6]]
    seat_logits, toks = _run_seat(w, prompts, steps=1)
    hf_logits = _hf_logits(_hf(w), prompts, toks)
    assert (seat_logits[0] - hf_logits[0]).abs().max().item() > 1e-3
