"""The reference's CPU seat path for a whole model -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A CPU restatement of ``MiniLLM`` (reference ``model/minillm.py:66-168``,
``model/layers.py:16-368``) driven the way the reference serves on a CPU: prefill through
the SDPA varlen arm (one ``scaled_dot_product_attention`` per request with ``is_causal``,
reference ``model/attention/varlen.py:259-290``) writing the K/V into a contiguous seat
slab (reference ``serve/engine.py:100-144``, ``model/slab.py:251-266``), and decode through
the slab's mask/bias and ``hand_baddbmm`` with the softmax in the activation dtype
(``oracle.seat``; reference ``model/attention/hand_baddbmm.py:80-126``). Everything is in
the weights' dtype (bf16), as the reference computes it.

This is the oracle for the end-to-end greedy check: the GPU path (this repository's HIP
kernels behind ``PackedPrefill``/``PagedKV``) must produce the same greedy tokens. It takes
the weight dictionary of ``miattn.qwen3.random_weights`` and shares no model code with it.

Pinned by: the attention pieces it uses are pinned in ``tests/test_oracle_seat.py`` and
``tests/test_oracle_varlen.py``; the whole model is checked in
``tests/test_oracle_qwen3.py`` against a float64 dense re-computation on a tiny
configuration (same weights, plain causal attention over the full prefix), and its
decode steps against its own full-prefix prefill (a decode step must equal re-running
prefill on the extended prompt).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from oracle.seat import SeatSlab

__all__ = ["SeatQwen3"]


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    # reference model/layers.py:348-350: sqrt(mean(x^2) + eps), divide, scale -- in x.dtype
    return x / torch.sqrt(x.pow(2).mean(-1, True) + eps) * w


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    # reference model/layers.py:65-94 (GPT-NeoX halves); cos/sin already shaped to broadcast
    h = x.shape[-1] // 2
    return torch.cat([x[..., :h] * cos - x[..., h:] * sin, x[..., :h] * sin + x[..., h:] * cos], dim=-1)


class SeatQwen3:
    """``n_rows`` seats of ``max_len`` positions; prefill whole prompts, then decode all rows."""

    def __init__(self, cfg, weights: dict, n_rows: int, max_len: int) -> None:
        self.c = cfg
        self.w = weights
        self.dtype = weights["embed"].dtype
        D = cfg.head_dim
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        ang = torch.outer(torch.arange(max_len + 1, dtype=torch.float32), inv)
        # reference rope_cos_sin(..., dtype=model dtype): the table itself is bf16
        self.cos, self.sin = ang.cos().to(self.dtype), ang.sin().to(self.dtype)
        self.slab = SeatSlab(cfg.n_layer, n_rows, cfg.n_kv_head, D, max_len, dtype=self.dtype, n_head=cfg.n_head)
        for r in range(n_rows):
            self.slab.freeze(r)

    def _proj(self, i, x):
        c, p = self.c, f"l{i}."
        lead = x.shape[:-1]
        q = _rms((x @ self.w[p + "wq"].T).view(*lead, c.n_head, c.head_dim), self.w[p + "qn"], c.eps)
        k = _rms((x @ self.w[p + "wk"].T).view(*lead, c.n_kv_head, c.head_dim), self.w[p + "kn"], c.eps)
        v = (x @ self.w[p + "wv"].T).view(*lead, c.n_kv_head, c.head_dim)
        return q, k, v

    def _mlp(self, i, x):
        p = f"l{i}."
        return (F.silu(x @ self.w[p + "wg"].T) * (x @ self.w[p + "wu"].T)) @ self.w[p + "wd"].T

    def _logits(self, x):
        return _rms(x, self.w["norm"], self.c.eps) @ self.w["embed"].T

    @torch.no_grad()
    def prefill(self, row: int, prompt: list[int]) -> torch.Tensor:
        """Whole-prompt prefill of one request into seat ``row``; last-token logits ``(vocab,)``."""
        c = self.c
        L = len(prompt)
        x = self.w["embed"][torch.tensor(prompt)]  # (L, C)
        cos, sin = self.cos[:L].unsqueeze(1), self.sin[:L].unsqueeze(1)  # (L, 1, D/2)
        for i in range(c.n_layer):
            h = _rms(x, self.w[f"l{i}.ln1"], c.eps)
            q, k, v = self._proj(i, h)
            q, k = _rotate(q, cos, sin), _rotate(k, cos, sin)
            # seat write-through sink: the slab row's first L columns (reference
            # serve/engine.py:120-144)
            self.slab.keys[i][row, :, :L] = k.transpose(0, 1)
            self.slab.values[i][row, :, :L] = v.transpose(0, 1)
            y = F.scaled_dot_product_attention(
                q.transpose(0, 1).unsqueeze(0), k.transpose(0, 1).unsqueeze(0), v.transpose(0, 1).unsqueeze(0),
                is_causal=True, scale=1.0 / math.sqrt(c.head_dim), enable_gqa=True,
            ).squeeze(0).transpose(0, 1)  # (L, H, D)
            x = x + y.reshape(L, -1) @ self.w[f"l{i}.wo"].T
            x = x + self._mlp(i, _rms(x, self.w[f"l{i}.ln2"], c.eps))
        self.slab.activate(row, L)
        return self._logits(x[-1])

    @torch.no_grad()
    def decode(self, tokens: torch.Tensor) -> torch.Tensor:
        """One step of every seat (reference ``MiniLLM.forward`` slab branch); ``(B, vocab)``."""
        c = self.c
        slab = self.slab
        slab.build_mask(next_token=True)
        pos = slab.pos
        cos, sin = self.cos[pos].view(-1, 1, 1, c.head_dim // 2), self.sin[pos].view(-1, 1, 1, c.head_dim // 2)
        x = self.w["embed"][tokens.view(-1, 1)]  # (B, 1, C)
        for i in range(c.n_layer):
            h = _rms(x, self.w[f"l{i}.ln1"], c.eps)
            q, k, v = self._proj(i, h)  # (B, 1, H, D)
            q, k = _rotate(q, cos, sin), _rotate(k, cos, sin)
            slab.write(i, k.transpose(1, 2), v.transpose(1, 2))
            y = slab.attend(i, q.transpose(1, 2))  # (B, H, 1, D)
            x = x + y.transpose(1, 2).reshape(x.shape[0], 1, -1) @ self.w[f"l{i}.wo"].T
            x = x + self._mlp(i, _rms(x, self.w[f"l{i}.ln2"], c.eps))
        slab.advance()
        return self._logits(x[:, 0])
