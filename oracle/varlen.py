"""Packed varlen prefill oracles on the CPU. Test infrastructure only.

* :func:`longhand_varlen` -- per segment: scores -> causal mask -> softmax -> ``@ v`` in
  fp32 with GQA expanded by ``repeat_interleave`` (reference
  ``tests/unit/test_attention_varlen.py:71-92``);
* :func:`sdpa_varlen` -- one ``scaled_dot_product_attention`` per segment with
  ``is_causal`` and ``enable_gqa`` (reference ``model/attention/varlen.py:259-290``), the
  reference's CPU arm.

Pinned by: the two formulations agree with each other in float64, with a brute-force
double loop on tiny segments, and by invariants the reference tests use -- a one-token
segment returns its own ``v`` row, and perturbing segment 0 leaves every other segment's
output bitwise unchanged (reference ``tests/unit/test_attention_varlen.py:305-335``);
checked in ``tests/test_oracle_varlen.py``.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = ["longhand_varlen", "sdpa_varlen", "brute_force_varlen"]


def longhand_varlen(q, k, v, cu_seqlens, *, scale: float | None = None, causal: bool = True,
                    dtype=torch.float32) -> torch.Tensor:
    """``(T, H, D)`` result in ``dtype`` (fp32 by default; float64 for pinning)."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    group = q.size(1) // k.size(1)
    outs = []
    for start, end in zip(cu_seqlens, cu_seqlens[1:]):
        qs = q[start:end].to(dtype).transpose(0, 1)
        ks = k[start:end].to(dtype).transpose(0, 1).repeat_interleave(group, dim=0)
        vs = v[start:end].to(dtype).transpose(0, 1).repeat_interleave(group, dim=0)
        scores = torch.matmul(qs, ks.transpose(-2, -1)) * scale
        if causal:
            n = scores.size(-1)
            scores = scores.masked_fill(~torch.ones(n, n, dtype=torch.bool).tril(), float("-inf"))
        outs.append(torch.matmul(torch.softmax(scores, dim=-1), vs).transpose(0, 1))
    return torch.cat(outs, dim=0)


def sdpa_varlen(q, k, v, cu_seqlens, *, scale: float | None = None, causal: bool = True) -> torch.Tensor:
    """The reference's SDPA-per-segment arm; result in ``q.dtype``."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    gqa = q.size(1) != k.size(1)
    segs = [
        F.scaled_dot_product_attention(
            q[s:e].transpose(0, 1).unsqueeze(0), k[s:e].transpose(0, 1).unsqueeze(0),
            v[s:e].transpose(0, 1).unsqueeze(0), attn_mask=None, dropout_p=0.0,
            is_causal=causal, scale=scale, enable_gqa=gqa,
        ).squeeze(0).transpose(0, 1)
        for s, e in zip(cu_seqlens, cu_seqlens[1:])
    ]
    return torch.cat(segs, dim=0)


def brute_force_varlen(q, k, v, cu_seqlens, *, scale: float | None = None, causal: bool = True) -> torch.Tensor:
    """Scalar double loop in float64 for tiny inputs."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    T, H, D = q.shape
    group = H // k.shape[1]
    out = torch.zeros(T, H, D, dtype=torch.float64)
    qd, kd, vd = q.double(), k.double(), v.double()
    for start, end in zip(cu_seqlens, cu_seqlens[1:]):
        for i in range(start, end):
            last = i if causal else end - 1
            for h in range(H):
                kv = h // group
                s = torch.tensor([float(qd[i, h] @ kd[j, kv]) * scale for j in range(start, last + 1)],
                                 dtype=torch.float64)
                p = torch.exp(s - s.max())
                p = p / p.sum()
                out[i, h] = sum(p[j - start] * vd[j, kv] for j in range(start, last + 1))
    return out
