"""Packed varlen prefill oracles on the CPU. Test infrastructure only.

* :func:`longhand_varlen` -- per segment: scores -> causal mask -> softmax -> ``@ v`` in
  fp32 with GQA expanded by ``repeat_interleave`` (reference
  ``tests/unit/test_attention_varlen.py:71-92``);
* :func:`sdpa_varlen` -- one ``scaled_dot_product_attention`` per segment with
  ``is_causal`` and ``enable_gqa`` (reference ``model/attention/varlen.py:259-290``), the
  reference's CPU arm;
* :func:`varlen_error_bound` -- the float64 result and a per-element bound on how far a
  kernel that feeds the probabilities to the PV product in the input dtype (16-bit MFMA
  operands, as flash attention does) may land from it.

Pinned by: the two formulations agree with each other in float64, with a brute-force
double loop on tiny segments, and by invariants the reference tests use -- a one-token
segment returns its own ``v`` row, and perturbing segment 0 leaves every other segment's
output bitwise unchanged (reference ``tests/unit/test_attention_varlen.py:305-335``);
checked in ``tests/test_oracle_varlen.py``. The bound is pinned there too: a float64
emulation of a 16-bit-P kernel stays inside it on every element, and the same emulation
with a planted mistake (P rounded to 6 significant bits, a 1% scale error, one dropped key)
leaves it.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = ["longhand_varlen", "sdpa_varlen", "brute_force_varlen", "varlen_error_bound", "UNIT_ROUNDOFF"]

# unit roundoff of round-to-nearest into the input dtype: 2^-p for a p-bit significand
UNIT_ROUNDOFF = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


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


def varlen_error_bound(q, k, v, cu_seqlens, *, scale: float | None = None, causal: bool = True):
    """``(ref, bound)``, both ``(T, H, D)``: the float64 result (as fp32) and, per element,
    the largest ``|out - ref|`` a kernel may show that

    * computes the scores ``s = q.k * scale`` with fp32 accumulation of exact products,
    * forms ``p_j = exp(s_j - m)`` in fp32 and rounds each to the input dtype (unit
      roundoff ``u``: 2^-8 bf16, 2^-11 fp16) before the PV product, which accumulates in fp32,
    * normalises by a row sum of either the rounded or the unrounded ``p``,
    * and rounds the output to the input dtype.

    With ``pi_j`` the exact probabilities and ``o`` the exact output, rounding ``p_j`` to
    ``p_j (1 + e_j)``, ``|e_j| <= u``, moves the output by ``sum_j pi_j e_j (v_j - c)`` to
    first order, where ``c = o`` when the row sum is taken over the rounded values and
    ``c = 0`` when it is not. So the probability term is ``u * max(A, B)`` with
    ``A = sum_j pi_j |v_j|`` and ``B = sqrt(sum_j pi_j v_j^2 - o^2)``, the probability-weighted
    spread of ``v``, which bounds ``sum_j pi_j |v_j - o|`` (Jensen). The rest:

    * output rounding ``u |o|``;
    * the fp32 score error, at most ``gamma_D * scale * |q_i| * max_j |k_j|`` (Cauchy-Schwarz
      on the accumulated products, ``gamma_n = n 2^-24 / (1 - n 2^-24)``), moves each
      ``p_j`` and the row sum by a relative ``delta`` and the output by ``2 delta (A + |o|)``;
    * fp32 accumulation of the PV product and the row sum over the row's ``n`` keys, and the
      final division: ``2 gamma_(n+1) (A + |o|)``;
    * the hardware exp2 (a few ulp) and the shift by the running maximum: ``2^-20 (A + |o|)``;
    * second-order terms in ``u``: the probability term carries a factor ``1 + 2u``.
    """
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    if q.dtype not in UNIT_ROUNDOFF:
        raise ValueError(f"no 16-bit unit roundoff for {q.dtype}")
    u = UNIT_ROUNDOFF[q.dtype]
    D = q.shape[-1]
    group = q.size(1) // k.size(1)
    gamma = lambda n: n * 2.0 ** -24 / (1.0 - n * 2.0 ** -24)  # noqa: E731
    refs, bounds = [], []
    for start, end in zip(cu_seqlens, cu_seqlens[1:]):
        n = end - start
        qs = q[start:end].double().transpose(0, 1)
        ks = k[start:end].double().transpose(0, 1).repeat_interleave(group, dim=0)
        vs = v[start:end].double().transpose(0, 1).repeat_interleave(group, dim=0)
        scores = torch.matmul(qs, ks.transpose(-2, -1)) * scale
        if causal:
            scores = scores.masked_fill(~torch.ones(n, n, dtype=torch.bool).tril(), float("-inf"))
            keys = torch.arange(1, n + 1, dtype=torch.float64)[None, :, None]
        else:
            keys = torch.full((1, n, 1), float(n), dtype=torch.float64)
        pi = torch.softmax(scores, dim=-1)
        o = torch.matmul(pi, vs)
        a = torch.matmul(pi, vs.abs())
        b = (torch.matmul(pi, vs * vs) - o * o).clamp_min(0.0).sqrt()
        delta = gamma(D) * scale * qs.norm(dim=-1, keepdim=True) * ks.norm(dim=-1).amax(dim=-1)[:, None, None]
        accum = 2.0 * gamma(keys + 1.0)
        rest = (2.0 * delta + accum + 2.0 ** -20) * (a + o.abs())
        bound = u * o.abs() + u * (1.0 + 2.0 * u) * torch.maximum(a, b) + rest
        refs.append(o.transpose(0, 1))
        bounds.append(bound.transpose(0, 1))
    return torch.cat(refs).float(), torch.cat(bounds).float()
