"""Paged-decode attention oracles on the CPU. Test infrastructure only.

Two independent formulations, as in the reference's three-way split (reference
``tests/unit/test_triton_decode.py:4-8``):

* :func:`dense_decode_f64` -- every logical token looked up through the block table one at
  a time, float64 softmax per query head (reference
  ``tests/unit/test_triton_decode.py:75-105``);
* :func:`reference_paged_decode` -- gather the row's pages with ``index_select``, fp32
  einsum scores, softmax, einsum with V (reference ``tests/reference/paged.py:225-274``).

Pinned by: agreement with ``torch.nn.functional.scaled_dot_product_attention`` in float64
on the gathered dense K/V (a library routine, independent of both loops), and by closed
forms -- seqlen 0 gives exact zeros (reference ``tests/reference/paged.py:259-262``), seqlen
1 gives ``v`` exactly, equal keys give the mean of V, and the GQA map ``kv = h // G``
(reference ``model/triton_decode.py:584-585``) -- checked in ``tests/test_oracle_decode.py``.
"""

from __future__ import annotations

import math

import numpy as np
import torch

__all__ = ["dense_decode_f64", "reference_paged_decode", "dense_kv"]


def dense_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, table_row, length: int):
    """``(length, H_kv, D)`` K and V of one row, gathered token by token."""
    bs = k_cache.shape[1]
    ids = [int(table_row[t // bs]) for t in range(length)]
    offs = [t % bs for t in range(length)]
    return k_cache[ids, offs], v_cache[ids, offs]


def dense_decode_f64(q, k_cache, v_cache, block_table, seqlen, scale: float | None = None) -> torch.Tensor:
    """Per-token, per-head float64 softmax attention; returns ``q.dtype``."""
    B, H, D = q.shape
    H_kv = k_cache.shape[2]
    G = H // H_kv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty(q.shape, dtype=q.dtype)
    for row in range(B):
        n = int(seqlen[row])
        if n == 0:
            out[row].zero_()
            continue
        k, v = dense_kv(k_cache, v_cache, block_table[row], n)
        k = k.to(torch.float64).numpy()
        v = v.to(torch.float64).numpy()
        for head in range(H):
            kv = head // G
            s = (k[:, kv, :] @ q[row, head].to(torch.float64).numpy()) * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            out[row, head] = torch.from_numpy(p @ v[:, kv, :]).to(q.dtype)
    return out


def reference_paged_decode(q, k_cache, v_cache, block_table, seqlen, *, scale: float | None = None,
                           out_dtype=None) -> torch.Tensor:
    """Gather + fp32 einsum oracle (reference ``tests/reference/paged.py:225-274``).

    ``out_dtype=torch.float32`` keeps the fp32 result unrounded, for the 1e-3 bar against
    an fp32 softmax.
    """
    B, H, D = q.shape
    bs = k_cache.shape[1]
    H_kv = k_cache.shape[2]
    G = H // H_kv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty(q.shape, dtype=out_dtype or q.dtype)
    table = block_table.to(torch.long)
    qf = q.to(torch.float32).reshape(B, H_kv, G, D)
    for b in range(B):
        n = int(seqlen[b])
        if n <= 0:
            out[b].zero_()
            continue
        pages = (n + bs - 1) // bs
        ids = table[b, :pages]
        k = k_cache.index_select(0, ids).reshape(pages * bs, H_kv, D)[:n]
        v = v_cache.index_select(0, ids).reshape(pages * bs, H_kv, D)[:n]
        kf = k.to(torch.float32).permute(1, 0, 2)
        vf = v.to(torch.float32).permute(1, 0, 2)
        scores = torch.einsum("hgd,hnd->hgn", qf[b], kf) * scale
        probs = torch.softmax(scores, dim=-1)
        ctx = torch.einsum("hgn,hnd->hgd", probs, vf)
        out[b] = ctx.reshape(H, D).to(out.dtype)
    return out
