"""The reference's CPU seat path (contiguous KV slab + hand_baddbmm decode). Test
infrastructure only; also the CPU baseline that ``bench.py`` times.

Restated in the reference's operation order, because the seat path's numerics (bf16
softmax, scale folded into q) are what the GPU path's greedy tokens are compared against:

* :class:`SeatSlab` -- one ``(B, H_kv, max_len, D)`` K/V buffer per layer, ``scatter_``
  write at ``pos`` (reference ``model/slab.py:251-266``), bool allow-mask
  ``column < (valid + next_token) * active`` turned into the additive bias once per step
  (``:302-328``), ``advance`` by ``active`` (``:227-248``);
* :func:`additive_bias` -- mask -> 0 / -inf bias, rows with no allowed key zeroed
  (reference ``model/attention/hand_baddbmm.py:129-149``);
* :func:`seat_decode` -- ``q * (1/sqrt(D))`` -> ``baddbmm(bias, q, k^T)`` -> softmax in the
  input dtype -> ``bmm(p, v)``, GQA kept unexpanded as ``(B*H_kv, G, .)`` (reference
  ``model/attention/hand_baddbmm.py:80-126``).

Pinned by: agreement with the float64 decode oracle within the bf16 tolerance and exactly
(fp32 inputs, 1e-5) when run in fp32; a dead row (no allowed key) decodes to the mean of V
rather than NaN, as the zeroed bias implies; checked in ``tests/test_oracle_seat.py``.
"""

from __future__ import annotations

import math

import torch

__all__ = ["SeatSlab", "additive_bias", "seat_decode"]


def additive_bias(mask: torch.Tensor, dtype, B: int, H_kv: int, G: int) -> torch.Tensor:
    alive = mask.any(dim=-1, keepdim=True)
    bias = torch.where(mask, 0.0, float("-inf"))
    bias = torch.where(alive, bias, 0.0)
    L = bias.shape[-1]
    return bias.to(dtype).expand(B, H_kv, G, L).reshape(B * H_kv, G, L)


def seat_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """``q`` ``(B, H, 1, D)`` against ``k``/``v`` ``(B, H_kv, L, D)``; returns ``(B, H, 1, D)``."""
    B, H, _, D = q.shape
    H_kv, L = k.shape[1], k.shape[2]
    G = H // H_kv
    qg = (q * (1.0 / math.sqrt(D))).reshape(B * H_kv, G, D)
    kT = k.transpose(-2, -1).reshape(B * H_kv, D, L)
    vg = v.reshape(B * H_kv, L, D)
    scores = torch.bmm(qg, kT) if bias is None else torch.baddbmm(bias, qg, kT, beta=1.0, alpha=1.0)
    probs = torch.softmax(scores, dim=-1)
    return torch.bmm(probs, vg).reshape(B, H, 1, D)


class SeatSlab:
    """Minimal ``KvSlab``: fixed K/V buffers per layer, per-row cursors, mask and bias."""

    def __init__(self, n_layer: int, batch: int, n_kv_head: int, head_dim: int, max_len: int, *,
                 dtype=torch.float32, n_head: int | None = None) -> None:
        self.n_layer, self.batch, self.n_kv_head, self.head_dim, self.max_len = n_layer, batch, n_kv_head, head_dim, max_len
        self.n_head = n_kv_head if n_head is None else n_head
        self.n_group = self.n_head // n_kv_head
        self.dtype = dtype
        shape = (batch, n_kv_head, max_len, head_dim)
        self.keys = [torch.zeros(shape, dtype=dtype) for _ in range(n_layer)]
        self.values = [torch.zeros(shape, dtype=dtype) for _ in range(n_layer)]
        self.pos = torch.zeros(batch, dtype=torch.long)
        self.valid = torch.zeros(batch, dtype=torch.long)
        self.active = torch.ones(batch, dtype=torch.bool)
        self.mask = torch.zeros(batch, 1, 1, max_len, dtype=torch.bool)
        self.bias = torch.zeros(batch * n_kv_head, self.n_group, max_len, dtype=dtype)
        self._columns = self.pos.view(-1, 1, 1, 1).expand(batch, n_kv_head, 1, head_dim)
        self._positions = torch.arange(max_len).view(1, 1, 1, max_len)

    def activate(self, row: int, length: int) -> None:
        self.pos[row] = length
        self.valid[row] = length
        self.active[row] = True

    def freeze(self, row: int) -> None:
        self.pos[row] = 0
        self.valid[row] = 0
        self.active[row] = False

    def build_mask(self, *, next_token: bool = False) -> torch.Tensor:
        limit = (self.valid + int(next_token)) * self.active
        if int(limit.max()) > self.max_len:
            raise IndexError(f"KvSlab overflow: needs {int(limit.max())} columns, max_len={self.max_len}")
        self.mask.copy_((self._positions < limit.view(-1, 1, 1, 1)).expand_as(self.mask))
        self.bias.copy_(additive_bias(self.mask, self.dtype, self.batch, self.n_kv_head, self.n_group))
        return self.mask

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        self.keys[layer].scatter_(2, self._columns, k.to(self.dtype))
        self.values[layer].scatter_(2, self._columns, v.to(self.dtype))

    def attend(self, layer: int, q: torch.Tensor) -> torch.Tensor:
        return seat_decode(q, self.keys[layer], self.values[layer], self.bias)

    def advance(self) -> None:
        self.pos.add_(self.active)
        self.valid.copy_(torch.maximum(self.valid, self.pos))
