"""Packed whole-prompt prefill container: the drop-in for ``model/packed.py``.

``PackedPrefill`` (reference ``model/packed.py:85-222``) carries one FIFO group of whole
prompts through a forward on a single packed token axis: it owns ``cu_seqlens``, the
request-local RoPE positions and one write sink per request; per layer it hands the packed
K/V to the sinks (``write``) and runs the varlen backend (``attend``). With no backend given
it takes ``backend_for(positions.device)``: the HIP kernel on a HIP device, per-segment SDPA
on the host.

Group write: when every sink is a paged sink of one pool (the engine's group prefill), the
whole group's K/V goes through **one** slot-write launch with the members' slot maps
concatenated, instead of one launch per request per layer; the bytes written are the same
as the per-sink loop's. ``write_rope`` additionally fuses the layer's q/k norm and RoPE into
that launch.
"""

from __future__ import annotations

from typing import Sequence

import torch

__all__ = ["PackedPrefill", "as_packed_prefill", "PACKED_PREFILL_FLAG"]

#: attribute a container sets to opt into the packed-prefill protocol
PACKED_PREFILL_FLAG = "packed_prefill"

_HOOKS = ("cu_seqlens", "positions", "last_token_index", "total_tokens", "n_seqs", "past_len", "write", "attend")


def as_packed_prefill(past):
    """``past`` when it opts into the packed protocol, else ``None``; an object that opts in
    but lacks a hook is a caller bug (``TypeError``) (reference ``model/packed.py:65-82``)."""
    if past is None or not getattr(past, PACKED_PREFILL_FLAG, False):
        return None
    missing = [h for h in _HOOKS if not hasattr(past, h)]
    if missing:
        raise TypeError(f"container {type(past).__name__} sets {PACKED_PREFILL_FLAG}=True but is missing "
                        f"packed-prefill hook(s) {missing}")
    return past


def _request_local(cu: list[int]) -> torch.Tensor:
    """Positions 0..L-1 of every segment, concatenated."""
    lengths = torch.tensor([b - a for a, b in zip(cu, cu[1:])])
    starts = torch.tensor(cu[:-1])
    seg = torch.repeat_interleave(torch.arange(len(lengths)), lengths)
    return torch.arange(cu[-1]) - starts[seg]


class PackedPrefill:
    """One varlen forward over a FIFO group of whole prompts."""

    packed_prefill = True

    def __init__(self, *, cu_seqlens: Sequence[int], positions: torch.Tensor, sinks: Sequence[object],
                 backend=None) -> None:
        cu = [int(c) for c in cu_seqlens]
        if len(cu) < 2:
            raise ValueError("PackedPrefill needs at least one request (cu_seqlens length >= 2)")
        if cu[0] != 0:
            raise ValueError(f"cu_seqlens must start at 0, got {cu[0]}")
        if min(b - a for a, b in zip(cu, cu[1:])) <= 0:
            raise ValueError(f"cu_seqlens must be strictly increasing, got {cu}")
        sinks = list(sinks)
        if len(sinks) != len(cu) - 1:
            raise ValueError(f"PackedPrefill needs one sink per request ({len(cu) - 1}), got {len(sinks)}")
        total = cu[-1]
        if positions.dim() != 1 or positions.numel() != total:
            raise ValueError(f"positions must be a 1-D tensor of {total} entries, got {tuple(positions.shape)}")
        positions = positions.long()
        # positions restart at 0 in every request (one host comparison per group)
        wrong = (positions.cpu() != _request_local(cu)).nonzero()
        if wrong.numel():
            t = int(wrong[0, 0])
            row = max(i for i in range(len(cu) - 1) if cu[i] <= t)
            raise ValueError(f"request {row}: positions must be request-local 0..{cu[row + 1] - cu[row] - 1} "
                             "(a packed layout does not share one increasing position axis)")
        if backend is None:
            from .varlen import backend_for

            backend = backend_for(positions.device)
        self.backend = backend
        self.cu_seqlens = cu
        self.positions = positions
        self.sinks = sinks
        self.total_tokens = total
        self.n_seqs = len(sinks)
        self.max_seqlen = max(b - a for a, b in zip(cu, cu[1:]))
        self.rope_len = self.max_seqlen
        self.last_token_index = torch.tensor(cu[1:], dtype=torch.long, device=positions.device) - 1
        self._group = self._one_pool_slots()

    def _one_pool_slots(self):
        """``(pool, slots)`` when every sink writes one paged pool through a slot map."""
        pools = {id(getattr(s, "pool", None)) for s in self.sinks}
        if len(pools) != 1 or not all(getattr(s, "slots", None) is not None for s in self.sinks):
            return None
        pool = self.sinks[0].pool
        if not hasattr(pool, "write_slots"):
            return None
        return pool, torch.cat([s.slots.long() for s in self.sinks])

    @property
    def group_slots(self) -> torch.Tensor | None:
        """The concatenated slot map of a one-pool group (``None`` otherwise)."""
        return None if self._group is None else self._group[1]

    def _claim_all(self, layer: int) -> None:
        """Mark ``layer`` written in every sink, refusing before any mark if one already is."""
        if any(getattr(s, "_written", [False] * (layer + 1))[layer] for s in self.sinks):
            raise RuntimeError(f"layer {layer} was already written: a paged sink holds exactly one whole prompt "
                               "(past_len == 0)")
        for sink in self.sinks:
            claim = getattr(sink, "claim", None)
            if claim is not None:
                claim(layer)

    # ---------------------------------------------------------------- layer hooks
    def past_len(self, layer: int | None = None) -> int:
        return 0

    def get_kv(self, layer: int) -> tuple[None, None]:
        return (None, None)

    def _segments(self):
        return zip(self.sinks, self.cu_seqlens, self.cu_seqlens[1:])

    def set_kv(self, layer: int, kv) -> None:
        """Dense ``(1, H_kv, total, D)`` hook of the ordinary cache protocol, split by request."""
        k, v = kv
        if k.dim() != 4 or k.shape[0] != 1:
            raise ValueError(f"set_kv needs (1, H, L, D) k/v, got {tuple(k.shape)}")
        for sink, a, b in self._segments():
            sink.set_kv(layer, (k[:, :, a:b], v[:, :, a:b]))

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write each request's part of the packed ``(1, total, H_kv, D)`` k/v of one layer
        (reference ``model/packed.py:187-202``)."""
        if k.dim() != 4 or k.shape[0] != 1 or k.shape[1] != self.total_tokens:
            raise ValueError(f"write needs packed (1, {self.total_tokens}, H, D) k/v, got "
                             f"{tuple(k.shape)} / {tuple(v.shape)}")
        if k.shape != v.shape:
            raise ValueError(f"k/v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
        if self._group is not None:
            pool, slots = self._group
            self._claim_all(layer)
            pool.write_prefill_slots(layer, slots, k[0], v[0])
            return
        for sink, a, b in self._segments():
            sink.set_kv(layer, (k[0, a:b].transpose(0, 1).unsqueeze(0), v[0, a:b].transpose(0, 1).unsqueeze(0)))

    def write_rope(self, layer: int, qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                   cos: torch.Tensor, sin: torch.Tensor, eps: float, *, rotary_dim: int | None = None,
                   zero_centred_norm: bool = False):
        """This layer's q/k norm + RoPE at each token's request-local position and the group's
        K/V write in one HIP launch (``PagedPool.write_qk_norm_rope`` over the packed projection
        ``qkv`` ``(total, (H + 2 H_kv) D)``), in place of the tensor ops and :meth:`write`.
        Needs one paged pool behind every sink. Returns packed ``(1, total, H, D)`` q and
        ``(1, total, H_kv, D)`` k and v for :meth:`attend`."""
        if self._group is None:
            raise RuntimeError("write_rope needs every sink on one paged pool (use write() otherwise)")
        pool, slots = self._group
        self._claim_all(layer)
        shape = (self.total_tokens, pool.n_kv_head, pool.head_dim)
        k = torch.empty(shape, dtype=pool.dtype, device=qkv.device)
        v = torch.empty_like(k)
        q = pool.write_qk_norm_rope(layer, slots, qkv, q_norm_w, k_norm_w, cos, sin, self.positions, eps,
                                    k_out=k, v_out=v, rotary_dim=rotary_dim, zero_centred_norm=zero_centred_norm)
        return q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)

    def attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """Causal attention inside each request over the packed axis (reference
        ``model/packed.py:204-218``)."""
        if q.dim() != 4 or q.shape[0] != 1 or q.shape[1] != self.total_tokens:
            raise ValueError(f"attend needs packed (1, {self.total_tokens}, H, D) q, got {tuple(q.shape)}")
        out = self.backend.prefill_varlen(q[0].contiguous(), k[0].contiguous(), v[0].contiguous(),
                                          cu_seqlens=self.cu_seqlens, max_seqlen=self.max_seqlen, causal=True)
        return out.unsqueeze(0)

    @property
    def backend_name(self) -> str:
        return str(getattr(self.backend, "name", type(self.backend).__name__))
