"""Packed whole-prompt prefill container on the HIP varlen kernel.

Drop-in for the reference's ``model/packed.py`` (``PackedPrefill`` ``:85-222``,
``as_packed_prefill`` ``:65-82``): it owns ``cu_seqlens``, the request-local RoPE
positions and one write sink per request, slices each layer's packed K/V to the sinks and
runs the varlen backend over the packed token axis. The default backend is
:class:`miattn.varlen.HipVarlen` (via ``backend_for(positions.device)``).

One addition, ``write_packed``: when every sink is a paged sink of the same pool (the
engine's group prefill), the whole group's K/V is written by **one** slot-write launch over
the packed token axis with one concatenated slot map, instead of one launch per request
per layer. The bytes written are identical to the per-sink loop (a pure copy through the
same slot maps).
"""

from __future__ import annotations

from typing import Sequence

import torch

__all__ = ["PackedPrefill", "as_packed_prefill", "PACKED_PREFILL_FLAG"]

PACKED_PREFILL_FLAG = "packed_prefill"

_PACKED_HOOKS = (
    "cu_seqlens", "positions", "last_token_index", "total_tokens", "n_seqs", "past_len",
    "write", "attend",
)


def as_packed_prefill(past):
    """``past`` if it is a packed-prefill container, else ``None`` (reference ``:65-82``)."""
    if past is None or not getattr(past, PACKED_PREFILL_FLAG, False):
        return None
    missing = [name for name in _PACKED_HOOKS if not hasattr(past, name)]
    if missing:
        raise TypeError(
            f"container {type(past).__name__} sets {PACKED_PREFILL_FLAG}=True but is missing "
            f"packed-prefill hook(s) {missing}; implement the PackedPrefill protocol or drop the flag"
        )
    return past


class PackedPrefill:
    """One varlen forward over a FIFO group of whole prompts."""

    packed_prefill = True

    def __init__(self, *, cu_seqlens: Sequence[int], positions: torch.Tensor,
                 sinks: Sequence[object], backend=None) -> None:
        cumulative = [int(value) for value in cu_seqlens]
        if len(cumulative) < 2:
            raise ValueError("PackedPrefill needs at least one request (cu_seqlens length >= 2)")
        if cumulative[0] != 0:
            raise ValueError(f"cu_seqlens must start at 0, got {cumulative[0]}")
        if any(b <= a for a, b in zip(cumulative, cumulative[1:])):
            raise ValueError(f"cu_seqlens must be strictly increasing, got {cumulative}")
        total = cumulative[-1]
        if len(sinks) != len(cumulative) - 1:
            raise ValueError(
                f"PackedPrefill needs one sink per request ({len(cumulative) - 1}), got {len(sinks)}"
            )
        if positions.dim() != 1 or int(positions.numel()) != total:
            raise ValueError(
                f"positions must be a 1-D tensor of {total} entries, got {tuple(positions.shape)}"
            )
        positions = positions.to(dtype=torch.long)
        expected = torch.cat([torch.arange(b - a, dtype=torch.long) for a, b in zip(cumulative, cumulative[1:])])
        got = positions.cpu()
        if not torch.equal(got, expected):
            bad = int((got != expected).nonzero()[0, 0])
            row = next(i for i in range(len(cumulative) - 1) if cumulative[i] <= bad < cumulative[i + 1])
            start, end = cumulative[row], cumulative[row + 1]
            raise ValueError(
                f"request {row}: positions must be request-local 0..{end - start - 1} "
                "(a packed layout does not share one increasing position axis)"
            )
        if backend is None:
            from .varlen import backend_for

            backend = backend_for(positions.device)
        self.backend = backend
        self.cu_seqlens = cumulative
        self.positions = positions
        self.sinks = list(sinks)
        self.total_tokens = total
        self.n_seqs = len(self.sinks)
        self.max_seqlen = max(b - a for a, b in zip(cumulative, cumulative[1:]))
        self.rope_len = max(self.max_seqlen, 1)
        self.last_token_index = torch.tensor(
            [end - 1 for end in cumulative[1:]], dtype=torch.long, device=positions.device
        )
        self._packed_slots = self._group_slot_map()

    def _group_slot_map(self):
        """One slot map over the packed axis when every sink writes one pool's blocks."""
        pools = {id(getattr(sink, "pool", None)) for sink in self.sinks}
        if len(pools) != 1 or any(getattr(sink, "slots", None) is None for sink in self.sinks):
            return None
        pool = self.sinks[0].pool
        if not hasattr(pool, "write_slots"):
            return None
        return pool, torch.cat([sink.slots.to(torch.long) for sink in self.sinks])

    # ---------------------------------------------------------------- layer hooks
    def past_len(self, layer: int | None = None) -> int:
        return 0

    def get_kv(self, layer: int) -> tuple[None, None]:
        return (None, None)

    def set_kv(self, layer: int, kv) -> None:
        """Dense ``(1, H, L, D)`` compatibility hook, split over the sinks (reference ``:171-185``)."""
        k, v = kv
        if k.dim() != 4 or k.shape[0] != 1:
            raise ValueError(f"set_kv needs (1, H, L, D) k/v, got {tuple(k.shape)}")
        start = 0
        for sink, end in zip(self.sinks, self.cu_seqlens[1:]):
            sink.set_kv(layer, (k[:, :, start:end], v[:, :, start:end]))
            start = end

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write each request's K/V of one layer (reference ``:187-202``).

        ``k``/``v`` are packed ``(1, total, H_kv, D)``. A group whose sinks share one paged
        pool is written by one slot-write launch (see the module docstring); any other
        sink mix goes through each sink's ``set_kv``.
        """
        if k.dim() != 4 or k.shape[0] != 1 or k.shape[1] != self.total_tokens:
            raise ValueError(
                f"write needs packed (1, {self.total_tokens}, H, D) k/v, got "
                f"{tuple(k.shape)} / {tuple(v.shape)}"
            )
        if tuple(k.shape) != tuple(v.shape):
            raise ValueError(f"k/v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
        if self._packed_slots is not None:
            pool, slots = self._packed_slots
            for sink in self.sinks:
                written = getattr(sink, "_written", None)
                if written is not None:
                    if written[layer]:
                        raise RuntimeError(
                            f"layer {layer} was already written: the paged write-through sink "
                            "holds exactly one full prefill (past_len == 0)"
                        )
            pool.write_prefill_slots(layer, slots, k[0], v[0])
            for sink in self.sinks:
                written = getattr(sink, "_written", None)
                if written is not None:
                    written[layer] = True
            return
        start = 0
        for sink, end in zip(self.sinks, self.cu_seqlens[1:]):
            layer_k = k[0, start:end].transpose(0, 1).unsqueeze(0)
            layer_v = v[0, start:end].transpose(0, 1).unsqueeze(0)
            sink.set_kv(layer, (layer_k, layer_v))
            start = end

    def write_rope(self, layer: int, qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                   cos: torch.Tensor, sin: torch.Tensor, eps: float):
        """This layer's q/k RMSNorm + RoPE (at each token's request-local position) and the
        group's K/V write in one HIP launch (``PagedPool.write_qk_norm_rope`` over the packed
        projection ``qkv`` ``(total, (H + 2 H_kv) D)``), in place of the reference's tensor
        ops and :meth:`write`. Needs one paged pool behind every sink. Returns packed
        ``(1, total, H, D)`` q and ``(1, total, H_kv, D)`` k and v for :meth:`attend`."""
        if self._packed_slots is None:
            raise RuntimeError("write_rope needs every sink on one paged pool (use write() otherwise)")
        pool, slots = self._packed_slots
        for sink in self.sinks:
            written = getattr(sink, "_written", None)
            if written is not None and written[layer]:
                raise RuntimeError(
                    f"layer {layer} was already written: the paged write-through sink holds exactly one "
                    "full prefill (past_len == 0)"
                )
        T = self.total_tokens
        k = torch.empty((T, pool.n_kv_head, pool.head_dim), dtype=pool.dtype, device=qkv.device)
        v = torch.empty_like(k)
        q = pool.write_qk_norm_rope(layer, slots, qkv, q_norm_w, k_norm_w, cos, sin, self.positions, eps,
                                    k_out=k, v_out=v)
        for sink in self.sinks:
            written = getattr(sink, "_written", None)
            if written is not None:
                written[layer] = True
        return q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)

    def attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """Per-request causal attention over the packed axis (reference ``:204-218``)."""
        if q.dim() != 4 or q.shape[0] != 1 or q.shape[1] != self.total_tokens:
            raise ValueError(f"attend needs packed (1, {self.total_tokens}, H, D) q, got {tuple(q.shape)}")
        out = self.backend.prefill_varlen(
            q[0].contiguous(), k[0].contiguous(), v[0].contiguous(),
            cu_seqlens=self.cu_seqlens, max_seqlen=self.max_seqlen, causal=True,
        )
        return out.unsqueeze(0)

    @property
    def backend_name(self) -> str:
        return str(getattr(self.backend, "name", type(self.backend).__name__))
