"""Packed varlen prefill attention on the HIP MFMA kernel: the CUDA arm of
``model/attention/varlen.py``.

``HipVarlen`` replaces the reference's ``FlashVarlen`` (reference
``model/attention/varlen.py:293-357``) behind the same interface::

    backend.name                                   # provenance string
    backend.prefill_varlen(q, k, v, *, cu_seqlens, max_seqlen,
                           softmax_scale=None, causal=True) -> (total, H, D)

with the same contract: ``q`` ``(total, H, D)``, ``k``/``v`` ``(total, H_kv, D)``;
``cu_seqlens`` a list or 1-D integer tensor starting at 0, strictly increasing, ending at
``total``; ``max_seqlen`` equal to the longest segment; fp16/bf16 only; shape and offset
errors raise ``ValueError`` and device/dtype capability errors ``RuntimeError``
(reference ``:101-233``, ``:331-343``).

The kernel's tile schedule (heaviest causal tiles first) and the device copy of
``cu_seqlens`` depend only on the segment bounds, so they are cached per bounds tuple: the
28 layers of one packed forward upload them once, where the reference re-uploads
``cu_seqlens`` on every call (reference ``:344``).

``backend_for(device)`` selects this arm for CUDA (HIP) devices. CPU/MPS devices are the
reference's ``SdpaVarlen`` arm, which stays the reference's own code; this module has no
CPU implementation and never substitutes one.
"""

from __future__ import annotations

import ctypes
import math
import operator
from collections import OrderedDict
from typing import Sequence

import torch

from . import _lib

__all__ = ["HipVarlen", "backend_for"]


def _as_int(value, name: str) -> int:
    try:
        return operator.index(value)
    except TypeError:
        raise ValueError(f"{name} must be an int, got {type(value).__name__} ({value!r})") from None


def _segment_bounds(cu_seqlens, total_tokens: int) -> list[int]:
    """Validated segment bounds as a list (reference ``:101-158``)."""
    if isinstance(cu_seqlens, torch.Tensor):
        if cu_seqlens.dim() != 1:
            raise ValueError(
                "cu_seqlens must be a 1-D int tensor of n_seqs + 1 offsets, got shape "
                f"{tuple(cu_seqlens.shape)}; the packed layout has no batch dimension"
            )
        if cu_seqlens.dtype.is_floating_point or cu_seqlens.dtype.is_complex:
            raise ValueError(
                f"cu_seqlens must hold integers (token offsets), got dtype {cu_seqlens.dtype}"
            )
        entries = cu_seqlens.tolist()
    else:
        if isinstance(cu_seqlens, (str, bytes)):
            raise ValueError(
                "cu_seqlens must be a sequence of ints or a 1-D int tensor, got "
                f"{type(cu_seqlens).__name__}"
            )
        try:
            entries = list(cu_seqlens)
        except TypeError:
            raise ValueError(
                "cu_seqlens must be a sequence of ints or a 1-D int tensor, got "
                f"{type(cu_seqlens).__name__}"
            ) from None
    bounds = [_as_int(entry, "every cu_seqlens entry") for entry in entries]
    if len(bounds) < 2:
        raise ValueError(
            "cu_seqlens needs n_seqs + 1 entries (one start offset per segment plus the "
            f"final end offset); got {len(bounds)}"
        )
    if bounds[0] != 0:
        raise ValueError(f"cu_seqlens must start at 0, got {bounds[0]} (cu_seqlens={bounds})")
    if bounds[-1] != total_tokens:
        raise ValueError(
            f"cu_seqlens must end at total_tokens={total_tokens} (q.size(0)), got "
            f"{bounds[-1]} (cu_seqlens={bounds})"
        )
    for index in range(1, len(bounds)):
        if bounds[index] <= bounds[index - 1]:
            raise ValueError(
                "cu_seqlens must be strictly increasing (one non-empty segment per request); "
                f"entry {index} is {bounds[index]} after {bounds[index - 1]} (cu_seqlens={bounds})"
            )
    return bounds


def _validate_packed(q, k, v, cu_seqlens, max_seqlen) -> list[int]:
    """Packed-layout checks (reference ``:161-233``); returns the segment bounds."""
    for name, tensor in (("q", q), ("k", k), ("v", v)):
        if not isinstance(tensor, torch.Tensor):
            raise ValueError(f"{name} must be a torch.Tensor, got {type(tensor).__name__}")
        if tensor.dim() != 3:
            raise ValueError(
                "packed prefill takes 3-D (total_tokens, n_head, head_dim) tensors with no "
                f"batch dimension, got {name}.shape={tuple(tensor.shape)}"
            )
    if q.device != k.device or q.device != v.device:
        raise ValueError(
            f"q, k, v must be on the same device, got q={q.device}, k={k.device}, v={v.device}"
        )
    if not q.dtype.is_floating_point:
        raise ValueError(f"packed prefill needs floating-point q/k/v, got dtype {q.dtype}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(
            f"q, k, v must share one dtype, got q={q.dtype}, k={k.dtype}, v={v.dtype}"
        )
    total_tokens, n_head, head_dim = q.shape
    if k.size(0) != total_tokens or v.size(0) != total_tokens:
        raise ValueError(
            "q, k, v must cover the same packed tokens: got "
            f"q={total_tokens}, k={k.size(0)}, v={v.size(0)} rows"
        )
    n_kv_head = k.size(1)
    if k.size(1) != v.size(1):
        raise ValueError(
            f"k and v must have the same number of heads, got k={k.size(1)}, v={v.size(1)}"
        )
    if n_head <= 0 or n_kv_head <= 0:
        raise ValueError(f"n_head and n_kv_head must be positive, got {n_head} and {n_kv_head}")
    if n_head % n_kv_head:
        raise ValueError(
            "n_head must be a multiple of n_kv_head (GQA/MQA); got "
            f"n_head={n_head}, n_kv_head={n_kv_head}"
        )
    if k.size(2) != head_dim or v.size(2) != head_dim:
        raise ValueError(
            f"q, k, v must share head_dim; got q={head_dim}, k={k.size(2)}, v={v.size(2)}"
        )
    bounds = _segment_bounds(cu_seqlens, total_tokens)
    max_seqlen = _as_int(max_seqlen, "max_seqlen")
    lengths = [bounds[i + 1] - bounds[i] for i in range(len(bounds) - 1)]
    longest = max(lengths)
    if max_seqlen != longest:
        raise ValueError(
            f"max_seqlen={max_seqlen} does not match the longest segment ({longest}); "
            f"segment lengths={lengths}. The value is not clamped: it sizes the kernel's "
            "launch and a value smaller than the real maximum would index past a segment."
        )
    return bounds


def _resolve_scale(softmax_scale, head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)


class _ScheduleCache:
    """Small LRU of the device ``cu_seqlens``, the device schedule and its header counts
    (work pieces, merges, partials, workspace bytes) per packed group."""

    def __init__(self, capacity: int = 8) -> None:
        self.capacity = capacity
        self._items: OrderedDict = OrderedDict()

    def get(self, bounds: list[int], H: int, H_kv: int, D: int, causal: bool, device, kernel: int = -1):
        key = (tuple(bounds), H, H_kv, D, bool(causal), str(device), kernel)
        hit = self._items.get(key)
        if hit is not None:
            self._items.move_to_end(key)
            return hit
        n_seqs = len(bounds) - 1
        host_cu = (ctypes.c_int32 * len(bounds))(*bounds)
        words = _lib.lib.mi_varlen_schedule_for(host_cu, n_seqs, H, H_kv, D, int(causal), kernel, None, 0)
        if words < 0:
            _lib.check(words, "prefill_varlen schedule")
        host_sched = (ctypes.c_int32 * words)()
        rc = _lib.lib.mi_varlen_schedule_for(host_cu, n_seqs, H, H_kv, D, int(causal), kernel, host_sched,
                                             words)
        if rc < 0:
            _lib.check(rc, "prefill_varlen schedule")
        ws_bytes = int(_lib.lib.mi_varlen_workspace_size(host_sched, H))
        cu = torch.tensor(bounds, dtype=torch.int32).to(device)
        sched = torch.frombuffer(bytearray(host_sched), dtype=torch.int32).to(device)
        entry = (cu, sched, int(host_sched[0]), int(host_sched[1]), int(host_sched[2]), int(host_sched[3]),
                 ws_bytes)
        self._items[key] = entry
        if len(self._items) > self.capacity:
            self._items.popitem(last=False)
        return entry


_SCHEDULES = _ScheduleCache()


class HipVarlen:
    """The HIP MFMA varlen kernel (``mi_varlen_prefill``): replaces ``FlashVarlen``."""

    name = "hip-mfma-varlen"

    #: kernel names accepted by ``HipVarlen(kernel=...)``; ``None`` lets the library choose
    KERNELS = {None: -1, "staged": 0, "ring": 1, "wide": 2, "duo": 3}

    def __init__(self, kernel: str | None = None) -> None:
        _lib.require_library("the hip-mfma-varlen prefill backend")
        if kernel not in self.KERNELS:
            raise ValueError(f"unknown prefill kernel {kernel!r}; choose one of {sorted(k for k in self.KERNELS if k)}")
        self._kernel = self.KERNELS[kernel]

    def prefill_varlen(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        *,
        cu_seqlens: Sequence[int] | torch.Tensor,
        max_seqlen: int,
        softmax_scale: float | None = None,
        causal: bool = True,
    ) -> torch.Tensor:
        """Attend within each packed segment; return ``(total_tokens, n_head, head_dim)``."""
        bounds = _validate_packed(q, k, v, cu_seqlens, max_seqlen)
        scale = _resolve_scale(softmax_scale, q.size(-1))
        if not (q.is_cuda and k.is_cuda and v.is_cuda):
            raise RuntimeError(
                "HipVarlen is the CUDA (HIP) kernel path, but q/k/v are on "
                f"{q.device}/{k.device}/{v.device}. Use the reference SdpaVarlen on CPU/MPS; "
                "there is no fallback here."
            )
        if q.dtype not in (torch.float16, torch.bfloat16):
            raise RuntimeError(
                f"the MFMA varlen kernel computes fp16/bf16 only, got q.dtype={q.dtype}. Cast "
                "the packed batch to bf16/fp16, or run the fp32 check against the SDPA arm."
            )
        q = q.contiguous()
        k = k.contiguous()
        v = v.contiguous()
        total, H, D = q.shape
        H_kv = k.size(1)
        cu, sched, n_work, n_merge, n_partials, layout, ws_bytes = _SCHEDULES.get(
            bounds, H, H_kv, D, causal, q.device, self._kernel)
        out = torch.empty_like(q)
        # split-tile partials, consumed by the merge launch on the same stream
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
        rc = _lib.lib.mi_varlen_prefill(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), cu.data_ptr(),
            len(bounds) - 1, total, int(max_seqlen), sched.data_ptr(), n_work, n_merge, n_partials,
            layout, H, H_kv, D, float(scale), int(bool(causal)), _lib.dtype_code(q.dtype),
            ws.data_ptr() if ws is not None else None, ws_bytes, _lib.current_stream(q.device),
        )
        _lib.check(rc, "prefill_varlen")
        return out


def backend_for(device) -> HipVarlen:
    """Arm selection by device type (reference ``:360-381``): CUDA (HIP) -> ``HipVarlen``.

    CPU/MPS stay on the reference's ``SdpaVarlen`` arm, which this package does not
    re-implement; asking it for one is an error rather than a silent substitute.
    """
    resolved = device if isinstance(device, torch.device) else torch.device(device)
    if resolved.type == "cuda":
        return HipVarlen()
    raise ValueError(
        f"no packed-prefill backend for device {resolved!s} (type {resolved.type!r}) in the "
        "HIP package; CPU/MPS prefill is the reference's SdpaVarlen arm."
    )
