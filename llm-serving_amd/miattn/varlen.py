"""Packed varlen causal prefill attention: the arms of ``model/attention/varlen.py``.

Every arm answers the reference's backend interface (``model/attention/varlen.py:259-357``)::

    backend.name                                             # provenance string
    backend.prefill_varlen(q, k, v, *, cu_seqlens, max_seqlen,
                           softmax_scale=None, causal=True) -> (total, H, D)

``q`` is ``(total, H, D)`` and ``k``/``v`` ``(total, H_kv, D)`` over one packed token axis;
``cu_seqlens`` (a sequence or a 1-D integer tensor) starts at 0, increases strictly and ends
at ``total``; ``max_seqlen`` equals the longest segment. Layout and offset mistakes raise
``ValueError``; a device or dtype the arm cannot compute raises ``RuntimeError``.

* :class:`HipVarlen` -- the HIP MFMA kernel ``mi_varlen_prefill`` (``include/miattn.h``),
  standing in for the reference's CUDA arm ``FlashVarlen``. fp16/bf16 on a HIP device.
* :class:`SdpaVarlen` -- one ``scaled_dot_product_attention`` per segment, the reference's
  arm for CPU/MPS devices. It is selected by device type only: a tensor on a HIP device
  never reaches it.
* :func:`backend_for` -- the reference's device-type dispatch: ``cuda`` -> ``HipVarlen``,
  ``cpu``/``mps`` -> ``SdpaVarlen``.

The HIP kernel's tile schedule and the device copy of ``cu_seqlens`` depend only on the
segment lengths, so they are built once per packed group and reused by all of its layers
(the reference uploads ``cu_seqlens`` on every call).
"""

from __future__ import annotations

import ctypes
import math
from collections import OrderedDict
from types import SimpleNamespace
from typing import Sequence

import torch
import torch.nn.functional as F

from . import _lib
from ._contract import Rule, as_index, enforce

__all__ = ["HipVarlen", "SdpaVarlen", "backend_for", "check_prefill_errors", "segment_bounds", "validate_packed"]


def _entries(cu_seqlens) -> list:
    """The raw offsets of ``cu_seqlens`` as a Python list (not yet checked as integers)."""
    if isinstance(cu_seqlens, torch.Tensor):
        if cu_seqlens.dim() != 1:
            raise ValueError("cu_seqlens must be a 1-D int tensor of n_seqs + 1 offsets (the packed layout has "
                             f"no batch dimension), got shape {tuple(cu_seqlens.shape)}")
        if cu_seqlens.dtype.is_floating_point or cu_seqlens.dtype.is_complex:
            raise ValueError(f"cu_seqlens must hold integers (token offsets), got dtype {cu_seqlens.dtype}")
        return cu_seqlens.tolist()
    if isinstance(cu_seqlens, (str, bytes)) or not hasattr(cu_seqlens, "__iter__"):
        raise ValueError(f"cu_seqlens must be a sequence of ints or a 1-D int tensor, got {type(cu_seqlens).__name__}")
    return list(cu_seqlens)


def segment_bounds(cu_seqlens, total_tokens: int) -> list[int]:
    """``cu_seqlens`` checked against the packed-prefill contract, as a list of ints:
    ``0 = c[0] < c[1] < ... < c[n] = total_tokens`` (every segment non-empty)."""
    c = [as_index(x, "every cu_seqlens entry") for x in _entries(cu_seqlens)]
    if len(c) < 2:
        raise ValueError(f"cu_seqlens needs n_seqs + 1 entries (segment starts plus the final end), got {len(c)}")
    if c[0] != 0:
        raise ValueError(f"cu_seqlens must start at 0, got {c[0]} (cu_seqlens={c})")
    if c[-1] != total_tokens:
        raise ValueError(f"cu_seqlens must end at total_tokens={total_tokens} (q.size(0)), got {c[-1]} "
                         f"(cu_seqlens={c})")
    steps = [b - a for a, b in zip(c, c[1:])]
    flat = next((i for i, n in enumerate(steps) if n <= 0), None)
    if flat is not None:
        raise ValueError(f"cu_seqlens must be strictly increasing (one non-empty segment per request): entry "
                         f"{flat + 1} is {c[flat + 1]} after {c[flat]} (cu_seqlens={c})")
    return c


_PACKED = (
    Rule(lambda a: not all(isinstance(t, torch.Tensor) for t in (a.q, a.k, a.v)), ValueError,
         lambda a: "q, k and v must be torch.Tensors"),
    Rule(lambda a: any(t.dim() != 3 for t in (a.q, a.k, a.v)), ValueError,
         lambda a: "packed prefill takes 3-D (total_tokens, heads, head_dim) tensors with no batch dimension, got "
                   f"q {tuple(a.q.shape)}, k {tuple(a.k.shape)}, v {tuple(a.v.shape)}"),
    Rule(lambda a: not (a.q.device == a.k.device == a.v.device), ValueError,
         lambda a: f"q, k, v must be on the same device, got {a.q.device}, {a.k.device}, {a.v.device}"),
    Rule(lambda a: not a.q.dtype.is_floating_point, ValueError,
         lambda a: f"packed prefill needs floating-point q/k/v, got dtype {a.q.dtype}"),
    Rule(lambda a: not (a.q.dtype == a.k.dtype == a.v.dtype), ValueError,
         lambda a: f"q, k, v must share one dtype, got {a.q.dtype}, {a.k.dtype}, {a.v.dtype}"),
    Rule(lambda a: not (a.q.shape[0] == a.k.shape[0] == a.v.shape[0]), ValueError,
         lambda a: f"q, k, v must cover the same packed tokens, got {a.q.shape[0]}, {a.k.shape[0]}, {a.v.shape[0]} rows"),
    Rule(lambda a: a.k.shape[1] != a.v.shape[1], ValueError,
         lambda a: f"k and v must have the same number of heads, got {a.k.shape[1]} and {a.v.shape[1]}"),
    Rule(lambda a: a.q.shape[1] < 1 or a.k.shape[1] < 1, ValueError,
         lambda a: f"n_head and n_kv_head must be positive, got {a.q.shape[1]} and {a.k.shape[1]}"),
    Rule(lambda a: a.q.shape[1] % a.k.shape[1] != 0, ValueError,
         lambda a: f"n_head must be a multiple of n_kv_head (GQA/MQA), got {a.q.shape[1]} and {a.k.shape[1]}"),
    Rule(lambda a: not (a.q.shape[2] == a.k.shape[2] == a.v.shape[2]), ValueError,
         lambda a: f"q, k, v must share head_dim, got {a.q.shape[2]}, {a.k.shape[2]}, {a.v.shape[2]}"),
)


def validate_packed(q, k, v, cu_seqlens, max_seqlen) -> list[int]:
    """Apply the packed layout contract; returns the segment bounds."""
    enforce(_PACKED, SimpleNamespace(q=q, k=k, v=v))
    bounds = segment_bounds(cu_seqlens, int(q.shape[0]))
    longest = max(b - a for a, b in zip(bounds, bounds[1:]))
    claimed = as_index(max_seqlen, "max_seqlen")
    if claimed != longest:
        raise ValueError(f"max_seqlen={claimed} does not match the longest segment ({longest}); it is not clamped, "
                         "because it sizes the launch and a smaller value would cut segments short")
    return bounds


def _scale(softmax_scale, head_dim: int) -> float:
    return float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(head_dim)


class SdpaVarlen:
    """Per-segment ``F.scaled_dot_product_attention``: the reference's CPU/MPS arm
    (``model/attention/varlen.py:259-290``). Each segment is its own ``(1, H, L, D)``
    attention problem, so no query sees another request's keys."""

    name = "sdpa-varlen"

    def prefill_varlen(self, q, k, v, *, cu_seqlens: Sequence[int] | torch.Tensor, max_seqlen: int,
                       softmax_scale: float | None = None, causal: bool = True):
        bounds = validate_packed(q, k, v, cu_seqlens, max_seqlen)
        scale = _scale(softmax_scale, q.shape[-1])
        gqa = q.shape[1] != k.shape[1]
        out = torch.empty_like(q)
        for a, b in zip(bounds, bounds[1:]):
            qs, ks, vs = (t[a:b].transpose(0, 1).unsqueeze(0) for t in (q, k, v))
            y = F.scaled_dot_product_attention(qs, ks, vs, dropout_p=0.0, is_causal=bool(causal), scale=scale,
                                               enable_gqa=gqa)
            out[a:b] = y[0].transpose(0, 1)
        return out


class _Schedules:
    """LRU of per-group launch state: the device ``cu_seqlens``, the device schedule, its
    four header words and the split-piece workspace size.

    A schedule used while a HIP graph is being captured is pinned for the life of the
    process: the graph keeps its raw device pointers, so evicting it would let a replay
    read freed memory.
    """

    def __init__(self, capacity: int = 8) -> None:
        self.capacity = capacity
        self._lru: OrderedDict = OrderedDict()
        self._pinned: dict = {}

    def get(self, bounds: list[int], H: int, H_kv: int, D: int, causal: bool, device, kernel: int):
        key = (tuple(bounds), H, H_kv, D, bool(causal), str(device), kernel)
        entry = self._pinned.get(key) or self._lru.get(key)
        if entry is None:
            entry = self._build(bounds, H, H_kv, D, causal, device, kernel)
            self._lru[key] = entry
            while len(self._lru) > self.capacity:
                self._lru.popitem(last=False)
        elif key in self._lru:
            self._lru.move_to_end(key)
        if torch.cuda.is_current_stream_capturing():
            self._pinned[key] = entry
        return entry

    @staticmethod
    def _build(bounds, H, H_kv, D, causal, device, kernel):
        # the workspace lives with the schedule: the tall kernel's split-item counters at
        # its head must be zero before the first launch (every launch leaves them zero), so
        # it is zeroed once here and reused by every call of this packed group
        n_seqs = len(bounds) - 1
        host_cu = (ctypes.c_int32 * len(bounds))(*bounds)
        n_words = _lib.lib.mi_varlen_schedule_for(host_cu, n_seqs, H, H_kv, D, int(causal), kernel, None, 0)
        if n_words < 0:
            _lib.check(n_words, "prefill_varlen schedule")
        words = (ctypes.c_int32 * n_words)()
        rc = _lib.lib.mi_varlen_schedule_for(host_cu, n_seqs, H, H_kv, D, int(causal), kernel, words, n_words)
        if rc < 0:
            _lib.check(rc, "prefill_varlen schedule")
        ws_bytes = int(_lib.lib.mi_varlen_workspace_size(words, H))
        return SimpleNamespace(
            cu=torch.tensor(bounds, dtype=torch.int32).to(device),
            sched=torch.frombuffer(bytearray(words), dtype=torch.int32).to(device),
            header=tuple(int(words[i]) for i in range(4)),
            ws_bytes=ws_bytes,
            ws=torch.zeros(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None,
        )


_SCHEDULES = _Schedules()

#: what the kernels' error word codes mean (csrc/varlen_prefill.hip, kErr*)
_ERROR_CODES = {
    1: "a tall-kernel owner piece gave up waiting for its producer pieces",
    2: "a head_dim 256 duo wave gave up waiting for its partner wave",
}
_ERROR_WORDS: dict = {}


def _device_key(device) -> torch.device:
    dev = torch.device(device) if device is not None else torch.device("cuda")
    return torch.device(dev.type, dev.index if dev.index is not None else torch.cuda.current_device())


def _error_word(device) -> torch.Tensor:
    """The device's prefill error word (one int32, zero when no launch has given up),
    allocated once per device and kept for the life of the process, so a launch recorded in
    a HIP graph keeps a valid address."""
    key = _device_key(device)
    word = _ERROR_WORDS.get(key)
    if word is None:
        word = _ERROR_WORDS[key] = torch.zeros(1, dtype=torch.int32, device=key)
    return word


def check_prefill_errors(device=None) -> None:
    """Raise ``RuntimeError`` if a prefill launch on ``device`` (default: the current HIP
    device) gave up one of its bounded waits since the last check; the output of that launch
    is not to be trusted. One host read; the word is cleared when it raises."""
    key = _device_key(device)
    word = _ERROR_WORDS.get(key)
    if word is None:
        return
    code = int(word.item())
    if code:
        word.zero_()
        raise RuntimeError(f"prefill_varlen on {key}: {_ERROR_CODES.get(code, f'error code {code}')}; "
                           "the output of that launch is not valid")


class HipVarlen:
    """The HIP MFMA varlen kernel: the stand-in for the reference's ``FlashVarlen``
    (``model/attention/varlen.py:293-357``)."""

    name = "hip-mfma-varlen"

    #: ``HipVarlen(kernel=...)`` names; ``None`` lets the library choose per batch
    KERNELS = {None: -1, "staged": 0, "ring": 1, "duo": 3, "tall": 4}

    def __init__(self, kernel: str | None = None, *, strict: bool = False) -> None:
        """``strict=True`` checks the device error word after every call made outside HIP
        graph capture (one host read per call, :func:`check_prefill_errors`); by default calls
        never synchronise and the caller checks when it chooses."""
        _lib.require_library("the hip-mfma-varlen prefill backend")
        if kernel not in self.KERNELS:
            raise ValueError(f"unknown prefill kernel {kernel!r}; choose one of "
                             f"{sorted(k for k in self.KERNELS if k)}")
        self._kernel = self.KERNELS[kernel]
        self._strict = bool(strict)

    def prefill_varlen(self, q, k, v, *, cu_seqlens: Sequence[int] | torch.Tensor, max_seqlen: int,
                       softmax_scale: float | None = None, causal: bool = True):
        bounds = validate_packed(q, k, v, cu_seqlens, max_seqlen)
        scale = _scale(softmax_scale, q.shape[-1])
        if not (q.is_cuda and k.is_cuda and v.is_cuda):
            raise RuntimeError(f"HipVarlen is the CUDA (HIP) kernel path, but q/k/v are on {q.device}; "
                               "backend_for() gives host tensors the SDPA arm")
        if q.dtype not in (torch.float16, torch.bfloat16):
            raise RuntimeError(f"the MFMA varlen kernel computes fp16/bf16 only, got {q.dtype}; "
                               "cast the packed batch, or check fp32 against the SDPA arm on the host")
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        total, H, D = q.shape
        H_kv = int(k.shape[1])
        plan = _SCHEDULES.get(bounds, H, H_kv, D, causal, q.device, self._kernel)
        out = torch.empty_like(q)
        rc = _lib.lib.mi_varlen_prefill(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), plan.cu.data_ptr(), len(bounds) - 1, total,
            int(max_seqlen), plan.sched.data_ptr(), *plan.header, H, H_kv, D, scale, int(bool(causal)),
            _lib.dtype_code(q.dtype), None if plan.ws is None else plan.ws.data_ptr(), plan.ws_bytes,
            _error_word(q.device).data_ptr(), _lib.current_stream(q.device),
        )
        _lib.check(rc, "prefill_varlen")
        if self._strict and not torch.cuda.is_current_stream_capturing():
            check_prefill_errors(q.device)
        return out


#: the name under which the reference's module exposes its CUDA arm
FlashVarlen = HipVarlen


def backend_for(device):
    """The packed-prefill arm for a device type (reference ``model/attention/varlen.py:360-381``):
    ``cuda`` (HIP) -> :class:`HipVarlen`, ``cpu``/``mps`` -> :class:`SdpaVarlen`. Selection is
    by device type only; a missing HIP library makes ``HipVarlen()`` raise rather than
    choosing the other arm."""
    kind = (device if isinstance(device, torch.device) else torch.device(device)).type
    arms = {"cuda": HipVarlen, "cpu": SdpaVarlen, "mps": SdpaVarlen}
    if kind not in arms:
        raise ValueError(f"no packed-prefill backend for device {device!s} (type {kind!r}); the arms are "
                         "cuda (HIP MFMA kernel) and cpu/mps (per-segment SDPA)")
    return arms[kind]()
