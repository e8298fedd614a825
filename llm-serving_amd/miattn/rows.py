"""Decode-step projections: ``nn.Linear`` at a few rows as one HIP launch (``mi_rows_gemm``).

In the reference's decode step every projection (q/k/v, o, gate/up, down; reference
``model/layers.py:176-222``, ``:325-335``) and the tied lm_head (``model/minillm.py``) is an
``nn.Linear`` over one row per running sequence. At 32 rows such a product is a stream of the
weight matrix, and a library GEMM tuned for large tiles leaves most of the chip idle (at the
Qwen3-0.6B shapes hipBLASLt measured 8-11 us per projection, 0.5-1.1 TB/s). The HIP kernel
here keeps the whole weight matrix in flight at once and, when the output is too narrow to
fill the chip, splits K: the launch then leaves fp32 partial sums (:class:`Parts`) that the
next op of the step sums and rounds once (``add_rms_norm``, ``silu_mul``,
``PagedPool.write_qk_norm_rope`` take them), so the split costs no extra launch.
"""

from __future__ import annotations

import torch

from . import _lib

__all__ = ["MAX_ROWS", "Parts", "argmax_rows", "glu_weight", "rows_linear", "rows_swiglu", "rows_supported",
           "rows_tile_best", "split_for"]

MAX_ROWS = 32
_K_UNIT = 256  # k per workgroup step: 4 waves x 64


class Parts:
    """fp32 split-K partial sums of a projection ``x @ w.T``: ``data`` is ``(S, M, N)`` and the
    projection's value is the sum over S, in split order, rounded once to ``dtype`` -- what
    ``nn.Linear``'s own output holds up to the order of the fp32 sums."""

    __slots__ = ("data", "dtype")

    def __init__(self, data: torch.Tensor, dtype: torch.dtype) -> None:
        if data.dim() != 3 or data.dtype != torch.float32 or not data.is_contiguous():
            raise ValueError(f"Parts needs contiguous fp32 (S, M, N) sums, got {data.dtype} {tuple(data.shape)}")
        self.data = data
        self.dtype = dtype

    @property
    def shape(self) -> tuple[int, int]:
        return int(self.data.shape[1]), int(self.data.shape[2])

    @property
    def n_parts(self) -> int:
        return int(self.data.shape[0])

    @property
    def device(self) -> torch.device:
        return self.data.device

    def value(self) -> torch.Tensor:
        """The projection output ``(M, N)`` in ``dtype`` (sums in split order, as the consumers do)."""
        acc = self.data[0].clone()
        for s in range(1, self.n_parts):
            acc += self.data[s]
        return acc.to(self.dtype)


def split_for(M: int, N: int, K: int) -> int:
    """The K split ``mi_rows_gemm`` is tuned for at this shape (1 = no partials)."""
    _lib.require_library("rows_linear")
    return int(_lib.lib.mi_rows_gemm_split(M, N, K))


def rows_supported(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether :func:`rows_linear` takes this product: 1-32 rows of bf16/fp16 on a HIP device,
    K a multiple of 256, unit element stride and 16-byte aligned rows."""
    if x.dim() != 2 or w.dim() != 2 or x.dtype != w.dtype or x.dtype not in (torch.bfloat16, torch.float16):
        return False
    M, K = x.shape
    N, K2 = w.shape
    if not (1 <= M <= MAX_ROWS) or K != K2 or K % _K_UNIT or N < 1:
        return False
    if not (x.is_cuda and w.is_cuda) or x.stride(1) != 1 or w.stride(1) != 1:
        return False
    return x.stride(0) % 8 == 0 and w.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0


def rows_linear(x: torch.Tensor, w: torch.Tensor, *, n_split: int | None = None) -> torch.Tensor | Parts:
    """``F.linear(x, w)`` (no bias) for 1-32 rows in one HIP launch. Returns the ``(M, N)``
    output in ``x.dtype`` when the launch does not split K, else :class:`Parts` for a consumer
    that takes partial sums (``n_split=1`` forces a plain output; K must then be <= 1024)."""
    _lib.require_library("rows_linear")
    if not rows_supported(x, w):
        raise ValueError(
            f"rows_linear needs x (M <= {MAX_ROWS}, K) and w (N, K) bf16/fp16 HIP tensors with K a multiple of "
            f"{_K_UNIT}, unit element stride and 16-byte aligned rows; got x {tuple(x.shape)} {x.dtype}, "
            f"w {tuple(w.shape)} {w.dtype}"
        )
    M, K = x.shape
    N = int(w.shape[0])
    S = split_for(M, N, K) if n_split is None else int(n_split)
    stream = _lib.current_stream(x.device)
    code = _lib.dtype_code(x.dtype)
    if S == 1:
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
        rc = _lib.lib.mi_rows_gemm(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(), N, None,
                                   M, N, K, 1, code, stream)
        _lib.check(rc, "rows_linear")
        return out
    part = torch.empty((S, M, N), dtype=torch.float32, device=x.device)
    rc = _lib.lib.mi_rows_gemm(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), None, 0, part.data_ptr(),
                               M, N, K, S, code, stream)
    _lib.check(rc, "rows_linear")
    return Parts(part, x.dtype)


def glu_weight(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """The ``(2 * inter, K)`` weight :func:`rows_swiglu` takes: gate and up rows interleaved by
    16 (rows 32t..32t+15 = gate rows 16t..16t+15, rows 32t+16..32t+31 = up rows 16t..16t+15),
    so each 32-column tile of the product holds matching gate and up columns."""
    if w_gate.shape != w_up.shape or w_gate.dim() != 2 or w_gate.shape[0] % 16:
        raise ValueError(f"gate/up weights must be equal (inter, K) with inter % 16 == 0, got "
                         f"{tuple(w_gate.shape)} / {tuple(w_up.shape)}")
    inter, K = w_gate.shape
    return torch.stack([w_gate.view(inter // 16, 16, K), w_up.view(inter // 16, 16, K)], 1).reshape(2 * inter, K)


def rows_swiglu(x: torch.Tensor, w_glu: torch.Tensor) -> torch.Tensor:
    """``F.silu(x @ w_gate.T) * (x @ w_up.T)`` for 1-32 rows in one HIP launch
    (``mi_rows_gemm_glu``), ``w_glu`` from :func:`glu_weight`; rounded as the reference's
    ``F.silu(gate(x)) * up(x)`` is (each projection, the SiLU and the product to ``x.dtype``)."""
    _lib.require_library("rows_swiglu")
    if not rows_supported(x, w_glu) or x.shape[1] > 4 * _K_UNIT or w_glu.shape[0] % 32:
        raise ValueError(
            f"rows_swiglu needs x (M <= {MAX_ROWS}, K <= {4 * _K_UNIT}, K % {_K_UNIT} == 0) and w_glu "
            f"(2 * inter, K) with inter % 16 == 0; got x {tuple(x.shape)} {x.dtype}, w {tuple(w_glu.shape)}"
        )
    M, K = x.shape
    inter = int(w_glu.shape[0]) // 2
    out = torch.empty((M, inter), dtype=x.dtype, device=x.device)
    rc = _lib.lib.mi_rows_gemm_glu(x.data_ptr(), x.stride(0), w_glu.data_ptr(), w_glu.stride(0), out.data_ptr(),
                                   inter, M, inter, K, _lib.dtype_code(x.dtype), _lib.current_stream(x.device))
    _lib.check(rc, "rows_swiglu")
    return out


def rows_tile_best(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """The unsplit product ``x @ w.T`` (into ``out`` when given, else not stored) reduced, per
    row and per 32-column tile, to the tile's best column under ``torch.argmax``'s rule on
    the rounded outputs (``mi_rows_gemm_argmax``). Returns ``(M, n_tiles, 2)`` int32: word 0
    the value's fp32 bits, word 1 the column -- the input of ``greedy_advance_tiles``."""
    _lib.require_library("rows_tile_best")
    if not rows_supported(x, w) or x.shape[1] > 4 * _K_UNIT:
        raise ValueError(f"rows_tile_best needs an unsplit rows product (K <= {4 * _K_UNIT}), got x "
                         f"{tuple(x.shape)} w {tuple(w.shape)}")
    M, K = x.shape
    N = int(w.shape[0])
    if out is not None and (tuple(out.shape) != (M, N) or out.dtype != x.dtype or out.stride(1) != 1):
        raise ValueError(f"out must be ({M}, {N}) {x.dtype} with unit element stride")
    tiles = torch.empty((M, (N + 31) // 32, 2), dtype=torch.int32, device=x.device)
    rc = _lib.lib.mi_rows_gemm_argmax(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                      None if out is None else out.data_ptr(), 0 if out is None else out.stride(0),
                                      tiles.data_ptr(), M, N, K, _lib.dtype_code(x.dtype),
                                      _lib.current_stream(x.device))
    _lib.check(rc, "rows_tile_best")
    return tiles


def argmax_rows(x: torch.Tensor) -> torch.Tensor:
    """``x.argmax(-1)`` of a 2-D HIP tensor (unit element stride) in one HIP launch
    (``mi_argmax_rows``): int64 ``(rows,)``, the first index of each row's largest value, NaN
    above every number -- torch's rule."""
    _lib.require_library("argmax_rows")
    if x.dim() != 2 or x.stride(1) != 1 or not x.is_cuda or x.shape[1] < 1:
        raise ValueError(f"argmax_rows needs a 2-D HIP tensor with unit element stride, got {tuple(x.shape)}")
    out = torch.empty(x.shape[0], dtype=torch.int64, device=x.device)
    rc = _lib.lib.mi_argmax_rows(x.data_ptr(), x.stride(0), x.shape[0], x.shape[1], out.data_ptr(),
                                 _lib.dtype_code(x.dtype), _lib.current_stream(x.device))
    _lib.check(rc, "argmax_rows")
    return out

