"""Block-table paged decode on the HIP kernel: the drop-in for ``model/triton_decode.py``.

Public surface (names, signatures, ownership and exception split as in the reference,
``model/triton_decode.py:250-258, 331-538``):

* ``paged_decode(q, k_cache, v_cache, block_table, seqlen, *, scale=None) -> Tensor`` --
  one query token per row against a paged pool. Checks the whole contract, returns a new
  ``out`` and leaves every input untouched;
* ``paged_decode_plan(q, k_caches, v_caches, block_table, seqlen, *, scale=None)`` ->
  :class:`PagedDecodePlan`, whose ``run(layer, q)`` launches one layer. The plan checks all
  layers once and afterwards only the query of each call; it keeps the pools, the table
  and ``seqlen`` by reference, so in-place ``seqlen`` updates between steps are seen;
* ``TRITON_AVAILABLE`` -- the flag the reference's callers import. It names the decode
  backend being present, which here means ``libmiattn.so`` loaded.

Contract: ``q`` ``(B, H, D)``; pools ``(n_blocks, block_size, H_kv, D)`` in q's dtype
(fp32, fp16 or bf16), ``H % H_kv == 0``, power-of-two ``block_size`` and ``D``;
``block_table`` ``(B, width)`` int32; ``seqlen`` ``(B,)`` int32 or int64 within
``[0, width * block_size]``; all on one HIP device. ``scale=None`` is ``1/sqrt(D)``.

Underneath is ``mi_paged_decode`` (``include/miattn.h``): page-sweeping split-K workgroups
serving every query head of a KV head, plus a log-sum-exp merge launch for rows cut into
several splits. The split partials live in a workspace: ``paged_decode`` takes one from
torch's caching allocator per call; a plan owns one for all its layers, so one plan's runs
must stay ordered on one stream (a layer loop is).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from types import SimpleNamespace

import torch

from . import _lib
from ._contract import Rule, enforce, is_pow2

__all__ = ["TRITON_AVAILABLE", "HIP_AVAILABLE", "paged_decode", "paged_decode_plan", "PagedDecodePlan"]

HIP_AVAILABLE: bool = _lib.HIP_AVAILABLE
#: Availability flag under the name the reference's callers import.
TRITON_AVAILABLE: bool = HIP_AVAILABLE

_ELEMENT_TYPES = (torch.float16, torch.bfloat16, torch.float32)


@dataclass(frozen=True)
class DecodeGeometry:
    """Sizes one decode launch is built from (all read from tensor shapes)."""

    rows: int          # B
    q_heads: int       # H
    kv_heads: int      # H_kv
    head_dim: int      # D
    page: int          # block_size: tokens per physical block
    width: int         # block-table columns

    @property
    def capacity(self) -> int:
        return self.width * self.page

    def dims(self) -> tuple[int, int, int, int, int, int]:
        return (self.rows, self.q_heads, self.kv_heads, self.head_dim, self.page, self.width)


# -- the contract, in the order a caller learns about mistakes ------------------------
_LAYOUT = (
    Rule(lambda a: a.q.dim() != 3, ValueError,
         lambda a: f"q must be (B, H, D), got shape {tuple(a.q.shape)}"),
    Rule(lambda a: a.k.dim() != 4 or a.v.dim() != 4, ValueError,
         lambda a: "k_cache/v_cache must be (n_blocks, block_size, H_kv, D), got "
                   f"{tuple(a.k.shape)} / {tuple(a.v.shape)}"),
    Rule(lambda a: a.k.shape != a.v.shape, ValueError,
         lambda a: f"k_cache/v_cache shapes differ: {tuple(a.k.shape)} vs {tuple(a.v.shape)}"),
    Rule(lambda a: a.q.dtype not in _ELEMENT_TYPES, ValueError,
         lambda a: f"q dtype must be fp16, bf16 or fp32, got {a.q.dtype}"),
    Rule(lambda a: not (a.q.dtype == a.k.dtype == a.v.dtype), ValueError,
         lambda a: f"q/k_cache/v_cache must share one dtype, got {a.q.dtype}, {a.k.dtype}, {a.v.dtype}"),
)

_HEADS = (
    Rule(lambda a: a.q.shape[2] < 1, ValueError,
         lambda a: f"head_dim must be positive, got {a.q.shape[2]}"),
    Rule(lambda a: a.q.shape[2] != a.k.shape[3], ValueError,
         lambda a: f"q head_dim {a.q.shape[2]} != cache head_dim {a.k.shape[3]}"),
    Rule(lambda a: a.k.shape[2] < 1 or a.q.shape[1] % a.k.shape[2] != 0, ValueError,
         lambda a: f"n_head ({a.q.shape[1]}) must be a multiple of n_kv_head ({a.k.shape[2]})"),
    Rule(lambda a: not is_pow2(a.k.shape[1]), ValueError,
         lambda a: "block_size must be a power of two (16 and 32 are the supported sizes), "
                   f"got {a.k.shape[1]}"),
    Rule(lambda a: not is_pow2(a.q.shape[2]), ValueError,
         lambda a: f"head_dim must be a power of two for the kernel, got {a.q.shape[2]}"),
)

_INDEXING = (
    Rule(lambda a: a.table.dim() != 2, ValueError,
         lambda a: f"block_table must be (B, max_blocks), got shape {tuple(a.table.shape)}"),
    Rule(lambda a: a.table.shape[0] != a.q.shape[0], ValueError,
         lambda a: f"block_table batch {a.table.shape[0]} does not match q batch {a.q.shape[0]}"),
    Rule(lambda a: a.table.dtype != torch.int32, ValueError,
         lambda a: "paged_decode requires an int32 block_table (the kernel reads 32-bit block ids); "
                   f"got {a.table.dtype}. Convert once where the tables are built."),
    Rule(lambda a: a.seqlen.dim() != 1, ValueError,
         lambda a: f"seqlen must be (B,), got shape {tuple(a.seqlen.shape)}"),
    Rule(lambda a: a.seqlen.shape[0] != a.q.shape[0], ValueError,
         lambda a: f"seqlen has {a.seqlen.shape[0]} entries for a batch of {a.q.shape[0]}"),
    Rule(lambda a: a.seqlen.dtype not in (torch.int32, torch.int64), ValueError,
         lambda a: f"seqlen must be int32 or int64, got {a.seqlen.dtype}"),
    Rule(lambda a: any(t.device != a.q.device for t in (a.k, a.v, a.table, a.seqlen)), ValueError,
         lambda a: "all paged_decode tensors must share one device; got q on "
                   f"{a.q.device}, k_cache {a.k.device}, v_cache {a.v.device}, "
                   f"block_table {a.table.device}, seqlen {a.seqlen.device}"),
)

# The HIP kernel streams each (token, KV head) row of D elements as 16-byte pieces.
_POOL_LAYOUT = (
    Rule(lambda a: a.k.stride(3) != 1 or a.v.stride(3) != 1, ValueError,
         lambda a: "the HIP decode reads head_dim-contiguous pools; got strides "
                   f"{a.k.stride()} / {a.v.stride()}"),
    Rule(lambda a: (a.k.data_ptr() | a.v.data_ptr()) % 16 != 0, ValueError,
         lambda a: "the HIP decode needs 16-byte aligned pools"),
)


class _SeqlenWatch:
    """Range check of ``seqlen`` values, paid once per tensor version.

    Reading ``seqlen`` costs a host synchronisation, so the last tensor that passed is
    remembered with its version counter and the capacity it was checked against; the
    same tensor at the same version skips the read. Inference-mode tensors carry no
    version counter and are remembered under version -1, as the reference does
    (``model/triton_decode.py:207-231``). Keeping the tensor object alive in the watch is
    what makes the identity comparison safe.
    """

    __slots__ = ("_seen",)

    def __init__(self) -> None:
        self._seen: tuple[torch.Tensor, int, int] | None = None

    def confirm(self, seqlen: torch.Tensor, capacity: int) -> None:
        version = -1 if seqlen.is_inference() else int(seqlen._version)
        seen = self._seen
        if seen is not None and seen[0] is seqlen and seen[1] == version and seen[2] == capacity:
            return
        lo, hi = (int(x) for x in torch.stack(torch.aminmax(seqlen)).tolist())
        if lo < 0:
            raise ValueError(f"seqlen values must be >= 0, got {lo}")
        if hi > capacity:
            raise ValueError(f"seqlen {hi} exceeds the block table capacity {capacity}")
        self._seen = (seqlen, version, capacity)


_SEQLEN_WATCH = _SeqlenWatch()


def _require_backend() -> None:
    """No library or no device is an environment failure, never a reason to compute
    the attention some other way."""
    if not TRITON_AVAILABLE:
        raise RuntimeError(
            "paged_decode needs libmiattn.so, the HIP kernel that stands in for the Triton "
            f"decode kernel, and it is not loaded ({_lib.LOAD_ERROR or 'disabled'}); "
            "there is no eager implementation to use instead"
        )
    if not torch.cuda.is_available():
        raise RuntimeError(
            "paged_decode runs on a CUDA (HIP) device and torch reports none; "
            "the paged arm has no host implementation"
        )


def _require_device_tensors(named) -> None:
    for name, tensor in named:
        if not tensor.is_cuda:
            raise RuntimeError(
                f"paged_decode requires CUDA tensors; {name} is on {tensor.device} and "
                "nothing here computes on the host"
            )


def _check(q, k_cache, v_cache, block_table, seqlen) -> DecodeGeometry:
    """Apply the full contract and return the launch geometry."""
    a = SimpleNamespace(q=q, k=k_cache, v=v_cache, table=block_table, seqlen=seqlen)
    enforce(_LAYOUT, a)
    enforce(_HEADS, a)
    enforce(_INDEXING, a)
    g = DecodeGeometry(int(q.shape[0]), int(q.shape[1]), int(k_cache.shape[2]), int(q.shape[2]),
                       int(k_cache.shape[1]), int(block_table.shape[1]))
    if g.rows:
        _SEQLEN_WATCH.confirm(seqlen, g.capacity)
    return g


def _workspace_bytes(g: DecodeGeometry, dtype: torch.dtype) -> int:
    return int(_lib.lib.mi_paged_decode_workspace_size(*g.dims(), _lib.dtype_code(dtype)))


def _launch(g: DecodeGeometry, q, k_ptr: int, v_ptr: int, table_ptr: int, seqlen_ptr: int, out,
            strides, scale: float, ws_ptr, ws_bytes: int, what: str) -> None:
    rc = _lib.lib.mi_paged_decode(
        q.data_ptr(), k_ptr, v_ptr, table_ptr, seqlen_ptr, out.data_ptr(), *g.dims(), strides,
        scale, _lib.dtype_code(q.dtype), ws_ptr, ws_bytes, _lib.current_stream(q.device),
    )
    _lib.check(rc, what)


def paged_decode(q, k_cache, v_cache, block_table, seqlen, *, scale: float | None = None):
    """Decode one query token per row against a paged KV pool (reference
    ``model/triton_decode.py:250-328``)."""
    _require_backend()
    _require_device_tensors((("q", q), ("k_cache", k_cache), ("v_cache", v_cache),
                             ("block_table", block_table), ("seqlen", seqlen)))
    g = _check(q, k_cache, v_cache, block_table, seqlen)
    if g.rows == 0:
        return torch.empty_like(q)
    enforce(_POOL_LAYOUT, SimpleNamespace(k=k_cache, v=v_cache))
    q = q.contiguous()
    table = block_table if block_table.stride(1) == 1 else block_table.contiguous()
    lens = seqlen.to(torch.int32).contiguous()
    out = torch.empty_like(q)
    strides = _lib.int64_array((*q.stride(), *k_cache.stride(), *v_cache.stride(), *out.stride(),
                                table.stride(0)))
    n_ws = _workspace_bytes(g, q.dtype)
    ws = torch.empty(n_ws, dtype=torch.uint8, device=q.device) if n_ws else None
    _launch(g, q, k_cache.data_ptr(), v_cache.data_ptr(), table.data_ptr(), lens.data_ptr(), out, strides,
            float(1.0 / math.sqrt(g.head_dim) if scale is None else scale),
            None if ws is None else ws.data_ptr(), n_ws, "paged_decode")
    return out


# -- launch plan ------------------------------------------------------------------------
_PLAN_INPUTS = (
    Rule(lambda a: a.q.dim() != 3, ValueError,
         lambda a: f"q must be (B, H, D), got shape {tuple(a.q.shape)}"),
    Rule(lambda a: not a.q.is_contiguous(), ValueError,
         lambda a: f"paged_decode_plan needs a contiguous (B, H, D) query, got strides {a.q.stride()}"),
    Rule(lambda a: a.q.shape[0] == 0, ValueError,
         lambda a: "paged_decode_plan needs at least one row"),
    Rule(lambda a: a.seqlen.dtype != torch.int32, ValueError,
         lambda a: "paged_decode_plan requires an int32 seqlen: the plan reads the caller's tensor "
                   f"in place at every run, so it cannot keep a converted copy (got {a.seqlen.dtype})"),
    Rule(lambda a: a.seqlen.dim() != 1 or a.seqlen.stride(0) != 1, ValueError,
         lambda a: f"paged_decode_plan requires a contiguous 1-D seqlen, got strides {a.seqlen.stride()}"),
    Rule(lambda a: a.table.dim() != 2 or a.table.stride(1) != 1, ValueError,
         lambda a: "paged_decode_plan requires a column-contiguous block table, got strides "
                   f"{a.table.stride()}"),
    Rule(lambda a: len(a.ks) == 0 or len(a.ks) != len(a.vs), ValueError,
         lambda a: f"paged_decode_plan needs one k_cache and one v_cache per layer, got {len(a.ks)} / {len(a.vs)}"),
)


class PagedDecodePlan:
    """Checked-once launch state for the decode calls of one container (reference
    ``model/triton_decode.py:331-520``).

    Construction applies the full :func:`paged_decode` contract to every layer's pools
    and requires them to share one shape and one stride layout; it then freezes the
    launch arguments (geometry, stride block, scale, workspace). ``run`` only compares
    the query against the layout it was built for. Pools, table and ``seqlen`` are held
    by reference.
    """

    __slots__ = ("n_layer", "geometry", "q_signature", "_k_ptrs", "_v_ptrs", "_pools",
                 "_table", "_seqlen", "_strides", "_scale", "_ws", "_ws_bytes")

    def __init__(self, q, k_caches, v_caches, block_table, seqlen, *, scale=None) -> None:
        _require_backend()
        _require_device_tensors((("q", q), ("block_table", block_table), ("seqlen", seqlen)))
        ks, vs = list(k_caches), list(v_caches)
        enforce(_PLAN_INPUTS, SimpleNamespace(q=q, ks=ks, vs=vs, table=block_table, seqlen=seqlen))
        first = (tuple(ks[0].shape), ks[0].stride(), vs[0].stride())
        for layer, (k, v) in enumerate(zip(ks, vs)):
            _require_device_tensors(((f"k_cache[{layer}]", k), (f"v_cache[{layer}]", v)))
            g = _check(q, k, v, block_table, seqlen)
            enforce(_POOL_LAYOUT, SimpleNamespace(k=k, v=v))
            if (tuple(k.shape), k.stride(), v.stride()) != first or tuple(v.shape) != first[0]:
                raise ValueError(f"paged_decode_plan needs one pool shape and layout for every layer "
                                 f"(layer {layer} differs from layer 0)")
        self.n_layer = len(ks)
        self.geometry = g
        self.q_signature = (tuple(q.shape), q.dtype, q.device, q.stride())
        self._pools = (ks, vs)  # keeps the pool tensors alive
        self._k_ptrs = [k.data_ptr() for k in ks]
        self._v_ptrs = [v.data_ptr() for v in vs]
        self._table = block_table
        self._seqlen = seqlen
        # q and out share the checked contiguous (B, H, D) strides
        self._strides = _lib.int64_array((*q.stride(), *first[1], *first[2], *q.stride(), block_table.stride(0)))
        self._scale = float(1.0 / math.sqrt(g.head_dim) if scale is None else scale)
        self._ws_bytes = _workspace_bytes(g, q.dtype)
        self._ws = torch.empty(self._ws_bytes, dtype=torch.uint8, device=q.device) if self._ws_bytes else None

    def run(self, layer: int, q):
        """Launch one layer; ``q`` must have the layout the plan was built with."""
        if not 0 <= int(layer) < self.n_layer:
            raise IndexError(f"layer {layer} is outside the plan's {self.n_layer} layers")
        signature = (tuple(q.shape), q.dtype, q.device, q.stride())
        if signature != self.q_signature:
            raise ValueError(
                "paged_decode_plan.run: the query does not match the validated layout "
                f"(built for shape/dtype/device/strides {self.q_signature}, got {signature}); "
                "build a new plan for a new layout"
            )
        out = torch.empty_like(q)
        layer = int(layer)
        _launch(self.geometry, q, self._k_ptrs[layer], self._v_ptrs[layer], self._table.data_ptr(),
                self._seqlen.data_ptr(), out, self._strides, self._scale,
                None if self._ws is None else self._ws.data_ptr(), self._ws_bytes, "paged_decode_plan.run")
        return out


    def fused_supported(self, dtype: torch.dtype, rotary_dim: int, zero_centred_norm: bool = False) -> bool:
        """Whether :meth:`run_fused` covers this geometry: head_dim 128, whole-head RoPE, the
        Qwen3 q/k norm, fp16/bf16 (``mi_paged_decode_fused``)."""
        return (self.geometry.head_dim == 128 and int(rotary_dim) == 128 and not zero_centred_norm
                and dtype in (torch.float16, torch.bfloat16))

    def run_fused(self, layer: int, qkv, q_norm_w, k_norm_w, cos, sin, pos, slot_ids, eps: float, *,
                  error_word: torch.Tensor | None = None) -> torch.Tensor:
        """One layer's decode attention straight from its packed q/k/v projection: q/k RMSNorm,
        RoPE at ``pos`` and the new token's K/V write into this layer's pools, then the paged
        decode -- ``PagedPool.write_qk_norm_rope`` followed by :meth:`run`, with the same
        result bit for bit, in one launch pair (``mi_paged_decode_fused``). ``qkv`` is the
        ``(B, (H + 2 H_kv) D)`` projection or its split-K partial sums (an object with
        ``data`` ``(S, B, width)`` fp32 and ``n_parts``); ``pos`` int64 ``(B,)`` must be each
        row's last position (``seqlen - 1``); ``slot_ids`` int32/int64 ``(B,)``, -1 for an idle
        row. Rows refused for a position or slot out of range are reported through
        ``error_word`` (1 + row) and attend with q = 0. The new tokens' K/V are written while
        the launch reads the pools, so no row's slot may fall inside another row's first
        ``seqlen`` tokens (a block shared into another row's table below its length); the
        reference's per-row blocks never do. Returns ``(B, H, D)``."""
        if not 0 <= int(layer) < self.n_layer:
            raise IndexError(f"layer {layer} is outside the plan's {self.n_layer} layers")
        g = self.geometry
        dtype = self.q_signature[1]
        width = (g.q_heads + 2 * g.kv_heads) * g.head_dim
        if hasattr(qkv, "n_parts"):
            source, n_parts = qkv.data, int(qkv.n_parts)
            if tuple(source.shape[1:]) != (g.rows, width) or source.dtype != torch.float32:
                raise ValueError(f"qkv partials must be (S, {g.rows}, {width}) fp32, got {tuple(source.shape)}")
            row_stride = width
        else:
            source, n_parts = qkv, 0
            if qkv.dim() != 2 or tuple(qkv.shape) != (g.rows, width) or qkv.stride(1) != 1 or qkv.dtype != dtype:
                raise ValueError(f"qkv must be ({g.rows}, {width}) {dtype} with unit element stride, got "
                                 f"{qkv.dtype} {tuple(qkv.shape)}")
            row_stride = qkv.stride(0)
        rotary = 2 * int(cos.shape[-1])
        if not self.fused_supported(dtype, rotary):
            raise ValueError("run_fused covers head_dim 128 with whole-head RoPE in fp16/bf16; use "
                             "PagedPool.write_qk_norm_rope and run")
        if cos.shape != sin.shape or cos.dim() != 2 or not (cos.is_contiguous() and sin.is_contiguous()):
            raise ValueError(f"cos/sin must be contiguous (n_pos, 64) tables, got {tuple(cos.shape)}")
        if pos.dtype != torch.int64 or pos.numel() != g.rows or slot_ids.numel() != g.rows or \
                slot_ids.dtype not in (torch.int32, torch.int64):
            raise ValueError("pos must be int64 (B,) and slot_ids int32/int64 (B,)")
        out = torch.empty(self.q_signature[0], dtype=dtype, device=self.q_signature[2])
        k, v = self._pools[0][layer], self._pools[1][layer]
        rc = _lib.lib.mi_paged_decode_fused(
            source.data_ptr(), row_stride, n_parts, q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(),
            sin.data_ptr(), int(cos.shape[0]), rotary, pos.data_ptr(), slot_ids.data_ptr(),
            8 * slot_ids.element_size(), k.data_ptr(), v.data_ptr(), self._table.data_ptr(), self._seqlen.data_ptr(),
            out.data_ptr(), *g.dims(), int(k.shape[0]) * int(k.shape[1]), self._strides, self._scale, float(eps), 0,
            _lib.dtype_code(dtype), None if self._ws is None else self._ws.data_ptr(), self._ws_bytes,
            None if error_word is None else error_word.data_ptr(), _lib.current_stream(out.device),
        )
        _lib.check(rc, "paged_decode_plan.run_fused")
        return out


def paged_decode_plan(q, k_caches, v_caches, block_table, seqlen, *, scale=None) -> PagedDecodePlan:
    """Check one container's decode tensors once and freeze their launch arguments
    (reference ``model/triton_decode.py:523-538``)."""
    return PagedDecodePlan(q, k_caches, v_caches, block_table, seqlen, scale=scale)
