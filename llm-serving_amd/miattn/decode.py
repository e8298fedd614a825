"""Block-table paged decode on the HIP kernel: the drop-in for ``model/triton_decode.py``.

Entry points keep the reference's names, signatures, ownership and error behaviour
(reference ``model/triton_decode.py:250-538``):

* ``paged_decode(q, k_cache, v_cache, block_table, seqlen, *, scale=None) -> Tensor``
  validates the full contract on every call, allocates a fresh ``out`` and never mutates
  an input (reference ``:250-328``);
* ``paged_decode_plan(...) -> PagedDecodePlan`` validates every layer's pools once;
  ``PagedDecodePlan.run(layer, q)`` re-checks only the query layout (reference
  ``:331-538``). The plan holds the pools, block table and seqlen by reference, so the
  container's in-place seqlen updates are seen;
* ``TRITON_AVAILABLE`` -- the availability flag callers import (reference
  ``model/paged.py:58``, ``serve/engine.py:857-861``). It is True when the HIP library
  loaded; the name is kept so callers switch over unchanged.

Contract (unchanged from the reference): ``q`` ``(B, H, D)``; ``k_cache``/``v_cache``
``(n_blocks, block_size, H_kv, D)`` sharing q's dtype (fp32, fp16 or bf16);
``block_table`` ``(B, max_blocks)`` int32 on q's device; ``seqlen`` ``(B,)`` int32 or int64
with values in ``[0, max_blocks * block_size]``; ``scale=None`` means ``1/sqrt(D)``.

What differs underneath: the kernel is ``mi_paged_decode`` in ``libmiattn.so`` (one
workgroup per (row, split, KV-head group) sweeping whole pages for every KV head and
serving all GQA query heads; rows longer than one split are merged by a small
log-sum-exp launch). Split-K needs a workspace;
``paged_decode`` takes one from torch's caching allocator per call and a plan owns one for
all its layers, so the runs of one plan must stay ordered on one stream (the decode layer
loop is). The kernels also need the K/V
pools' ``head_dim`` to be contiguous and 16-byte aligned, which every pool
``PagedPool`` allocates is; any other layout raises ``ValueError``.
"""

from __future__ import annotations

import math

import torch

from . import _lib

__all__ = ["TRITON_AVAILABLE", "HIP_AVAILABLE", "paged_decode", "paged_decode_plan", "PagedDecodePlan"]

HIP_AVAILABLE: bool = _lib.HIP_AVAILABLE
#: Name kept from the reference so callers that gate on it switch over unchanged.
TRITON_AVAILABLE: bool = HIP_AVAILABLE

#: Last seqlen range validation: ``(seqlen, version, capacity)``; holding the tensor pins
#: its storage so an identity match cannot alias a freed tensor (reference :92, :207-231).
_SEQ_CHECK: tuple[torch.Tensor, int, int] | None = None


def _require_backend() -> None:
    """Fail loudly: there is no eager or CPU implementation behind this entry point."""
    if not TRITON_AVAILABLE:
        raise RuntimeError(
            "paged_decode requires the HIP kernel library libmiattn.so (the replacement of "
            "the Triton decode kernel), but it is unavailable: "
            f"{_lib.LOAD_ERROR or 'disabled'}. There is no eager fallback; the dense "
            "numeric oracle lives in oracle/."
        )
    if not torch.cuda.is_available():
        raise RuntimeError(
            "paged_decode requires CUDA (a HIP device), but torch.cuda is unavailable; the "
            "paged decode arm has no CPU fallback. The dense numeric oracle lives in oracle/."
        )


def _require_cuda_tensors(tensors) -> None:
    for name, tensor in tensors:
        if not tensor.is_cuda:
            raise RuntimeError(
                f"paged_decode requires CUDA tensors, got {name} on device {tensor.device}; "
                "there is no silent fallback to a dense implementation."
            )


def _validate(q, k_cache, v_cache, block_table, seqlen) -> None:
    """The reference's layout contract (reference :120-231): structural errors are
    ``ValueError``; the seqlen range check is cached per tensor version."""
    if q.dim() != 3:
        raise ValueError(f"q must be (B, H, D), got shape {tuple(q.shape)}")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError(
            "k_cache/v_cache must be (n_blocks, block_size, H_kv, D), got "
            f"{tuple(k_cache.shape)} / {tuple(v_cache.shape)}"
        )
    if tuple(k_cache.shape) != tuple(v_cache.shape):
        raise ValueError(
            f"k_cache/v_cache shapes differ: {tuple(k_cache.shape)} vs {tuple(v_cache.shape)}"
        )
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"q dtype must be fp16, bf16 or fp32, got {q.dtype}")
    if not (k_cache.dtype == v_cache.dtype == q.dtype):
        raise ValueError(
            "q/k_cache/v_cache must share one dtype, got "
            f"{q.dtype}, {k_cache.dtype}, {v_cache.dtype}"
        )
    B, H, D = q.shape
    _, block_size, H_kv, cache_d = k_cache.shape
    if D < 1:
        raise ValueError(f"head_dim must be positive, got {D}")
    if D != cache_d:
        raise ValueError(f"q head_dim {D} != cache head_dim {cache_d}")
    if H_kv < 1 or H % H_kv != 0:
        raise ValueError(f"n_head ({H}) must be a multiple of n_kv_head ({H_kv})")
    if block_size < 1:
        raise ValueError(f"block_size must be positive, got {block_size}")
    if block_size & (block_size - 1):
        raise ValueError(
            f"block_size must be a power of two (16 and 32 are the supported sizes), got {block_size}"
        )
    if D & (D - 1):
        raise ValueError(f"head_dim must be a power of two for the kernel, got {D}")
    if block_table.dim() != 2:
        raise ValueError(
            f"block_table must be (B, max_blocks), got shape {tuple(block_table.shape)}"
        )
    B_bt, max_blocks = block_table.shape
    if B_bt != B:
        raise ValueError(f"block_table batch {B_bt} does not match q batch {B}")
    if block_table.dtype != torch.int32:
        raise ValueError(
            "paged_decode requires an int32 block_table (the kernel's indexing contract); "
            f"got {block_table.dtype}. Cast at the allocator boundary, not per step."
        )
    if seqlen.dim() != 1:
        raise ValueError(f"seqlen must be (B,), got shape {tuple(seqlen.shape)}")
    if seqlen.shape[0] != B:
        raise ValueError(f"seqlen has {seqlen.shape[0]} entries for a batch of {B}")
    if seqlen.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"seqlen must be int32 or int64, got {seqlen.dtype}")
    for name, tensor in (
        ("q", q), ("k_cache", k_cache), ("v_cache", v_cache),
        ("block_table", block_table), ("seqlen", seqlen),
    ):
        if tensor.device != q.device:
            raise ValueError(
                f"{name} is on {tensor.device} but q is on {q.device}; all paged_decode "
                "tensors must share one device"
            )
    if B == 0:
        return
    capacity = max_blocks * block_size
    global _SEQ_CHECK
    version = -1 if seqlen.is_inference() else int(seqlen._version)
    cached = _SEQ_CHECK
    if cached is not None and cached[0] is seqlen and cached[1] == version and cached[2] == capacity:
        return
    low = int(seqlen.min())
    high = int(seqlen.max())
    if low < 0:
        raise ValueError(f"seqlen values must be >= 0, got {low}")
    if high > capacity:
        raise ValueError(
            f"seqlen {high} exceeds the block table capacity {capacity} "
            f"({max_blocks} blocks x {block_size} tokens)"
        )
    _SEQ_CHECK = (seqlen, version, capacity)


def _workspace(q, H: int, H_kv: int, D: int, block_size: int, max_blocks: int) -> torch.Tensor | None:
    """Split-K partials buffer, sized exactly for this shape and dtype (None if unneeded)."""
    n = int(_lib.lib.mi_paged_decode_workspace_size(q.shape[0], H, H_kv, D, block_size, max_blocks,
                                                     _lib.dtype_code(q.dtype)))
    if n == 0:
        return None
    return torch.empty(n, dtype=torch.uint8, device=q.device)


def _strides(q, k_cache, v_cache, out, block_table) -> list[int]:
    return [*q.stride(), *k_cache.stride(), *v_cache.stride(), *out.stride(), block_table.stride(0)]


def paged_decode(q, k_cache, v_cache, block_table, seqlen, *, scale: float | None = None):
    """Decode one query token per row against a paged KV pool (reference :250-328)."""
    _require_backend()
    _require_cuda_tensors(
        (("q", q), ("k_cache", k_cache), ("v_cache", v_cache),
         ("block_table", block_table), ("seqlen", seqlen))
    )
    _validate(q, k_cache, v_cache, block_table, seqlen)
    B, H, D = q.shape
    _, block_size, H_kv, _ = k_cache.shape
    if B == 0:
        return torch.empty_like(q)
    q = q.contiguous()
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    seqlen = seqlen.contiguous()
    seqlen32 = seqlen if seqlen.dtype == torch.int32 else seqlen.to(torch.int32)
    out = torch.empty_like(q)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    max_blocks = block_table.shape[1]
    ws = _workspace(q, H, H_kv, D, block_size, max_blocks)
    rc = _lib.lib.mi_paged_decode(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
        seqlen32.data_ptr(), out.data_ptr(), B, H, H_kv, D, block_size, max_blocks,
        _lib.int64_array(_strides(q, k_cache, v_cache, out, block_table)), float(scale),
        _lib.dtype_code(q.dtype), ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _lib.current_stream(q.device),
    )
    _lib.check(rc, "paged_decode")
    return out


class PagedDecodePlan:
    """Per-container launch metadata for repeated decode calls (reference :331-520).

    Validates every ``(k_cache, v_cache)`` pair once (the full ``paged_decode`` contract
    including the seqlen range check) and prebuilds the C-ABI argument block; ``run``
    re-checks only the query, the one input that changes per layer. Pools, block table
    and seqlen are held by reference: in-place seqlen/table updates are seen, replacing a
    pool tensor requires a new plan. The plan owns the split-K workspace shared by its
    layers, so its runs must be ordered on one stream.
    """

    __slots__ = (
        "n_layer", "q_shape", "q_dtype", "q_device", "q_strides", "_k", "_v",
        "_block_table", "_seqlen", "_scale", "_dims", "_strides", "_ws", "_ws_bytes", "_dtype",
    )

    def __init__(self, q, k_caches, v_caches, block_table, seqlen, *, scale=None) -> None:
        _require_backend()
        _require_cuda_tensors((("q", q), ("block_table", block_table), ("seqlen", seqlen)))
        if q.dim() != 3:
            raise ValueError(f"q must be (B, H, D), got shape {tuple(q.shape)}")
        if not q.is_contiguous():
            raise ValueError(
                "paged_decode_plan needs a contiguous (B, H, D) query, got strides "
                f"{q.stride()}; call .contiguous() once, not per layer"
            )
        b, h, d = q.shape
        if b == 0:
            raise ValueError("paged_decode_plan needs at least one row")
        if seqlen.dtype != torch.int32:
            raise ValueError(
                "paged_decode_plan requires an int32 seqlen so in-place updates are "
                f"visible; got {seqlen.dtype}. Cast once at the container boundary."
            )
        if seqlen.stride(0) != 1:
            raise ValueError(
                f"paged_decode_plan requires a contiguous 1-D seqlen; got strides {seqlen.stride()}"
            )
        if block_table.stride(1) != 1:
            raise ValueError(
                "paged_decode_plan requires a column-contiguous block table; got strides "
                f"{block_table.stride()}"
            )
        k_caches = list(k_caches)
        v_caches = list(v_caches)
        if len(k_caches) != len(v_caches) or not k_caches:
            raise ValueError(
                "paged_decode_plan needs one k_cache/v_cache per layer, got "
                f"{len(k_caches)} / {len(v_caches)}"
            )
        for layer, (k_cache, v_cache) in enumerate(zip(k_caches, v_caches)):
            _require_cuda_tensors(((f"k_cache[{layer}]", k_cache), (f"v_cache[{layer}]", v_cache)))
            _validate(q, k_cache, v_cache, block_table, seqlen)
            if tuple(k_cache.shape) != tuple(k_caches[0].shape) or tuple(v_cache.shape) != tuple(
                v_caches[0].shape
            ):
                raise ValueError("paged_decode_plan needs one pool shape for every layer")
            if k_cache.stride() != k_caches[0].stride():
                raise ValueError("paged_decode_plan needs one pool layout for every layer")
            if v_cache.stride() != v_caches[0].stride():
                raise ValueError("paged_decode_plan needs one v-pool layout for every layer")
        self.n_layer = len(k_caches)
        self._k = k_caches
        self._v = v_caches
        self._block_table = block_table
        self._seqlen = seqlen
        self.q_shape = (int(b), int(h), int(d))
        self.q_dtype = q.dtype
        self.q_device = q.device
        self.q_strides = (int(q.stride(0)), int(q.stride(1)), int(q.stride(2)))
        self._scale = float(1.0 / math.sqrt(d) if scale is None else scale)
        _, block_size, h_kv, _ = k_caches[0].shape
        max_blocks = int(block_table.shape[1])
        self._dims = (int(b), int(h), int(h_kv), int(d), int(block_size), max_blocks)
        # q and out share the validated contiguous (B, H, D) strides; every layer's pool
        # shares one stride tuple, so the 15-entry stride block is fixed for the plan.
        self._strides = _lib.int64_array(
            [*self.q_strides, *k_caches[0].stride(), *v_caches[0].stride(), *self.q_strides,
             block_table.stride(0)]
        )
        self._ws = _workspace(q, int(h), int(h_kv), int(d), int(block_size), max_blocks)
        self._ws_bytes = 0 if self._ws is None else int(self._ws.numel())
        self._dtype = _lib.dtype_code(q.dtype)

    def run(self, layer: int, q):
        """Launch the kernel for one layer; ``q`` must match the validated layout."""
        if not 0 <= int(layer) < self.n_layer:
            raise IndexError(f"layer {layer} outside the plan's {self.n_layer} layers")
        if (
            tuple(q.shape) != self.q_shape
            or q.dtype != self.q_dtype
            or q.device != self.q_device
            or q.stride() != self.q_strides
        ):
            raise ValueError(
                "paged_decode_plan.run got a query that does not match the validated "
                f"layout {(self.q_shape, self.q_dtype, self.q_strides)}; got "
                f"{(tuple(q.shape), q.dtype, q.stride())}. Rebuild the plan for a new layout."
            )
        out = torch.empty_like(q)
        b, h, h_kv, d, bs, mb = self._dims
        rc = _lib.lib.mi_paged_decode(
            q.data_ptr(), self._k[layer].data_ptr(), self._v[layer].data_ptr(),
            self._block_table.data_ptr(), self._seqlen.data_ptr(), out.data_ptr(),
            b, h, h_kv, d, bs, mb, self._strides, self._scale, self._dtype,
            None if self._ws is None else self._ws.data_ptr(), self._ws_bytes,
            _lib.current_stream(self.q_device),
        )
        _lib.check(rc, "paged_decode_plan.run")
        return out


def paged_decode_plan(q, k_caches, v_caches, block_table, seqlen, *, scale=None) -> PagedDecodePlan:
    """Validate one container's decode tensors once and cache their launch metadata
    (reference :523-538)."""
    return PagedDecodePlan(q, k_caches, v_caches, block_table, seqlen, scale=scale)
