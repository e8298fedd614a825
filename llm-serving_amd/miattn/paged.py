"""Paged KV pool, the block-table decode container and the paged prefill sink.

Drop-ins for the reference's ``model/paged.py`` (``PagedPool`` ``:82-306``, ``PagedKV``
``:309-586``) and ``serve/engine.py``'s ``PagedWriteSink`` (``:147-193``): same
constructor arguments, public attributes, step protocol and exception split.

Pool layout: per layer one ``(n_blocks, block_size, H_kv, D)`` K tensor and one V tensor,
allocated once. A *slot* is a row of the flat ``(n_blocks * block_size, H_kv, D)`` view;
logical token ``t`` of a request with block table ``T`` lives at slot
``T[t // block_size] * block_size + t % block_size``.

Where the bytes move: a pool on a HIP device is written by ``mi_kv_slot_write`` (one
launch for K and V, any source strides); a pool on the host is written with
``index_copy_`` on host tensors, which is what the reference does for host pools (its
CPU tests build them, ``tests/unit/test_paged_kv.py``). A device pool never takes the
host route: without ``libmiattn.so`` it raises. Decode (``PagedKV``) is HIP-only, as the
reference's is CUDA-only.

Out-of-range slots: on the host ``index_copy_`` raises. The HIP write never touches
memory outside the pool; it skips the token and records it in a per-pool device word
that :meth:`PagedPool.check_writes` turns into ``IndexError`` (one host read). With
``strict_writes=True`` every write checks at once; the default keeps the write free of
host synchronisation.
"""

from __future__ import annotations

import os
from types import SimpleNamespace

import numpy as np
import torch

from . import _lib
from ._contract import Rule, enforce, positive_int, same_device
from .decode import TRITON_AVAILABLE, paged_decode_plan
from .rows import Parts

__all__ = ["PagedPool", "PagedKV", "PagedWriteSink"]


def _kv_rules(what: str):
    """Shape rules for a ``(length, H_kv, D)`` k/v pair written into a pool ``a.pool``."""
    return (
        Rule(lambda a: a.k.dim() != 3 or a.v.dim() != 3, ValueError,
             lambda a: f"{what} needs (length, n_kv_head, head_dim) k/v, got {tuple(a.k.shape)} / {tuple(a.v.shape)}"),
        Rule(lambda a: a.k.shape != a.v.shape, ValueError,
             lambda a: f"k/v shapes differ: {tuple(a.k.shape)} vs {tuple(a.v.shape)}"),
        Rule(lambda a: tuple(a.k.shape[1:]) != (a.pool.n_kv_head, a.pool.head_dim), ValueError,
             lambda a: f"{what} needs head shape {(a.pool.n_kv_head, a.pool.head_dim)}, got {tuple(a.k.shape[1:])}"),
    )


_WRITE_SLOTS = _kv_rules("write_slots") + (
    Rule(lambda a: a.slots.dim() != 1 or a.slots.numel() != a.k.shape[0], ValueError,
         lambda a: f"slot_ids must be 1-D with one entry per token ({a.k.shape[0]}), got {tuple(a.slots.shape)}"),
    Rule(lambda a: a.slots.dtype not in (torch.int32, torch.int64), ValueError,
         lambda a: f"slot_ids must be an integer tensor (int32 or int64), got {a.slots.dtype}"),
    Rule(lambda a: not same_device(a.slots.device, a.pool.device), ValueError,
         lambda a: f"slot_ids are on {a.slots.device} but the pool is on {a.pool.device}"),
)

_WRITE_PREFILL = _kv_rules("write_prefill")


class PagedPool:
    """Physical KV blocks: ``(n_blocks, block_size, n_kv_head, head_dim)`` K and V per layer."""

    def __init__(self, n_layer: int, n_blocks: int, block_size: int, n_kv_head: int, head_dim: int, *,
                 dtype: torch.dtype = torch.float32, device: str | torch.device = "cpu",
                 n_head: int | None = None, strict_writes: bool | None = None) -> None:
        self.n_layer = positive_int("n_layer", n_layer)
        self.n_blocks = positive_int("n_blocks", n_blocks)
        self.block_size = positive_int("block_size", block_size)
        self.n_kv_head = positive_int("n_kv_head", n_kv_head)
        self.head_dim = positive_int("head_dim", head_dim)
        self.n_head = self.n_kv_head if n_head is None else int(n_head)
        if self.n_head < 1 or self.n_head % self.n_kv_head:
            raise ValueError(f"n_head ({self.n_head}) must be a multiple of n_kv_head ({self.n_kv_head})")
        self.n_group = self.n_head // self.n_kv_head
        self.dtype = dtype
        self.device = torch.device(device)
        self.n_slots = self.n_blocks * self.block_size
        if strict_writes is None:
            strict_writes = os.environ.get("MIATTN_STRICT_WRITES", "0") == "1"
        self.strict_writes = bool(strict_writes)
        block_shape = (self.n_blocks, self.block_size, self.n_kv_head, self.head_dim)
        self.keys = [torch.zeros(block_shape, dtype=dtype, device=self.device) for _ in range(self.n_layer)]
        self.values = [torch.zeros(block_shape, dtype=dtype, device=self.device) for _ in range(self.n_layer)]
        self._on_device = self.device.type == "cuda"
        # device word: 1 + index of the first token a HIP write skipped, 0 when none
        self._write_error = torch.zeros(1, dtype=torch.int32, device=self.device) if self._on_device else None
        self._slot_memo: tuple[tuple, torch.Tensor] | None = None

    # ------------------------------------------------------------------ tables and slots
    def _layer(self, layer) -> int:
        index = int(layer)
        if index < 0 or index >= self.n_layer:
            raise IndexError(f"layer {layer} is outside the pool's {self.n_layer} layers")
        return index

    def _check_block_ids(self, block_ids, needed: int) -> None:
        """Every id a plain int inside the pool, and enough of them for ``needed`` blocks."""
        bad_type = next((b for b in block_ids if isinstance(b, bool) or not isinstance(b, int)), None)
        if bad_type is not None:
            raise ValueError(f"block ids must be ints, got {bad_type!r}")
        outside = [b for b in block_ids if b < 0 or b >= self.n_blocks]
        if outside:
            raise IndexError(f"block id {outside[0]} is outside the pool's {self.n_blocks} blocks")
        if len(block_ids) < needed:
            raise IndexError(f"block table has {len(block_ids)} blocks, needs {needed} to address this write")

    def _blocks_for(self, start: int, length: int) -> int:
        return -(-(start + length) // self.block_size)

    def _slot_ids(self, block_table, start: int, length: int) -> torch.Tensor:
        """Slots of tokens ``[start, start+length)``, computed on the host and uploaded once;
        the last map is memoised, so a layer loop over one request builds it once."""
        key = (tuple(block_table), int(start), int(length))
        if self._slot_memo is not None and self._slot_memo[0] == key:
            return self._slot_memo[1]
        tokens = np.arange(start, start + length, dtype=np.int64)
        pages = np.asarray(block_table, dtype=np.int64)[tokens // self.block_size]
        slots = torch.from_numpy(pages * self.block_size + tokens % self.block_size).to(self.device)
        self._slot_memo = (key, slots)
        return slots

    def slot_ids(self, block_table, start: int, length: int) -> torch.Tensor:
        """The slot map a caller hands to :meth:`write_prefill_slots` for every layer."""
        start, length = int(start), int(length)
        if start < 0:
            raise ValueError(f"start must be >= 0, got {start}")
        if length < 0:
            raise ValueError(f"length must be >= 0, got {length}")
        self._check_block_ids(block_table, self._blocks_for(start, length))
        return self._slot_ids(block_table, start, length)

    # ------------------------------------------------------------------ writes
    def write_slots(self, layer: int, slot_ids: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """``pool_flat[slot_ids[i]] = k[i]`` and the same for ``v`` (reference
        ``model/paged.py:188-239``). ``k``/``v`` are ``(length, H_kv, D)`` with any strides;
        slots are int32 or int64 and distinct (with duplicates the winner is unspecified)."""
        layer = self._layer(layer)
        enforce(_WRITE_SLOTS, SimpleNamespace(pool=self, k=k, v=v, slots=slot_ids))
        if k.dtype != self.dtype:
            k = k.to(self.dtype)
        if v.dtype != self.dtype:
            v = v.to(self.dtype)
        if self._on_device:
            self._scatter_hip(layer, slot_ids, k, v)
        else:
            self._scatter_host(layer, slot_ids, k, v)

    def _scatter_host(self, layer: int, slot_ids, k, v) -> None:
        if k.is_cuda or v.is_cuda:
            raise ValueError(f"k/v are on {k.device}/{v.device} but the pool is on {self.device}")
        index = slot_ids.long()
        flat = (-1, self.n_kv_head, self.head_dim)
        self.keys[layer].view(flat).index_copy_(0, index, k)
        self.values[layer].view(flat).index_copy_(0, index, v)

    def _scatter_hip(self, layer: int, slot_ids, k, v) -> None:
        _lib.require_library("PagedPool.write_slots on a HIP pool")
        if not (k.is_cuda and v.is_cuda):
            raise RuntimeError(f"a HIP pool takes device k/v; got {k.device}/{v.device}")
        n = int(k.shape[0])
        if n == 0:
            return
        slot_ids = slot_ids.contiguous()
        rc = _lib.lib.mi_kv_slot_write(
            k.data_ptr(), v.data_ptr(), slot_ids.data_ptr(), 8 * slot_ids.element_size(),
            self.keys[layer].data_ptr(), self.values[layer].data_ptr(), n, self.n_kv_head, self.head_dim,
            self.n_slots, _lib.int64_array((*k.stride(), *v.stride())), _lib.dtype_code(self.dtype),
            self._write_error.data_ptr(), _lib.current_stream(k.device),
        )
        _lib.check(rc, "PagedPool.write_slots")
        if self.strict_writes:
            self.check_writes()

    def write_qk_norm_rope(self, layer: int, slot_ids: torch.Tensor, qkv, q_norm_w: torch.Tensor,
                           k_norm_w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor,
                           eps: float, *, k_out: torch.Tensor | None = None,
                           v_out: torch.Tensor | None = None, rotary_dim: int | None = None,
                           zero_centred_norm: bool = False) -> torch.Tensor:
        """One layer's attention epilogue in one HIP launch: per-head RMSNorm of q and k,
        NeoX RoPE at ``pos`` (int64, one per row) over the first ``rotary_dim`` elements of
        each head (all of them by default; 64, 128 or 256) from ``(n_pos, rotary_dim/2)``
        ``cos``/``sin`` tables, and the k/v rows written at ``slot_ids``. Returns q
        ``(B, n_head, head_dim)``. The norm is Qwen3's ``x / rms * w`` rounded op by op, or
        with ``zero_centred_norm`` Qwen3.5's ``x * rsqrt(mean(x^2) + eps) * (1 + w)`` in fp32
        rounded once (reference ``model/qwen35.py:67-89``).

        ``qkv`` is the packed projection ``(B, (n_head + 2 n_kv_head) head_dim)`` (rows
        ``[q | k | v]``, unit element stride) or its split-K partial sums (:class:`Parts`).
        The reference runs these as tensor ops (``model/layers.py:193-211``; partial RoPE
        ``model/qwen35.py:207-210``) followed by ``PagedKV.write``; the kernel rounds each
        step to the pool dtype as those ops do. A row whose position is outside the tables or
        whose slot is outside the pool is not written and is reported by
        :meth:`check_writes`. Slot -1 marks an idle seat (the seat decoder's rows with nothing
        to do this step): that row writes nothing and reports nothing. Both kinds of row come
        back as zeros in q (and in ``k_out``/``v_out``). ``k_out``/``v_out`` (contiguous
        ``(B, n_kv_head, head_dim)``) also receive the roped k and the v rows packed, for a
        packed prefill group.
        """
        layer = self._layer(layer)
        H, H_kv, D = self.n_head, self.n_kv_head, self.head_dim
        rotary = D if rotary_dim is None else int(rotary_dim)
        width = (H + 2 * H_kv) * D
        if isinstance(qkv, Parts):
            if qkv.shape[1] != width:
                raise ValueError(f"qkv must be (B, {width}), got partial sums of {qkv.shape}")
            source, row_stride, n_parts = qkv.data, width, qkv.n_parts
        else:
            if qkv.dim() != 2 or qkv.shape[1] != width or qkv.stride(1) != 1:
                raise ValueError(f"qkv must be (B, {width}) with unit element stride, got {tuple(qkv.shape)} "
                                 f"strides {tuple(qkv.stride())}")
            source, row_stride, n_parts = qkv, qkv.stride(0), 0
        B = int(qkv.shape[0])
        if rotary not in (64, 128, 256) or rotary > D:
            raise ValueError(f"rotary_dim must be 64, 128 or 256 and at most head_dim {D}, got {rotary}")
        for name, t in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w)):
            if tuple(t.shape) != (D,) or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous ({D},) tensor, got {tuple(t.shape)}")
        if cos.dim() != 2 or cos.shape[1] != rotary // 2 or cos.shape != sin.shape:
            raise ValueError(f"cos/sin must be (n_pos, {rotary // 2}), got {tuple(cos.shape)} / {tuple(sin.shape)}")
        if not (cos.is_contiguous() and sin.is_contiguous()):
            raise ValueError("cos/sin tables must be contiguous")
        if pos.dim() != 1 or pos.numel() != B or pos.dtype != torch.int64:
            raise ValueError(f"pos must be an int64 tensor of {B} positions, got {pos.dtype} {tuple(pos.shape)}")
        if slot_ids.dim() != 1 or slot_ids.numel() != B or slot_ids.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"slot_ids must be {B} int32/int64 slots, got {slot_ids.dtype} {tuple(slot_ids.shape)}")
        for name, t in (("qkv", qkv), ("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w), ("cos", cos), ("sin", sin)):
            if t.dtype != self.dtype:
                raise ValueError(f"{name} is {t.dtype}, the pool holds {self.dtype}")
        _lib.require_library("PagedPool.write_qk_norm_rope")
        if not self._on_device or not all(t.is_cuda for t in (source, q_norm_w, k_norm_w, cos, sin, pos, slot_ids)):
            raise RuntimeError("PagedPool.write_qk_norm_rope is a HIP kernel and needs a HIP pool and tensors")
        for name, t in (("k_out", k_out), ("v_out", v_out)):
            if t is not None and (tuple(t.shape) != (B, H_kv, D) or t.dtype != self.dtype
                                  or not t.is_contiguous() or not t.is_cuda):
                raise ValueError(f"{name} must be a contiguous ({B}, {H_kv}, {D}) {self.dtype} HIP tensor")
        slot_ids = slot_ids.contiguous()
        pos = pos.contiguous()
        q = torch.empty((B, H, D), dtype=self.dtype, device=self.device)
        rc = _lib.lib.mi_qk_norm_rope_write(
            source.data_ptr(), row_stride, n_parts, q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(),
            sin.data_ptr(), cos.shape[0], rotary, pos.data_ptr(), slot_ids.data_ptr(), 8 * slot_ids.element_size(),
            q.data_ptr(), self.keys[layer].data_ptr(), self.values[layer].data_ptr(),
            None if k_out is None else k_out.data_ptr(), None if v_out is None else v_out.data_ptr(),
            B, H, H_kv, D, self.n_slots, float(eps), int(bool(zero_centred_norm)), _lib.dtype_code(self.dtype),
            self._write_error.data_ptr(),
            _lib.current_stream(source.device),
        )
        _lib.check(rc, "PagedPool.write_qk_norm_rope")
        if self.strict_writes:
            self.check_writes()
        return q

    @property
    def write_error_word(self) -> torch.Tensor | None:
        """The device word a HIP write reports a refused token through (1 + its index; the
        first report wins until :meth:`check_writes` reads and clears it); None for a host
        pool."""
        return self._write_error

    def check_writes(self) -> None:
        """Raise ``IndexError`` if a HIP write since the last check skipped a token whose
        slot (or position) was out of range; every in-range token was written. One host
        read. Host pools raise at the write itself, so this is a no-op for them."""
        if self._write_error is None:
            return
        first_bad = int(self._write_error.item())
        if first_bad:
            self._write_error.zero_()
            raise IndexError(f"token {first_bad - 1} of a write had a slot outside the pool's {self.n_slots} "
                             f"slots ({self.n_blocks} blocks x {self.block_size}) and was not written")

    def write_prefill_slots(self, layer: int, slot_ids: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """The prefill name of :meth:`write_slots` (reference ``model/paged.py:241-250``)."""
        self.write_slots(layer, slot_ids, k, v)

    def write_prefill(self, layer: int, block_table, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write logical tokens ``[start, start + len(k))`` through ``block_table``
        (reference ``model/paged.py:252-295``)."""
        layer = self._layer(layer)
        enforce(_WRITE_PREFILL, SimpleNamespace(pool=self, k=k, v=v))
        start = int(start)
        if start < 0:
            raise ValueError(f"start must be >= 0, got {start}")
        length = int(k.shape[0])
        if length == 0:
            return
        self._check_block_ids(block_table, self._blocks_for(start, length))
        self.write_prefill_slots(layer, self._slot_ids(block_table, start, length), k, v)

    # ------------------------------------------------------------------ accounting
    def bytes(self) -> int:
        per_layer = self.n_slots * self.n_kv_head * self.head_dim * self.dtype.itemsize
        return 2 * self.n_layer * per_layer

    def mb(self) -> float:
        return self.bytes() / 2**20


class PagedKV:
    """Block-table decode container over a HIP :class:`PagedPool` (reference
    ``model/paged.py:309-586``).

    Rows are the active requests (``seats[row]`` is the caller's seat id). Per row the
    container keeps the position ``pos`` (next token to write), the filled length
    ``valid`` and ``active`` as device tensors, with host copies for bounds checks. The
    batch's block tables become one zero-padded ``(rows, widest)`` int32 tensor read by
    the decode kernel; ``seqlen`` is an int32 vector refreshed in place each step, so the
    container's launch plan (built at the first ``attend``) sees every step.

    Step protocol::

        kv.build_mask(next_token=True)   # seqlen := pos + 1
        for layer in layers:
            kv.write(layer, k, v)        # this step's k/v at pos (HIP slot write)
            y = kv.attend(layer, q)      # HIP block-table decode
        kv.advance()                     # pos += active; next write slots
    """

    decode_container = True
    block_table_decode = True

    def __init__(self, pool: PagedPool, block_tables, lengths, *, rope_len: int, seats=None,
                 n_head: int | None = None, check_bounds: bool = True) -> None:
        if not isinstance(pool, PagedPool):
            raise TypeError(f"PagedKV needs a PagedPool, got {type(pool).__name__}")
        if pool.device.type != "cuda":
            raise ValueError(f"paged decode is the HIP block-table kernel and needs a CUDA (HIP) pool; this pool "
                             f"is on {pool.device}. On the host, decode through the contiguous seat path instead.")
        if not TRITON_AVAILABLE:
            raise RuntimeError("paged decode needs libmiattn.so (the HIP stand-in for the Triton kernel), which "
                               f"did not load: {_lib.LOAD_ERROR}")
        tables = [list(t) for t in block_tables]
        lengths = [int(n) for n in lengths]
        rope_len = int(rope_len)
        if not tables:
            raise ValueError("PagedKV needs at least one row")
        if len(lengths) != len(tables):
            raise ValueError(f"PagedKV needs one length per block table, got {len(lengths)} for {len(tables)}")
        if rope_len < 1:
            raise ValueError(f"rope_len (the run's position bound) must be >= 1, got {rope_len}")
        seats = list(range(len(tables))) if seats is None else list(seats)
        if len(seats) != len(tables):
            raise ValueError(f"PagedKV needs one seat per row, got {len(seats)} for {len(tables)}")
        n_head = pool.n_kv_head if n_head is None else int(n_head)
        if n_head < 1 or n_head % pool.n_kv_head:
            raise ValueError(f"n_head ({n_head}) must be a multiple of n_kv_head ({pool.n_kv_head})")
        for row, (table, n) in enumerate(zip(tables, lengths)):
            if n < 0:
                raise ValueError(f"row {row}: length must be >= 0, got {n}")
            if n > len(table) * pool.block_size:
                raise IndexError(f"row {row}: length {n} exceeds its block table's capacity "
                                 f"({len(table)} blocks x {pool.block_size})")
            if n > rope_len:
                raise IndexError(f"row {row}: length {n} exceeds the run's position bound {rope_len}")
            if table:
                pool._check_block_ids(table, -(-max(n, 1) // pool.block_size))

        self.pool = pool
        self.n_layer, self.n_kv_head, self.head_dim = pool.n_layer, pool.n_kv_head, pool.head_dim
        self.n_head = n_head
        self.n_group = n_head // pool.n_kv_head
        self.dtype, self.device = pool.dtype, pool.device
        self.check_bounds = bool(check_bounds)
        self.block_tables = tables
        self.seats = seats
        self.row_of_seat = {seat: row for row, seat in enumerate(seats)}
        self.batch = len(tables)
        self.max_len = rope_len

        dev = self.device
        self.pos = torch.tensor(lengths, dtype=torch.long, device=dev)
        self.valid = self.pos.clone()
        self.active = torch.ones(self.batch, dtype=torch.bool, device=dev)
        # host copies of pos / valid / active for bounds checks without a device read
        self._hpos = list(lengths)
        self._hvalid = list(lengths)
        self._hactive = [True] * self.batch
        width = max(1, max(len(t) for t in tables))
        padded = np.zeros((self.batch, width), dtype=np.int32)
        for row, table in enumerate(tables):
            padded[row, :len(table)] = table
        self._block_table_tensor = torch.from_numpy(padded).to(dev)
        self._rows = torch.arange(self.batch, device=dev)
        self._seqlen = torch.zeros(self.batch, dtype=torch.int32, device=dev)
        self._slot_ids: torch.Tensor | None = None
        self._no_slot: tuple[int, int, int, int] | None = None
        self._plan = None
        self._written = False
        self._seqlen_fresh = False
        self._refresh_slots()

    # ---------------------------------------------------------------- step hooks
    def build_mask(self, *, next_token: bool = False) -> None:
        """Refresh ``seqlen`` in place to ``pos + next_token`` (the kernel masks by it)."""
        extra = int(bool(next_token))
        if self.check_bounds and max(self._hvalid) + extra > self.max_len:
            raise IndexError(f"PagedKV overflow: needs {max(self._hvalid) + extra} positions, the run's "
                             f"position bound is {self.max_len}")
        torch.add(self.pos, extra, out=self._seqlen)  # int64 + int -> cast into the int32 buffer
        self._written = False
        self._seqlen_fresh = True

    def _refresh_slots(self) -> None:
        """Next write slot of every row, or the first row whose position has no block."""
        bs = self.pool.block_size
        self._no_slot = next(
            ((row, p, p // bs, len(self.block_tables[row])) for row, p in enumerate(self._hpos)
             if p // bs >= len(self.block_tables[row])),
            None,
        )
        if self._no_slot is not None:
            self._slot_ids = None  # a write at this position raises before touching the pool
            return
        # on the device, from pos and the padded table: no host-to-device copy per step
        page = torch.div(self.pos, bs, rounding_mode="floor")
        block = self._block_table_tensor[self._rows, page].long()
        self._slot_ids = block * bs + (self.pos - page * bs)

    def _ready_to_write(self) -> torch.Tensor:
        if self.check_bounds and max(self._hpos) >= self.max_len:
            raise IndexError(f"PagedKV overflow: write position {max(self._hpos)} >= max_len {self.max_len}")
        if self._slot_ids is None:
            row, p, need, have = self._no_slot
            raise IndexError(f"row {row}: position {p} needs block {need}, but its block table has {have} blocks")
        return self._slot_ids

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write this step's ``(B, H_kv, 1, D)`` k/v of every row at its position."""
        want = (self.batch, self.n_kv_head, 1, self.head_dim)
        if tuple(k.shape) != want or tuple(v.shape) != want:
            raise ValueError(f"write needs {want}, got {tuple(k.shape)} / {tuple(v.shape)}")
        slots = self._ready_to_write()
        self.pool.write_slots(layer, slots, k[:, :, 0, :], v[:, :, 0, :])
        self._written = True

    def write_rope(self, layer: int, qkv, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                   cos: torch.Tensor, sin: torch.Tensor, eps: float, *, rotary_dim: int | None = None) -> torch.Tensor:
        """This step's q/k RMSNorm + RoPE at each row's position and the k/v write in one HIP
        launch (:meth:`PagedPool.write_qk_norm_rope`), in place of the tensor ops and
        :meth:`write`. Returns q ``(B, n_head, 1, head_dim)`` for :meth:`attend`."""
        slots = self._ready_to_write()
        q = self.pool.write_qk_norm_rope(layer, slots, qkv, q_norm_w, k_norm_w, cos, sin, self.pos, eps,
                                         rotary_dim=rotary_dim)
        self._written = True
        return q.unsqueeze(2)

    def attend(self, layer: int, q: torch.Tensor, *, dropout_p: float = 0.0) -> torch.Tensor:
        """Decode one layer: ``q`` ``(B, H, 1, D)`` -> ``(B, H, 1, D)``."""
        if not self._seqlen_fresh:
            raise RuntimeError("PagedKV.attend() before build_mask(): seqlen is stale")
        if not self._written:
            raise RuntimeError("PagedKV.attend() before write(): this step has no token yet")
        if dropout_p:
            raise ValueError("paged decode is inference-only; dropout_p must be 0")
        want = (self.batch, self.n_head, 1, self.head_dim)
        if tuple(q.shape) != want:
            raise ValueError(f"attend needs q {want}, got {tuple(q.shape)}")
        q3 = q.squeeze(2).contiguous()
        if self._plan is None:
            self._plan = paged_decode_plan(q3, self.pool.keys, self.pool.values, self._block_table_tensor,
                                           self._seqlen, scale=self.head_dim ** -0.5)
        return self._plan.run(layer, q3).unsqueeze(2)

    def advance(self) -> None:
        """Move every active row one token forward."""
        self.pos += self.active
        torch.maximum(self.valid, self.pos, out=self.valid)
        for row, live in enumerate(self._hactive):
            if live:
                self._hpos[row] += 1
                self._hvalid[row] = max(self._hvalid[row], self._hpos[row])
        self._written = False
        self._seqlen_fresh = False
        if self.check_bounds and max(self._hpos) > self.max_len:
            raise IndexError(f"PagedKV overflow: a row decoded past the run's position bound {self.max_len}")
        self._refresh_slots()

    # ---------------------------------------------------------------- helpers
    def past_len(self) -> int:
        return max(self._hvalid, default=0)

    def bytes(self) -> int:
        return self.pool.bytes()

    def mb(self) -> float:
        return self.bytes() / 2**20


class PagedWriteSink:
    """One request's prefill written straight into its blocks (reference
    ``serve/engine.py:147-193``).

    ``set_kv(layer, (k, v))`` takes ``(1, H_kv, L, D)`` and writes it through the request's
    slot map; each layer accepts exactly one write (a whole prompt, no chunking). ``slots``
    is built once at construction and kept public, so a packed group can write all its
    members with one concatenated map (``PackedPrefill.write``).
    """

    def __init__(self, pool: PagedPool, block_table, length: int, *, slots=None) -> None:
        self.pool = pool
        self.block_table = list(block_table)
        self.length = int(length)
        self.slots = pool.slot_ids(self.block_table, 0, self.length) if slots is None else slots
        self._written = [False] * pool.n_layer

    def past_len(self, layer: int | None = None) -> int:
        return 0

    def get_kv(self, layer: int) -> tuple[None, None]:
        return (None, None)

    def claim(self, layer: int) -> None:
        """Mark ``layer`` written; a second write of one layer is refused."""
        if self._written[layer]:
            raise RuntimeError(f"layer {layer} was already written: this sink holds exactly one whole prompt "
                               "(past_len == 0)")
        self._written[layer] = True

    def set_kv(self, layer: int, kv) -> None:
        k, v = kv
        want = (1, self.pool.n_kv_head, self.length, self.pool.head_dim)
        if tuple(k.shape) != want or tuple(v.shape) != want:
            raise ValueError(f"set_kv needs {want}, got {tuple(k.shape)} / {tuple(v.shape)}")
        self.claim(layer)
        self.pool.write_prefill_slots(layer, self.slots, k[0].transpose(0, 1), v[0].transpose(0, 1))
