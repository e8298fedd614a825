"""Paged KV pool and the block-table decode container on the HIP kernels.

Drop-in for the reference's ``model/paged.py`` (``PagedPool`` ``:82-306``, ``PagedKV``
``:309-586``): same constructor arguments, attributes, step protocol and error behaviour,
with the KV write going through ``mi_kv_slot_write`` instead of two ``index_copy_`` calls
and the decode through :mod:`miattn.decode`.

Pool layout in HBM: one contiguous ``(n_blocks, block_size, H_kv, D)`` K tensor and one V
tensor per layer, allocated once and never replaced. A slot id is a row of the flat
``(n_blocks * block_size, H_kv, D)`` view: ``slot(t) = block_table[t // bs] * bs + t % bs``.

Slot-range errors: the reference's ``index_copy_`` raises on an out-of-range slot on the
CPU and device-asserts on a GPU. The HIP write never touches memory outside the pool: it
skips such a token and records it in a per-pool device error word, which
:meth:`PagedPool.check_writes` reads (one host sync) and turns into ``IndexError``. With
``strict_writes=True`` every write checks immediately; the default keeps the hot path free
of host synchronisation, as the reference does (reference ``:204-205``).
"""

from __future__ import annotations

import os

import torch

from . import _lib
from .decode import TRITON_AVAILABLE, paged_decode_plan
from .rows import Parts

__all__ = ["PagedPool", "PagedKV", "PagedWriteSink"]


def _check_positive(name: str, value: int) -> int:
    if not isinstance(value, int) or isinstance(value, bool) or value < 1:
        raise ValueError(f"{name} must be a positive int, got {value!r}")
    return value


def _same_device(a: torch.device, b: torch.device) -> bool:
    """``cuda`` (current device) and ``cuda:0`` name the same device (reference ``:69-79``)."""
    return a.type == b.type and (a.index is None or b.index is None or a.index == b.index)


class PagedPool:
    """Physical KV blocks: ``(n_blocks, block_size, n_kv_head, head_dim)`` K and V per layer."""

    def __init__(
        self,
        n_layer: int,
        n_blocks: int,
        block_size: int,
        n_kv_head: int,
        head_dim: int,
        *,
        dtype: torch.dtype = torch.float32,
        device: str | torch.device = "cpu",
        n_head: int | None = None,
        strict_writes: bool | None = None,
    ) -> None:
        self.n_layer = _check_positive("n_layer", n_layer)
        self.n_blocks = _check_positive("n_blocks", n_blocks)
        self.block_size = _check_positive("block_size", block_size)
        self.n_kv_head = _check_positive("n_kv_head", n_kv_head)
        self.head_dim = _check_positive("head_dim", head_dim)
        n_head = self.n_kv_head if n_head is None else int(n_head)
        if n_head % self.n_kv_head != 0:
            raise ValueError(f"n_head ({n_head}) must be a multiple of n_kv_head ({self.n_kv_head})")
        self.n_head = n_head
        self.n_group = n_head // self.n_kv_head
        self.dtype = dtype
        self.device = torch.device(device)
        if strict_writes is None:
            strict_writes = os.environ.get("MIATTN_STRICT_WRITES", "0") == "1"
        self.strict_writes = bool(strict_writes)
        shape = (self.n_blocks, self.block_size, self.n_kv_head, self.head_dim)
        self.keys = [torch.zeros(shape, dtype=dtype, device=self.device) for _ in range(self.n_layer)]
        self.values = [torch.zeros(shape, dtype=dtype, device=self.device) for _ in range(self.n_layer)]
        self.n_slots = self.n_blocks * self.block_size
        # First bad token of a write (1 + index), 0 when every slot was in range.
        self._write_error = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._prefill_key: tuple | None = None
        self._prefill_slots: torch.Tensor | None = None

    # ------------------------------------------------------------------ io
    def _check_layer(self, layer: int) -> int:
        if not 0 <= int(layer) < self.n_layer:
            raise IndexError(f"layer {layer} outside the pool's {self.n_layer} layers")
        return int(layer)

    def _check_block_ids(self, block_ids, needed: int) -> None:
        for block_id in block_ids:
            if not isinstance(block_id, int) or isinstance(block_id, bool):
                raise ValueError(f"block ids must be ints, got {block_id!r}")
            if not 0 <= block_id < self.n_blocks:
                raise IndexError(f"block id {block_id} outside the pool's {self.n_blocks} blocks")
        if len(block_ids) < needed:
            raise IndexError(
                f"block table has {len(block_ids)} blocks, needs {needed} to address this write"
            )

    def _slot_ids(self, block_table, start: int, length: int) -> torch.Tensor:
        """Flat slots of logical tokens ``[start, start+length)``, cached per key
        (reference ``:150-168``)."""
        key = (tuple(block_table), start, length)
        if key == self._prefill_key and self._prefill_slots is not None:
            return self._prefill_slots
        table = torch.tensor(list(block_table), dtype=torch.long, device=self.device)
        positions = torch.arange(start, start + length, dtype=torch.long, device=self.device)
        slots = table[positions // self.block_size] * self.block_size + positions % self.block_size
        self._prefill_key = key
        self._prefill_slots = slots
        return slots

    def slot_ids(self, block_table, start: int, length: int) -> torch.Tensor:
        """Public slot-map builder; validates ids and table coverage (reference ``:170-186``)."""
        start = int(start)
        length = int(length)
        if start < 0:
            raise ValueError(f"start must be >= 0, got {start}")
        if length < 0:
            raise ValueError(f"length must be >= 0, got {length}")
        self._check_block_ids(block_table, (start + length + self.block_size - 1) // self.block_size)
        return self._slot_ids(block_table, start, length)

    def write_slots(self, layer: int, slot_ids: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """``pool_flat[slot_ids[i]] = k[i]`` (and v) in one HIP launch (reference ``:188-239``).

        ``k``/``v`` are ``(length, n_kv_head, head_dim)`` views with any strides (the
        engine's sinks hand in permuted views); ``slot_ids`` int32 or int64, distinct.
        """
        layer = self._check_layer(layer)
        if k.dim() != 3 or v.dim() != 3:
            raise ValueError(
                f"write_slots needs (length, n_kv_head, head_dim), got {tuple(k.shape)} / {tuple(v.shape)}"
            )
        if tuple(k.shape) != tuple(v.shape):
            raise ValueError(f"k/v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
        if k.shape[1:] != (self.n_kv_head, self.head_dim):
            raise ValueError(
                f"write_slots needs head shape {(self.n_kv_head, self.head_dim)}, got {tuple(k.shape[1:])}"
            )
        if slot_ids.dim() != 1 or slot_ids.numel() != k.shape[0]:
            raise ValueError(
                f"slot_ids must be 1-D with one entry per token ({k.shape[0]}), got {tuple(slot_ids.shape)}"
            )
        if slot_ids.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"slot_ids must be an integer tensor, got {slot_ids.dtype}")
        if not _same_device(slot_ids.device, self.device):
            raise ValueError(f"slot_ids on {slot_ids.device} but the pool is on {self.device}")
        _lib.require_library("PagedPool.write_slots")
        if self.device.type != "cuda" or not (k.is_cuda and v.is_cuda and slot_ids.is_cuda):
            raise RuntimeError(
                "PagedPool.write_slots is the HIP slot-write kernel and needs a CUDA (HIP) "
                f"pool and tensors; got pool on {self.device}, k on {k.device}, v on {v.device}, "
                f"slot_ids on {slot_ids.device}. There is no CPU fallback."
            )
        if k.dtype != self.dtype:
            k = k.to(self.dtype)
        if v.dtype != self.dtype:
            v = v.to(self.dtype)
        if not slot_ids.is_contiguous():
            slot_ids = slot_ids.contiguous()
        n = int(k.shape[0])
        if n == 0:
            return
        rc = _lib.lib.mi_kv_slot_write(
            k.data_ptr(), v.data_ptr(), slot_ids.data_ptr(), 32 if slot_ids.dtype == torch.int32 else 64,
            self.keys[layer].data_ptr(), self.values[layer].data_ptr(), n, self.n_kv_head,
            self.head_dim, self.n_slots, _lib.int64_array([*k.stride(), *v.stride()]),
            _lib.dtype_code(self.dtype), self._write_error.data_ptr(), _lib.current_stream(k.device),
        )
        _lib.check(rc, "PagedPool.write_slots")
        if self.strict_writes:
            self.check_writes()

    def write_qk_norm_rope(self, layer: int, slot_ids: torch.Tensor, qkv,
                           q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, cos: torch.Tensor,
                           sin: torch.Tensor, pos: torch.Tensor, eps: float, *, k_out: torch.Tensor | None = None,
                           v_out: torch.Tensor | None = None) -> torch.Tensor:
        """One decode step's attention epilogue in one HIP launch: per-head RMSNorm of q and k
        (weights ``q_norm_w``/``k_norm_w``, ``(head_dim,)``), NeoX RoPE at ``pos`` (int64,
        one per row) from the ``(n_pos, head_dim/2)`` ``cos``/``sin`` tables, k and v written
        at ``slot_ids``; returns q ``(B, n_head, head_dim)``, contiguous for the paged decode.

        ``qkv`` is the packed projection output ``(B, (n_head + 2 * n_kv_head) * head_dim)``
        (rows ``[q | k | v]``, unit element stride), or its split-K partial sums
        (:class:`~miattn.rows.Parts`, summed and rounded once). The reference runs this as tensor ops
        (``model/layers.py:193-211``: q_norm/k_norm, ``apply_rotary_emb``) followed by
        ``PagedKV.write`` (``model/paged.py:503-520``); the kernel rounds each step to the
        pool dtype as those ops do. A row whose position is outside the tables or whose slot
        is outside the pool is not written and is reported by :meth:`check_writes`.
        ``k_out``/``v_out`` (contiguous ``(B, n_kv_head, head_dim)``, optional) also receive the
        roped k and the v rows packed -- a packed prefill group's attention inputs.
        """
        layer = self._check_layer(layer)
        H, H_kv, D = self.n_head, self.n_kv_head, self.head_dim
        if isinstance(qkv, Parts):
            if qkv.shape[1] != (H + 2 * H_kv) * D:
                raise ValueError(f"qkv must be (B, {(H + 2 * H_kv) * D}), got partial sums of {qkv.shape}")
            qkv_ptr, qkv_row, qkv_parts, qkv_data = qkv.data.data_ptr(), qkv.shape[1], qkv.n_parts, qkv.data
        else:
            if qkv.dim() != 2 or qkv.shape[1] != (H + 2 * H_kv) * D or qkv.stride(1) != 1:
                raise ValueError(
                    f"qkv must be (B, {(H + 2 * H_kv) * D}) with unit element stride, got {tuple(qkv.shape)} "
                    f"strides {tuple(qkv.stride())}"
                )
            qkv_ptr, qkv_row, qkv_parts, qkv_data = qkv.data_ptr(), qkv.stride(0), 0, qkv
        B = int(qkv.shape[0])
        for name, t, shape in (("q_norm_w", q_norm_w, (D,)), ("k_norm_w", k_norm_w, (D,))):
            if tuple(t.shape) != shape or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous ({D},) tensor, got {tuple(t.shape)}")
        if cos.dim() != 2 or cos.shape[1] != D // 2 or tuple(sin.shape) != tuple(cos.shape):
            raise ValueError(f"cos/sin must be (n_pos, {D // 2}), got {tuple(cos.shape)} / {tuple(sin.shape)}")
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
        tensors = (qkv_data, q_norm_w, k_norm_w, cos, sin, pos, slot_ids)
        if self.device.type != "cuda" or not all(t.is_cuda for t in tensors):
            raise RuntimeError("PagedPool.write_qk_norm_rope is a HIP kernel and needs CUDA (HIP) tensors")
        for name, t in (("k_out", k_out), ("v_out", v_out)):
            if t is not None and (tuple(t.shape) != (B, H_kv, D) or t.dtype != self.dtype or not t.is_contiguous()
                                  or not t.is_cuda):
                raise ValueError(f"{name} must be a contiguous ({B}, {H_kv}, {D}) {self.dtype} HIP tensor")
        slot_ids = slot_ids.contiguous()
        pos = pos.contiguous()
        q = torch.empty((B, H, D), dtype=self.dtype, device=self.device)
        rc = _lib.lib.mi_qk_norm_rope_write(
            qkv_ptr, qkv_row, qkv_parts, q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(),
            sin.data_ptr(), cos.shape[0], pos.data_ptr(), slot_ids.data_ptr(),
            32 if slot_ids.dtype == torch.int32 else 64, q.data_ptr(), self.keys[layer].data_ptr(),
            self.values[layer].data_ptr(), None if k_out is None else k_out.data_ptr(),
            None if v_out is None else v_out.data_ptr(), B, H, H_kv, D, self.n_slots, float(eps),
            _lib.dtype_code(self.dtype), self._write_error.data_ptr(), _lib.current_stream(qkv.device),
        )
        _lib.check(rc, "PagedPool.write_qk_norm_rope")
        if self.strict_writes:
            self.check_writes()
        return q

    def check_writes(self) -> None:
        """Raise ``IndexError`` if a write since the last check met an out-of-range slot.

        One host synchronisation. The offending token was not written; every in-range
        token of the same call was.
        """
        bad = int(self._write_error.item())
        if bad:
            self._write_error.zero_()
            raise IndexError(
                f"slot id of token {bad - 1} is outside the pool's {self.n_slots} slots "
                f"({self.n_blocks} blocks x {self.block_size}); that token was not written"
            )

    def write_prefill_slots(self, layer: int, slot_ids: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """Named prefill entry point over :meth:`write_slots` (reference ``:241-250``)."""
        self.write_slots(layer, slot_ids, k, v)

    def write_prefill(self, layer: int, block_table, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write ``L`` logical tokens ``[start, start+L)`` through ``block_table``
        (reference ``:252-295``)."""
        layer = self._check_layer(layer)
        if k.dim() != 3 or v.dim() != 3:
            raise ValueError(
                f"write_prefill needs (length, n_kv_head, head_dim), got {tuple(k.shape)} / {tuple(v.shape)}"
            )
        if tuple(k.shape) != tuple(v.shape):
            raise ValueError(f"k/v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
        if k.shape[1:] != (self.n_kv_head, self.head_dim):
            raise ValueError(
                f"write_prefill needs head shape {(self.n_kv_head, self.head_dim)}, got {tuple(k.shape[1:])}"
            )
        start = int(start)
        if start < 0:
            raise ValueError(f"start must be >= 0, got {start}")
        length = k.shape[0]
        if length == 0:
            return
        self._check_block_ids(block_table, (start + length + self.block_size - 1) // self.block_size)
        self.write_prefill_slots(layer, self._slot_ids(block_table, start, length), k, v)

    # ------------------------------------------------------------------ accounting
    def bytes(self) -> int:
        return 2 * self.n_layer * self.n_blocks * self.block_size * self.n_kv_head * self.head_dim * self.dtype.itemsize

    def mb(self) -> float:
        return self.bytes() / 2**20


class PagedKV:
    """Decode-time container over a :class:`PagedPool` (reference ``:309-586``).

    Step protocol, once per decode step (reference ``:37-45``)::

        paged.build_mask(next_token=True)   # seqlen := pos + 1 (int32), in place
        for layer in layers:
            paged.write(layer, k, v)        # HIP slot write of this step's token
            y = paged.attend(layer, q)      # HIP block-table decode
        paged.advance()                     # pos += active, slot map refreshed
    """

    decode_container = True
    block_table_decode = True

    def __init__(self, pool: PagedPool, block_tables, lengths, *, rope_len: int, seats=None,
                 n_head: int | None = None, check_bounds: bool = True) -> None:
        if not isinstance(pool, PagedPool):
            raise TypeError(f"PagedKV needs a PagedPool, got {type(pool).__name__}")
        if pool.device.type != "cuda":
            raise ValueError(
                "paged decode is the HIP block-table kernel and needs a CUDA (HIP) pool; "
                f"the pool is on {pool.device}. Use the seat path on CPU; the dense numeric "
                "oracle lives in oracle/."
            )
        if not TRITON_AVAILABLE:
            raise RuntimeError(
                "paged decode requires libmiattn.so (the HIP replacement of the Triton kernel); "
                f"it could not be loaded: {_lib.LOAD_ERROR}. There is no eager fallback."
            )
        n_rows = len(block_tables)
        if n_rows < 1:
            raise ValueError("PagedKV needs at least one row")
        if len(lengths) != n_rows:
            raise ValueError(f"PagedKV needs one length per block table, got {len(lengths)} for {n_rows}")
        rope_len = int(rope_len)
        if rope_len < 1:
            raise ValueError(f"rope_len (the run's position bound) must be >= 1, got {rope_len}")
        self.pool = pool
        self.n_layer = pool.n_layer
        self.n_kv_head = pool.n_kv_head
        self.head_dim = pool.head_dim
        self.n_head = pool.n_kv_head if n_head is None else int(n_head)
        if self.n_head % self.n_kv_head != 0:
            raise ValueError(f"n_head ({self.n_head}) must be a multiple of n_kv_head ({self.n_kv_head})")
        self.n_group = self.n_head // self.n_kv_head
        self.dtype = pool.dtype
        self.device = pool.device
        self.check_bounds = bool(check_bounds)
        self.block_tables = [list(bt) for bt in block_tables]
        self.seats = list(range(n_rows)) if seats is None else list(seats)
        if len(self.seats) != n_rows:
            raise ValueError(f"PagedKV needs one seat per row, got {len(self.seats)} for {n_rows}")
        self.row_of_seat = {seat: row for row, seat in enumerate(self.seats)}
        self.batch = n_rows
        self.max_len = rope_len
        lengths = [int(n) for n in lengths]
        for row, (block_table, length) in enumerate(zip(self.block_tables, lengths)):
            if length < 0:
                raise ValueError(f"row {row}: length must be >= 0, got {length}")
            if length > len(block_table) * pool.block_size:
                raise IndexError(
                    f"row {row}: length {length} exceeds its block table's capacity "
                    f"({len(block_table)} blocks x {pool.block_size})"
                )
            if length > rope_len:
                raise IndexError(f"row {row}: length {length} exceeds the run's position bound {rope_len}")
        self.pos = torch.tensor(lengths, dtype=torch.long, device=self.device)
        self.valid = torch.tensor(lengths, dtype=torch.long, device=self.device)
        self.active = torch.ones(n_rows, dtype=torch.bool, device=self.device)
        self._host_pos = list(lengths)
        self._host_valid = list(lengths)
        self._host_active = [True] * n_rows
        # One zero-padded int32 table for the batch, read by the decode kernel and by the
        # slot-map builder; fixed for the container's life (reference :416-436).
        max_blocks = max((len(table) for table in self.block_tables), default=1)
        host_table = torch.zeros((n_rows, max(max_blocks, 1)), dtype=torch.int32)
        for row, block_table in enumerate(self.block_tables):
            if not block_table:
                continue
            pool._check_block_ids(block_table, (max(lengths[row], 1) + pool.block_size - 1) // pool.block_size)
            host_table[row, : len(block_table)] = torch.tensor(block_table, dtype=torch.int32)
        self._block_table_tensor = host_table.to(self.device)
        self._block_table_i64 = self._block_table_tensor.to(torch.int64)
        self._seqlen = torch.zeros(n_rows, dtype=torch.int32, device=self.device)
        self._slot_ids: torch.Tensor | None = None
        self._slot_error: tuple[int, int, int, int] | None = None
        self._refresh_slots()
        self._decode_plan = None
        self._step_written = False
        self._seqlen_ready = False

    # ---------------------------------------------------------------- step hooks
    def build_mask(self, *, next_token: bool = False) -> None:
        """Refresh the int32 seqlen in place: ``pos + next_token`` (reference ``:454-472``)."""
        counts = [length + int(next_token) for length in self._host_valid]
        longest = max(counts)
        if self.check_bounds and longest > self.max_len:
            raise IndexError(f"PagedKV overflow: needs {longest} positions, run position bound is {self.max_len}")
        self._seqlen.copy_((self.pos + int(next_token)).to(torch.int32))
        self._step_written = False
        self._seqlen_ready = True
        return None

    def _refresh_slots(self) -> None:
        """Per-row write slot ``table[pos // bs] * bs + pos % bs`` (reference ``:474-501``)."""
        bs = self.pool.block_size
        self._slot_error = None
        for row, position in enumerate(self._host_pos):
            block_index = position // bs
            if block_index >= len(self.block_tables[row]):
                self._slot_error = (row, position, block_index, len(self.block_tables[row]))
                break
        if self._slot_error is not None:
            self._slot_ids = None
            return
        block = torch.div(self.pos, bs, rounding_mode="floor")
        block_id = self._block_table_i64.gather(1, block.view(-1, 1)).squeeze(1)
        self._slot_ids = block_id * bs + (self.pos % bs)

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Scatter this step's token of every row at its own position (reference ``:503-520``)."""
        expected = (self.batch, self.n_kv_head, 1, self.head_dim)
        if tuple(k.shape) != expected or tuple(v.shape) != expected:
            raise ValueError(f"write needs {expected}, got {tuple(k.shape)} / {tuple(v.shape)}")
        if self.check_bounds and max(self._host_pos) >= self.max_len:
            raise IndexError(f"PagedKV overflow: write position {max(self._host_pos)} >= max_len {self.max_len}")
        if self._slot_ids is None:
            row, position, block_index, have = self._slot_error or (-1, -1, -1, -1)
            raise IndexError(
                f"row {row}: position {position} needs block {block_index}, but its block table has {have} blocks"
            )
        self.pool.write_slots(layer, self._slot_ids, k[:, :, 0, :], v[:, :, 0, :])
        self._step_written = True

    def write_rope(self, layer: int, qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                   cos: torch.Tensor, sin: torch.Tensor, eps: float) -> torch.Tensor:
        """This step's q/k RMSNorm + RoPE (at each row's position) and K/V write in one HIP
        launch (:meth:`PagedPool.write_qk_norm_rope`, in place of the reference's tensor ops
        and :meth:`write`); ``qkv`` is the packed projection ``(B, (H + 2 H_kv) D)``. Returns
        q ``(B, n_head, 1, head_dim)`` for :meth:`attend`."""
        if self.check_bounds and max(self._host_pos) >= self.max_len:
            raise IndexError(f"PagedKV overflow: write position {max(self._host_pos)} >= max_len {self.max_len}")
        if self._slot_ids is None:
            row, position, block_index, have = self._slot_error or (-1, -1, -1, -1)
            raise IndexError(
                f"row {row}: position {position} needs block {block_index}, but its block table has {have} blocks"
            )
        q = self.pool.write_qk_norm_rope(layer, self._slot_ids, qkv, q_norm_w, k_norm_w, cos, sin, self.pos, eps)
        self._step_written = True
        return q.unsqueeze(2)

    def attend(self, layer: int, q: torch.Tensor, *, dropout_p: float = 0.0) -> torch.Tensor:
        """Block-table decode of one layer; ``q`` ``(B, H, 1, D)`` -> same shape
        (reference ``:522-557``)."""
        if not self._seqlen_ready:
            raise RuntimeError("PagedKV.attend() before build_mask(): seqlen is stale")
        if not self._step_written:
            raise RuntimeError("PagedKV.attend() before write(): this step has no token yet")
        if dropout_p:
            raise ValueError("paged decode is inference-only; dropout_p must be 0")
        expected = (self.batch, self.n_head, 1, self.head_dim)
        if tuple(q.shape) != expected:
            raise ValueError(f"attend needs q {expected}, got {tuple(q.shape)}")
        q3 = q[:, :, 0, :].contiguous()
        if self._decode_plan is None:
            self._decode_plan = paged_decode_plan(
                q3, self.pool.keys, self.pool.values, self._block_table_tensor, self._seqlen,
                scale=1.0 / (self.head_dim ** 0.5),
            )
        return self._decode_plan.run(layer, q3).unsqueeze(2)

    def advance(self) -> None:
        """Move every active row one token (reference ``:559-574``)."""
        self.pos.add_(self.active)
        self.valid.copy_(torch.maximum(self.valid, self.pos))
        for row in range(self.batch):
            if not self._host_active[row]:
                continue
            self._host_pos[row] += 1
            self._host_valid[row] = max(self._host_valid[row], self._host_pos[row])
        self._step_written = False
        self._seqlen_ready = False
        if self.check_bounds and max(self._host_pos) > self.max_len:
            raise IndexError(f"PagedKV overflow: max_len={self.max_len}; a request decoded past its budget")
        self._refresh_slots()

    # ---------------------------------------------------------------- helpers
    def past_len(self) -> int:
        return max(self._host_valid) if self._host_valid else 0

    def bytes(self) -> int:
        return self.pool.bytes()

    def mb(self) -> float:
        return self.bytes() / 2**20


class PagedWriteSink:
    """One request's prefill write-through into its blocks (reference serve/engine.py:147-193).

    ``set_kv(layer, (k, v))`` takes ``(1, H_kv, L, D)`` and writes it through the request's
    precomputed slot map; each layer may be written once (one full prefill, no chunking).
    ``slots`` is kept public so a packed group can concatenate its members' maps into one
    launch (``PackedPrefill.write``).
    """

    def __init__(self, pool: PagedPool, block_table, length: int, *, slots=None) -> None:
        self.pool = pool
        self.block_table = list(block_table)
        self.length = int(length)
        self.slots = slots if slots is not None else pool.slot_ids(self.block_table, 0, self.length)
        self._written = [False] * pool.n_layer

    def past_len(self, layer: int | None = None) -> int:
        return 0

    def get_kv(self, layer: int) -> tuple[None, None]:
        return (None, None)

    def set_kv(self, layer: int, kv) -> None:
        if self._written[layer]:
            raise RuntimeError(
                f"layer {layer} was already written: the paged write-through sink holds "
                "exactly one full prefill (past_len == 0)"
            )
        k, v = kv
        expected = (1, self.pool.n_kv_head, self.length, self.pool.head_dim)
        if tuple(k.shape) != expected or tuple(v.shape) != expected:
            raise ValueError(f"set_kv needs {expected}, got {tuple(k.shape)} / {tuple(v.shape)}")
        self.pool.write_prefill_slots(layer, self.slots, k[0].permute(1, 0, 2), v[0].permute(1, 0, 2))
        self._written[layer] = True
