"""Random-init Qwen3-0.6B driven through the MI355X attention path (the end-to-end harness).

The model is the reference's ``MiniLLM`` at the Qwen3 shape (reference ``model/minillm.py``,
``model/layers.py``): tied token embedding, 28 blocks of pre-norm attention + SwiGLU MLP,
per-head q/k RMSNorm, NeoX RoPE with theta 1e6, RMSNorm computed in the activation dtype,
bf16 weights drawn N(0, 0.02). Only the attention path is this package's: packed prefill
goes through :class:`~miattn.packed.PackedPrefill` (HIP varlen kernel + one slot-write
launch per layer) and decode through :class:`~miattn.paged.PagedKV` (HIP slot write +
block-table decode), exactly the containers the reference's layers call
(reference ``model/layers.py:217-250``). Projections and the residual-stream norms are
plain torch in prefill. In decode every projection and the lm_head is one HIP rows-GEMM
launch (``rows_linear``, q/k/v and gate/up over stacked weights), the q/k norms, RoPE and the
K/V write are one HIP launch per layer (``PagedPool.write_qk_norm_rope``), each residual add
with the next RMSNorm is one launch (``add_rms_norm``) and the MLP's SiLU * up another
(``silu_mul``); the ops after a split-K projection sum its partials, and every op keeps the
reference ops' rounding.

:class:`GraphDecoder` is the decode step with no host work per step: slot map, seqlen,
RoPE rows, 28 layers, lm_head and the greedy argmax are captured once in a HIP graph and
replayed (the reference parks this, ``serve/graph.py:1-40``; the host-bound step it
measures is ``serve/graph.py:9-10``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _lib
from .decode import paged_decode_plan
from .packed import PackedPrefill
from .paged import PagedKV, PagedPool, PagedWriteSink
from .rows import Parts, argmax_rows, glu_weight, rows_linear, rows_supported, rows_swiglu, rows_tile_best

__all__ = ["Qwen3Config", "random_weights", "Qwen3", "GraphDecoder"]


@dataclass(frozen=True)
class Qwen3Config:
    """Qwen3-0.6B (reference ``model/config.py`` fields, Qwen3 values)."""

    vocab: int = 151936
    hidden: int = 1024
    inter: int = 3072
    n_layer: int = 28
    n_head: int = 16
    n_kv_head: int = 8
    head_dim: int = 128
    eps: float = 1e-6
    rope_theta: float = 1e6
    std: float = 0.02


def random_weights(cfg: Qwen3Config, seed: int, dtype=torch.bfloat16) -> dict:
    """N(0, std) embedding and projections, unit norms (reference ``_init_weights``,
    ``model/minillm.py:57-64``), drawn on the CPU in a fixed order so every host and test
    sees the same values for a seed."""
    gen = torch.Generator().manual_seed(seed)

    def normal(*shape):
        return (torch.randn(*shape, generator=gen) * cfg.std).to(dtype)

    H, Hk, D, C = cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.hidden
    w = {"embed": normal(cfg.vocab, C), "norm": torch.ones(C, dtype=dtype)}
    for i in range(cfg.n_layer):
        p = f"l{i}."
        w[p + "wq"] = normal(H * D, C)
        w[p + "wk"] = normal(Hk * D, C)
        w[p + "wv"] = normal(Hk * D, C)
        w[p + "wo"] = normal(C, H * D)
        w[p + "wg"] = normal(cfg.inter, C)
        w[p + "wu"] = normal(cfg.inter, C)
        w[p + "wd"] = normal(C, cfg.inter)
        for n in ("ln1", "ln2"):
            w[p + n] = torch.ones(C, dtype=dtype)
        for n in ("qn", "kn"):
            w[p + n] = torch.ones(D, dtype=dtype)
    return w


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``x / sqrt(mean(x^2) + eps) * weight`` in x's dtype (reference ``model/layers.py:342-350``)."""
    rms = torch.sqrt(x.pow(2).mean(-1, True) + eps)
    return x / rms * weight


def rope_table(head_dim: int, theta: float, length: int, device, dtype):
    """cos/sin ``(length, head_dim/2)`` in the model dtype (reference ``rope_cos_sin``)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    angles = torch.outer(torch.arange(length, dtype=torch.float32, device=device), inv_freq)
    return angles.cos().to(dtype), angles.sin().to(dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """NeoX halves rotation; ``cos``/``sin`` broadcast against ``x``'s ``(..., H, D)``
    with a head axis inserted (reference ``apply_rotary_emb``)."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    cos, sin = cos.unsqueeze(-2), sin.unsqueeze(-2)
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)


def _proj_arg(t, rows: int, cols: int, dtype: torch.dtype, name: str):
    """(pointer, parts) of a projection output given as a tensor or as split-K :class:`Parts`."""
    if isinstance(t, Parts):
        if t.shape != (rows, cols) or t.dtype != dtype:
            raise ValueError(f"{name} must be ({rows}, {cols}) {dtype}, got partial sums {t.shape} {t.dtype}")
        return t.data.data_ptr(), t.n_parts
    if not t.is_contiguous() or tuple(t.shape) != (rows, cols) or t.dtype != dtype:
        raise ValueError(f"{name} must be contiguous ({rows}, {cols}) {dtype}, got {tuple(t.shape)} {t.dtype}")
    return t.data_ptr(), 0


def add_rms_norm(x: torch.Tensor, delta, weight: torch.Tensor, eps: float):
    """``x + delta`` (in place into ``x``) and its RMSNorm in one HIP launch (``mi_add_rms_norm``),
    rounded op by op as :func:`rms_norm` and the residual add are; returns ``(x, h)``.
    ``x``: contiguous ``(rows, cols)``; ``delta``: the same, or the :class:`Parts` of the
    projection that produces it, or None (normalise ``x`` as is)."""
    rows, cols = x.shape
    _proj_arg(x, rows, cols, x.dtype, "x")
    d_ptr, d_parts = (None, 0) if delta is None else _proj_arg(delta, rows, cols, x.dtype, "delta")
    if tuple(weight.shape) != (cols,) or weight.dtype != x.dtype:
        raise ValueError(f"weight must be ({cols},) {x.dtype}")
    h = torch.empty_like(x)
    rc = _lib.lib.mi_add_rms_norm(x.data_ptr(), d_ptr, d_parts, weight.data_ptr(),
                                  x.data_ptr() if delta is not None else None, h.data_ptr(), rows, cols, float(eps),
                                  _lib.dtype_code(x.dtype), _lib.current_stream(x.device))
    _lib.check(rc, "add_rms_norm")
    return x, h


def silu_mul(gate_up) -> torch.Tensor:
    """``silu(gate) * up`` of a ``(rows, 2 * inter)`` ``[gate | up]`` projection (a tensor or its
    :class:`Parts`) in one HIP launch (``mi_silu_mul``), rounded op by op as ``F.silu(g) * u`` is."""
    rows, two = gate_up.shape
    if two % 2:
        raise ValueError(f"gate_up must be (rows, 2 * inter), got {tuple(gate_up.shape)}")
    ptr, parts = _proj_arg(gate_up, rows, two, gate_up.dtype, "gate_up")
    out = torch.empty((rows, two // 2), dtype=gate_up.dtype, device=gate_up.device)
    rc = _lib.lib.mi_silu_mul(ptr, parts, out.data_ptr(), rows, two // 2, _lib.dtype_code(gate_up.dtype),
                              _lib.current_stream(gate_up.device))
    _lib.check(rc, "silu_mul")
    return out


def decode_step_begin(tokens: torch.Tensor, pos: torch.Tensor, table: torch.Tensor, block_size: int,
                      embed: torch.Tensor, norm_w: torch.Tensor, eps: float, seqlen: torch.Tensor,
                      slots: torch.Tensor, x: torch.Tensor, h: torch.Tensor, error: torch.Tensor) -> None:
    """One HIP launch (``mi_decode_step_begin``) for the start of a decode step, in place:
    ``seqlen = pos + 1`` (int32), ``slots = table[pos // bs] * bs + pos % bs`` (int64),
    ``x = embed[tokens]`` and ``h = rms_norm(x, norm_w)``. A row with an out-of-range token or
    position is left unwritten and reported through ``error`` (int32, row + 1)."""
    B = tokens.numel()
    V, C = embed.shape
    for name, t, dt in (("tokens", tokens, torch.int64), ("pos", pos, torch.int64), ("slots", slots, torch.int64),
                        ("seqlen", seqlen, torch.int32), ("error", error, torch.int32)):
        if t.dtype != dt or not t.is_contiguous() or (t.numel() < 1 if name == "error" else t.numel() != B):
            raise ValueError(f"{name} must be a contiguous {dt} tensor of {'at least 1' if name == 'error' else B} "
                             f"{'word' if name == 'error' else 'rows'}")
    if table.dtype != torch.int32 or table.dim() != 2 or table.shape[0] != B or table.stride(1) != 1:
        raise ValueError("table must be an int32 (B, max_blocks) block table with contiguous rows")
    for name, t in (("x", x), ("h", h)):
        if tuple(t.shape) != (B, C) or t.dtype != embed.dtype or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous ({B}, {C}) {embed.dtype}")
    if tuple(norm_w.shape) != (C,) or norm_w.dtype != embed.dtype or not embed.is_contiguous():
        raise ValueError(f"norm_w must be ({C},) {embed.dtype} and embed contiguous")
    rc = _lib.lib.mi_decode_step_begin(
        tokens.data_ptr(), pos.data_ptr(), table.data_ptr(), table.stride(0), block_size, table.shape[1],
        embed.data_ptr(), V, norm_w.data_ptr(), C, float(eps), seqlen.data_ptr(), slots.data_ptr(), x.data_ptr(),
        h.data_ptr(), B, _lib.dtype_code(embed.dtype), error.data_ptr(), _lib.current_stream(x.device))
    _lib.check(rc, "decode_step_begin")


def _check_step_state(B: int, tokens, pos, history, steps) -> None:
    for name, t in (("tokens", tokens), ("pos", pos), ("steps", steps)):
        if t.dtype != torch.int64 or t.numel() != B or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int64 tensor of {B} rows")
    if history.dtype != torch.int64 or history.dim() != 2 or history.shape[0] != B or history.stride(1) != 1:
        raise ValueError(f"history must be an int64 ({B}, max_steps) tensor with contiguous rows")


def greedy_advance_tiles(tiles: torch.Tensor, tokens: torch.Tensor, pos: torch.Tensor, history: torch.Tensor,
                         steps: torch.Tensor) -> None:
    """:func:`greedy_advance` from ``rows_tile_best``'s per-tile picks ``(B, n_tiles, 2)``
    (``mi_greedy_advance_tiles``): the same pick and updates without the logits."""
    if tiles.dtype != torch.int32 or tiles.dim() != 3 or tiles.shape[2] != 2 or not tiles.is_contiguous():
        raise ValueError("tiles must be the contiguous (B, n_tiles, 2) int32 output of rows_tile_best")
    B, n_tiles, _ = tiles.shape
    _check_step_state(B, tokens, pos, history, steps)
    rc = _lib.lib.mi_greedy_advance_tiles(tiles.data_ptr(), n_tiles, B, tokens.data_ptr(), pos.data_ptr(),
                                          history.data_ptr(), history.stride(0), steps.data_ptr(), history.shape[1],
                                          _lib.current_stream(tiles.device))
    _lib.check(rc, "greedy_advance_tiles")


def greedy_advance(logits: torch.Tensor, tokens: torch.Tensor, pos: torch.Tensor, history: torch.Tensor,
                   steps: torch.Tensor) -> None:
    """One HIP launch (``mi_greedy_advance``) for the end of a greedy decode step, in place:
    ``tokens = logits.argmax(-1)``, ``history[r, steps[r]] = tokens[r]`` while ``steps[r]`` is
    inside ``history``, ``steps += 1``, ``pos += 1`` (all int64)."""
    B, V = logits.shape
    if logits.stride(1) != 1:
        raise ValueError("logits must have unit element stride")
    _check_step_state(B, tokens, pos, history, steps)
    rc = _lib.lib.mi_greedy_advance(logits.data_ptr(), logits.stride(0), B, V, _lib.dtype_code(logits.dtype),
                                    tokens.data_ptr(), pos.data_ptr(), history.data_ptr(), history.stride(0),
                                    steps.data_ptr(), history.shape[1], _lib.current_stream(logits.device))
    _lib.check(rc, "greedy_advance")


class Qwen3:
    """The model on one HIP device, attention through this package's containers."""

    def __init__(self, cfg: Qwen3Config, weights: dict, device, *, max_pos: int = 8192) -> None:
        _lib.require_library("the Qwen3 end-to-end harness")
        self.cfg = cfg
        self.device = torch.device(device)
        self.w = {k: v.to(self.device) for k, v in weights.items()}
        # decode projects q, k and v with one GEMM over the stacked weights (the same dot
        # products as three separate projections); its output rows are [q | k | v]
        for i in range(cfg.n_layer):
            p = f"l{i}."
            self.w[p + "wqkv"] = torch.cat([self.w[p + "wq"], self.w[p + "wk"], self.w[p + "wv"]], 0).contiguous()
            self.w[p + "wgu"] = torch.cat([self.w[p + "wg"], self.w[p + "wu"]], 0).contiguous()
            # the same rows interleaved by 16 for the one-launch gate/up + SiLU * up
            self.w[p + "wglu"] = glu_weight(self.w[p + "wg"], self.w[p + "wu"]).contiguous()
        self.dtype = self.w["embed"].dtype
        self.cos, self.sin = rope_table(cfg.head_dim, cfg.rope_theta, max_pos, self.device, self.dtype)

    # ------------------------------------------------------------------ pieces
    def new_pool(self, n_blocks: int, block_size: int = 16) -> PagedPool:
        c = self.cfg
        return PagedPool(c.n_layer, n_blocks, block_size, c.n_kv_head, c.head_dim, dtype=self.dtype,
                         device=self.device, n_head=c.n_head)

    # ------------------------------------------------------------------ prefill
    def prefill(self, prompts: list[list[int]], pool: PagedPool, tables: list[list[int]]) -> torch.Tensor:
        """Packed prefill of whole prompts (reference ``MiniLLM.forward`` packed branch,
        ``model/minillm.py:76-106``); writes every layer's K/V into ``pool`` through the
        requests' block tables and returns the last-token logits ``(n_prompts, vocab)``.
        Projections are ``F.linear`` (thousands of rows); q/k norm + RoPE + the K/V write, each
        residual add with the next RMSNorm and SiLU * up are one HIP launch each, as in
        decode."""
        c = self.cfg
        lengths = [len(p) for p in prompts]
        cu = [0]
        for n in lengths:
            cu.append(cu[-1] + n)
        positions = torch.cat([torch.arange(n) for n in lengths]).to(self.device)
        sinks = [PagedWriteSink(pool, t, n) for t, n in zip(tables, lengths)]
        packed = PackedPrefill(cu_seqlens=cu, positions=positions, sinks=sinks)
        tokens = torch.tensor([t for p in prompts for t in p], dtype=torch.long, device=self.device)
        x = F.embedding(tokens, self.w["embed"])  # (T, C), the residual stream (updated in place)
        T = x.shape[0]
        _, h = add_rms_norm(x, None, self.w["l0.ln1"], c.eps)
        for i in range(c.n_layer):
            p = f"l{i}."
            # q/k norm + RoPE + the group's K/V write in one launch over one stacked projection
            q, k, v = packed.write_rope(i, F.linear(h, self.w[p + "wqkv"]), self.w[p + "qn"], self.w[p + "kn"],
                                        self.cos, self.sin, c.eps)
            y = packed.attend(q, k, v)
            _, h = add_rms_norm(x, F.linear(y.reshape(T, -1), self.w[p + "wo"]), self.w[p + "ln2"], c.eps)
            m = silu_mul(F.linear(h, self.w[p + "wgu"]))
            nxt = self.w[f"l{i + 1}.ln1"] if i + 1 < c.n_layer else self.w["norm"]
            _, h = add_rms_norm(x, F.linear(m, self.w[p + "wd"]), nxt, c.eps)
        return F.linear(h[packed.last_token_index], self.w["embed"])

    # ------------------------------------------------------------------ decode
    def _decode_stack(self, x: torch.Tensor, attend, h0: torch.Tensor | None = None) -> torch.Tensor:
        """The 28 layers of a decode step on the ``(B, C)`` residual stream ``x`` (updated in
        place): residual adds fused with the next RMSNorm (``add_rms_norm``), one GEMM for
        q/k/v and one for gate/up, SiLU * up in one launch, and ``attend(i, qkv)`` giving
        layer i's attention output ``(B, H * D)`` from its packed projection. Returns the
        final RMSNorm of the stream (the lm_head input); ``h0``, when given, is layer 0's input
        norm of ``x`` already computed. Same arithmetic as the reference's block
        (``model/layers.py:365-367``) op by op."""
        c = self.cfg
        h = h0 if h0 is not None else add_rms_norm(x, None, self.w["l0.ln1"], c.eps)[1]
        for i in range(c.n_layer):
            p = f"l{i}."
            y = attend(i, self._proj(h, self.w[p + "wqkv"]))
            _, h = add_rms_norm(x, self._proj(y, self.w[p + "wo"]), self.w[p + "ln2"], c.eps)
            m = self._mlp_in(h, p)
            nxt = self.w[f"l{i + 1}.ln1"] if i + 1 < c.n_layer else self.w["norm"]
            _, h = add_rms_norm(x, self._proj(m, self.w[p + "wd"]), nxt, c.eps)
        return h

    def _mlp_in(self, h: torch.Tensor, p: str) -> torch.Tensor:
        """``silu(gate(h)) * up(h)``: one HIP launch (``rows_swiglu``) where it applies, else the
        gate/up projection followed by ``silu_mul``."""
        w = self.w[p + "wglu"]
        if rows_supported(h, w) and h.shape[1] <= 1024:
            return rows_swiglu(h, w)
        return silu_mul(self._proj(h, self.w[p + "wgu"]))

    @staticmethod
    def _proj(h: torch.Tensor, w: torch.Tensor):
        """A decode-step projection: the HIP rows GEMM (``rows_linear``; its output may be split-K
        :class:`Parts` for the next op to sum) where it applies (up to 32 rows), else
        ``F.linear``."""
        return rows_linear(h, w) if rows_supported(h, w) else F.linear(h, w)

    def _lm_head(self, h: torch.Tensor) -> torch.Tensor:
        """Logits ``(B, vocab)`` of the final-norm rows (tied embedding), one HIP launch."""
        w = self.w["embed"]
        if rows_supported(h, w) and h.shape[1] <= 1024:
            return rows_linear(h, w, n_split=1)
        return F.linear(h, w)

    def decode(self, paged: PagedKV, tokens: torch.Tensor) -> torch.Tensor:
        """One decode step of every row (reference ``MiniLLM.forward`` decode-container
        branch, ``model/minillm.py:111-136``); returns logits ``(B, vocab)``."""
        c = self.cfg
        paged.build_mask(next_token=True)
        x = F.embedding(tokens.view(-1), self.w["embed"])  # (B, C)
        B = x.shape[0]

        def attend(i: int, qkv) -> torch.Tensor:
            # q/k norm + RoPE + K/V write in one HIP launch (the reference's tensor ops + write)
            p = f"l{i}."
            q = paged.write_rope(i, qkv, self.w[p + "qn"], self.w[p + "kn"], self.cos, self.sin, c.eps)
            return paged.attend(i, q).reshape(B, -1)

        h = self._decode_stack(x, attend)
        paged.advance()
        return self._lm_head(h)


class GraphDecoder:
    """Greedy decode steps of a fixed batch, each replayed from one captured HIP graph.

    Device state per row: the next input token, its position, an int32 seqlen, and the
    row's block table. A step is HIP launches only: one computes the write slot
    ``table[pos // bs] * bs + pos % bs`` (reference ``model/paged.py:499-501``), ``seqlen =
    pos + 1``, the embedding row and layer 0's input norm; then the 28 layers; then the
    lm_head and one launch for the argmax, ``history``, the next tokens and ``pos + 1``.
    ``history`` collects the generated tokens (``step_idx`` counts each row's steps).
    """

    def __init__(self, model: Qwen3, pool: PagedPool, tables: list[list[int]], lengths: list[int],
                 first_tokens: torch.Tensor, max_new: int) -> None:
        c = model.cfg
        dev = model.device
        self.model, self.pool = model, pool
        B = len(tables)
        max_blocks = max(len(t) for t in tables)
        for t, n in zip(tables, lengths):
            if (n + max_new + pool.block_size - 1) // pool.block_size > len(t):
                raise ValueError(f"block table of {len(t)} blocks cannot hold {n} + {max_new} tokens")
        # rows padded with -1 past their own blocks: the step-begin launch refuses a row whose
        # position reaches the padding instead of writing into another row's block
        bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
        for r, t in enumerate(tables):
            bt[r, : len(t)] = torch.tensor(t, dtype=torch.int32)
        self.table = bt.to(dev)
        self.pos = torch.tensor(lengths, dtype=torch.long, device=dev)
        self.seqlen = (self.pos + 1).to(torch.int32)
        self.tokens = first_tokens.to(dev, torch.long).clone()
        self.history = torch.zeros(B, max_new, dtype=torch.long, device=dev)
        self.step_idx = torch.zeros(B, dtype=torch.long, device=dev)  # steps taken, per row
        self.slots = torch.zeros(B, dtype=torch.long, device=dev)
        self.error = torch.zeros(1, dtype=torch.int32, device=dev)
        self.max_new = max_new
        self.B = B
        q0 = torch.zeros(B, c.n_head, c.head_dim, dtype=model.dtype, device=dev)
        self.plan = paged_decode_plan(q0, pool.keys, pool.values, self.table, self.seqlen,
                                      scale=1.0 / math.sqrt(c.head_dim))
        # q/k norm + RoPE + K/V write fused into the decode launch where the shape allows
        self.fused = self.plan.fused_supported(model.dtype, 2 * int(model.cos.shape[-1]))
        self.graph = None

    def _step(self) -> None:
        m, c, bs = self.model, self.model.cfg, self.pool.block_size
        x = torch.empty(self.B, c.hidden, dtype=m.dtype, device=m.device)
        h0 = torch.empty_like(x)
        # seqlen, write slots, embedding lookup and layer 0's input norm: one launch
        decode_step_begin(self.tokens, self.pos, self.table, bs, m.w["embed"], m.w["l0.ln1"], c.eps, self.seqlen,
                          self.slots, x, h0, self.error)
        slots = self.slots

        def attend(i: int, qkv) -> torch.Tensor:
            p = f"l{i}."
            if self.fused:
                return self.plan.run_fused(i, qkv, m.w[p + "qn"], m.w[p + "kn"], m.cos, m.sin, self.pos, slots,
                                           c.eps, error_word=self.pool.write_error_word).view(self.B, -1)
            q = self.pool.write_qk_norm_rope(i, slots, qkv, m.w[p + "qn"], m.w[p + "kn"], m.cos, m.sin,
                                             self.pos, c.eps)
            return self.plan.run(i, q).view(self.B, -1)

        h = m._decode_stack(x, attend, h0)
        w = m.w["embed"]
        if rows_supported(h, w) and h.shape[1] <= 1024:
            # lm_head reduced to per-tile picks in its own launch (the logits are not stored),
            # then the pick, history, next tokens and positions in one more
            greedy_advance_tiles(rows_tile_best(h, w), self.tokens, self.pos, self.history, self.step_idx)
        else:
            greedy_advance(m._lm_head(h), self.tokens, self.pos, self.history, self.step_idx)

    def capture(self, stream=None) -> None:
        """Record one step (run once eagerly first so lazily built state exists) and undo
        that warm-up step's effects on positions, history and the step counter."""
        saved = (self.pos.clone(), self.tokens.clone())
        self._step()
        torch.cuda.synchronize()
        self.pos.copy_(saved[0])
        self.tokens.copy_(saved[1])
        self.step_idx.zero_()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self._step()
        # capture recorded but did not run the step: restore the pre-step state
        self.pos.copy_(saved[0])
        self.tokens.copy_(saved[1])
        self.step_idx.zero_()
        torch.cuda.synchronize()

    def step(self) -> None:
        if self.graph is None:
            self._step()
        else:
            self.graph.replay()

    def check(self) -> None:
        """Raise ``IndexError`` if a step met a token outside the vocabulary or a position
        outside its row's own blocks (that row was made inert: no K/V written, zero
        attention), or if a write of the step was refused by the pool; host reads only."""
        bad = int(self.error.item())
        if bad:
            self.error.zero_()
            try:
                self.pool.check_writes()  # the refused row's epilogue writes were skipped too
            except IndexError:
                pass
            raise IndexError(f"row {bad - 1}: token or position out of range in a decode step; the row was skipped")
        self.pool.check_writes()
