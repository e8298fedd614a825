"""Seeded synthetic inputs for the hot path's five benchmark configurations.

Shapes are the Qwen3-0.6B attention shape: H=16 query heads, H_kv=8 KV heads, D=128,
bf16, block size 16. Every builder is deterministic in its seed. Small tensors are drawn
on the CPU (so a CPU oracle sees the same values); large pools are drawn on the target
device with a seeded device generator, since the 28-layer pools (14-30 GiB) are too large
to draw on the host.

* config 1 -- seat decode: B=8, 511 cached + 1 new token, RoPE theta 1e6 pre-applied.
* config 2 -- paged decode: B=32, seqlen ~ U[128, 2048], 8192 blocks per layer, 28 layers,
  disjoint block tables cut from one seeded permutation.
* config 3 -- packed prefill + slot write: 8 prompts, length lognormal(median 512,
  sigma 0.6) clipped to [64, 2048], a seeded disjoint block mapping.
* config 4 -- long-context split-K decode: B=32 x 8192 tokens, 16384 blocks per layer.
* config 5 -- end-to-end Qwen3-0.6B trace (see ``e2e``): Poisson arrivals 4 req/s,
  prompts lognormal(median 256, sigma 0.6) clipped to [32, 2048], 128 new tokens.

The lognormal sigma is not fixed by the benchmark definition; 0.6 is this build's choice
and is recorded in every result line that uses it.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

__all__ = [
    "QWEN3_ATTN",
    "PROMPT_SIGMA",
    "rope",
    "block_tables_from_perm",
    "slot_map",
    "seat_decode_config1",
    "paged_decode_config",
    "prefill_config3",
    "lognormal_lengths",
]

QWEN3_ATTN = dict(H=16, H_kv=8, D=128, block_size=16, rope_theta=1e6)
PROMPT_SIGMA = 0.6


def rope(x: torch.Tensor, positions: torch.Tensor, theta: float) -> torch.Tensor:
    """NeoX-style rotary embedding (rotate the two halves of D), computed in fp32.

    ``x`` is ``(..., T, D)`` and ``positions`` ``(T,)``; the result has ``x``'s dtype.
    """
    D = x.shape[-1]
    inv_freq = theta ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    angles = positions.to(torch.float64)[:, None] * inv_freq[None, :]
    cos = torch.cat([angles.cos(), angles.cos()], dim=-1).to(torch.float32)
    sin = torch.cat([angles.sin(), angles.sin()], dim=-1).to(torch.float32)
    xf = x.to(torch.float32)
    half = D // 2
    rotated = torch.cat([-xf[..., half:], xf[..., :half]], dim=-1)
    return (xf * cos.to(x.device) + rotated * sin.to(x.device)).to(x.dtype)


def block_tables_from_perm(lengths, n_blocks: int, block_size: int, seed: int) -> list[list[int]]:
    """Disjoint per-sequence tables cut in order from one seeded permutation of the pool."""
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(n_blocks, generator=gen).tolist()
    tables, offset = [], 0
    for length in lengths:
        need = max(1, -(-int(length) // block_size))
        if offset + need > n_blocks:
            raise ValueError(f"pool of {n_blocks} blocks cannot hold the tables ({offset + need} needed)")
        tables.append(perm[offset: offset + need])
        offset += need
    return tables


def slot_map(table, start: int, length: int, block_size: int) -> np.ndarray:
    """``slot(t) = table[t // bs] * bs + t % bs`` for ``t`` in ``[start, start+length)``."""
    t = np.arange(start, start + length, dtype=np.int64)
    return np.asarray(table, dtype=np.int64)[t // block_size] * block_size + t % block_size


def lognormal_lengths(n: int, median: float, sigma: float, lo: int, hi: int, seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    draw = rng.lognormal(mean=math.log(median), sigma=sigma, size=n)
    return [int(v) for v in np.clip(np.rint(draw), lo, hi)]


def seat_decode_config1(seed: int = 1, B: int = 8, cached: int = 511, dtype=torch.bfloat16):
    """Config 1 on the CPU: q ``(B, H, 1, D)``, K/V ``(B, H_kv, L, D)`` with L = cached + 1.

    Q, K, V ~ N(0, 1) drawn in fp32 from one generator, RoPE (theta 1e6) applied to q at
    position ``cached`` and to K at positions ``0..cached``, then cast to ``dtype``.
    """
    H, H_kv, D, theta = QWEN3_ATTN["H"], QWEN3_ATTN["H_kv"], QWEN3_ATTN["D"], QWEN3_ATTN["rope_theta"]
    L = cached + 1
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, 1, D, generator=gen)
    k = torch.randn(B, H_kv, L, D, generator=gen)
    v = torch.randn(B, H_kv, L, D, generator=gen)
    q = rope(q, torch.tensor([cached]), theta)
    k = rope(k, torch.arange(L), theta)
    return q.to(dtype), k.to(dtype), v.to(dtype)


@dataclass
class PagedDecodeInputs:
    q: list            # per layer (B, H, D)
    k_caches: list     # per layer (n_blocks, bs, H_kv, D)
    v_caches: list
    block_table: torch.Tensor  # (B, max_blocks) int32
    seqlen: torch.Tensor       # (B,) int32
    tables: list
    lengths: list
    block_size: int

    @property
    def tokens(self) -> int:
        return int(sum(self.lengths))


def paged_decode_config(
    *, B: int = 32, lengths=None, lo: int = 128, hi: int = 2048, n_blocks: int = 8192,
    n_layer: int = 28, seed: int = 2, device="cuda", dtype=torch.bfloat16, max_blocks: int | None = None,
    H: int | None = None, H_kv: int | None = None, D: int | None = None, block_size: int | None = None,
    head_major: bool = False,
) -> PagedDecodeInputs:
    """Configs 2 and 4: a paged pool per layer, disjoint permuted tables, seqlen per row.

    ``lengths`` overrides the U[lo, hi] draw (config 4 passes ``[8192] * 32``).
    ``head_major`` stores each pool as (n_blocks, H_kv, block_size, D) in memory (each KV
    head's tokens of a block contiguous) and hands out its (n_blocks, block_size, H_kv, D)
    view, the reference's logical layout, with the strides of the head-major storage.
    """
    H = H or QWEN3_ATTN["H"]
    H_kv = H_kv or QWEN3_ATTN["H_kv"]
    D = D or QWEN3_ATTN["D"]
    bs = block_size or QWEN3_ATTN["block_size"]
    gen = torch.Generator().manual_seed(seed)
    if lengths is None:
        lengths = torch.randint(lo, hi + 1, (B,), generator=gen).tolist()
    lengths = [int(x) for x in lengths]
    tables = block_tables_from_perm(lengths, n_blocks, bs, seed + 1)
    width = max_blocks or max(len(t) for t in tables)
    table = torch.zeros(B, width, dtype=torch.int32)
    for row, t in enumerate(tables):
        table[row, : len(t)] = torch.tensor(t, dtype=torch.int32)
    dev = torch.device(device)
    dgen = torch.Generator(device=dev).manual_seed(seed + 2)
    if head_major:
        shape = (n_blocks, H_kv, bs, D)
        k_caches = [_randn(shape, dgen, dev, dtype).permute(0, 2, 1, 3) for _ in range(n_layer)]
        v_caches = [_randn(shape, dgen, dev, dtype).permute(0, 2, 1, 3) for _ in range(n_layer)]
    else:
        shape = (n_blocks, bs, H_kv, D)
        k_caches = [_randn(shape, dgen, dev, dtype) for _ in range(n_layer)]
        v_caches = [_randn(shape, dgen, dev, dtype) for _ in range(n_layer)]
    q = [_randn((B, H, D), dgen, dev, dtype) for _ in range(n_layer)]
    return PagedDecodeInputs(q, k_caches, v_caches, table.to(dev), torch.tensor(lengths, dtype=torch.int32, device=dev),
                             tables, lengths, bs)


def _randn(shape, gen, device, dtype) -> torch.Tensor:
    """N(0, 1) drawn in fp32 and cast, in slabs so a multi-GiB pool never needs a second
    full-size fp32 copy."""
    out = torch.empty(shape, dtype=dtype, device=device)
    flat = out.view(-1)
    step = 1 << 26
    for start in range(0, flat.numel(), step):
        n = min(step, flat.numel() - start)
        flat[start: start + n] = torch.randn(n, generator=gen, device=device, dtype=torch.float32).to(dtype)
    return out


@dataclass
class PrefillInputs:
    q: torch.Tensor   # (T, H, D)
    k: torch.Tensor   # (T, H_kv, D)
    v: torch.Tensor
    cu_seqlens: list
    lengths: list
    tables: list
    slots: torch.Tensor  # (T,) int64 packed slot map
    n_blocks: int
    block_size: int


def prefill_config3(*, n_prompts: int = 8, median: float = 512, sigma: float = PROMPT_SIGMA, lo: int = 64,
                    hi: int = 2048, seed: int = 3, n_blocks: int = 4096, device="cpu",
                    dtype=torch.bfloat16, lengths=None, H: int | None = None, H_kv: int | None = None,
                    D: int | None = None) -> PrefillInputs:
    """Config 3: packed prompts, Q/K/V ~ N(0, 1), and a seeded disjoint slot mapping."""
    H = H or QWEN3_ATTN["H"]
    H_kv = H_kv or QWEN3_ATTN["H_kv"]
    D = D or QWEN3_ATTN["D"]
    bs = QWEN3_ATTN["block_size"]
    if lengths is None:
        lengths = lognormal_lengths(n_prompts, median, sigma, lo, hi, seed)
    lengths = [int(x) for x in lengths]
    total = sum(lengths)
    cu = [0]
    for length in lengths:
        cu.append(cu[-1] + length)
    gen = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(total, H, D, generator=gen).to(dtype)
    k = torch.randn(total, H_kv, D, generator=gen).to(dtype)
    v = torch.randn(total, H_kv, D, generator=gen).to(dtype)
    tables = block_tables_from_perm(lengths, n_blocks, bs, seed + 2)
    slots = torch.from_numpy(np.concatenate([slot_map(t, 0, n, bs) for t, n in zip(tables, lengths)]))
    dev = torch.device(device)
    return PrefillInputs(q.to(dev), k.to(dev), v.to(dev), cu, lengths, tables, slots.to(dev), n_blocks, bs)
