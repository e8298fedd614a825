"""Pin the CPU seat-path restatement: slab write/mask/bias + hand_baddbmm math."""

from __future__ import annotations

import math

import torch

from oracle.decode import dense_decode_f64
from oracle.seat import SeatSlab, additive_bias, seat_decode


def _paged_view(k, v, lengths):
    """Lay a (B, H_kv, L, D) slab into a trivially paged pool (one row per block run)."""
    B, H_kv, L, D = k.shape
    bs = 16
    pages = (L + bs - 1) // bs
    pool_k = torch.zeros(B * pages, bs, H_kv, D, dtype=k.dtype)
    pool_v = torch.zeros_like(pool_k)
    table = torch.zeros(B, pages, dtype=torch.int32)
    for b in range(B):
        for p in range(pages):
            blk = b * pages + p
            table[b, p] = blk
            cols = slice(p * bs, min(L, p * bs + bs))
            n = cols.stop - cols.start
            pool_k[blk, :n] = k[b, :, cols].permute(1, 0, 2)
            pool_v[blk, :n] = v[b, :, cols].permute(1, 0, 2)
    return pool_k, pool_v, table, torch.tensor(lengths, dtype=torch.int32)


def test_seat_decode_matches_float64_oracle_fp32_and_bf16():
    gen = torch.Generator().manual_seed(4)
    B, H, H_kv, L, D = 3, 8, 4, 40, 32
    lengths = [40, 17, 1]
    q = torch.randn(B, H, 1, D, generator=gen)
    k = torch.randn(B, H_kv, L, D, generator=gen)
    v = torch.randn(B, H_kv, L, D, generator=gen)
    mask = torch.arange(L).view(1, 1, 1, L) < torch.tensor(lengths).view(-1, 1, 1, 1)
    pk, pv, table, seqlen = _paged_view(k, v, lengths)
    ref = dense_decode_f64(q[:, :, 0], pk, pv, table, seqlen).double()
    for dtype, atol in ((torch.float32, 1e-5), (torch.bfloat16, 2e-2)):
        bias = additive_bias(mask, dtype, B, H_kv, H // H_kv)
        out = seat_decode(q.to(dtype), k.to(dtype), v.to(dtype), bias)[:, :, 0]
        torch.testing.assert_close(out.double(), ref, atol=atol, rtol=0)


def test_dead_row_bias_is_zeroed_not_nan():
    mask = torch.zeros(1, 1, 1, 5, dtype=torch.bool)
    bias = additive_bias(mask, torch.float32, 1, 1, 2)
    assert torch.equal(bias, torch.zeros(1, 2, 5))
    q = torch.randn(1, 2, 1, 4)
    k = torch.zeros(1, 1, 5, 4)
    v = torch.randn(1, 1, 5, 4)
    out = seat_decode(q, k, v, bias)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out[0, 0, 0], v[0, 0].mean(0))


def test_slab_step_protocol_writes_and_masks():
    slab = SeatSlab(1, 2, 1, 4, 8, n_head=2)
    slab.activate(0, 3)
    slab.activate(1, 0)
    slab.build_mask(next_token=True)
    assert slab.mask[0, 0, 0].tolist() == [True] * 4 + [False] * 4
    assert slab.mask[1, 0, 0].tolist() == [True] + [False] * 7
    k = torch.randn(2, 1, 1, 4)
    slab.write(0, k, k)
    assert torch.equal(slab.keys[0][0, :, 3], k[0, :, 0]) and torch.equal(slab.keys[0][1, :, 0], k[1, :, 0])
    slab.advance()
    assert slab.pos.tolist() == [4, 1] and slab.valid.tolist() == [4, 1]
    slab.freeze(1)
    slab.build_mask(next_token=True)
    assert not slab.mask[1].any(), "a frozen seat is closed"


def test_seat_softmax_runs_in_the_input_dtype():
    """bf16 scores/probabilities are what the reference computes (reference
    model/attention/hand_baddbmm.py:28-30); an fp32-upcast softmax differs in the last bits."""
    gen = torch.Generator().manual_seed(9)
    q = torch.randn(2, 2, 1, 64, generator=gen).bfloat16()
    k = torch.randn(2, 1, 300, 64, generator=gen).bfloat16()
    v = torch.randn(2, 1, 300, 64, generator=gen).bfloat16()
    out = seat_decode(q, k, v, None)
    assert out.dtype == torch.bfloat16
    qg = (q.float() / math.sqrt(64)).reshape(2, 2, 64)
    up = torch.bmm(torch.softmax(torch.bmm(qg, k.float().reshape(2, 300, 64).transpose(1, 2)), -1),
                   v.float().reshape(2, 300, 64)).reshape(2, 2, 1, 64)
    assert (out.float() - up).abs().max() < 2e-2
