"""Pin the paged-decode oracles: both formulations against float64 SDPA on the gathered
dense K/V, plus closed forms (empty row, one token, equal keys, GQA head map)."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle.decode import dense_decode_f64, dense_kv, reference_paged_decode


def _build(B, H, H_kv, D, bs, lengths, *, seed=0, n_blocks=None, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    pages = [(n + bs - 1) // bs for n in lengths]
    max_pages = max(max(pages), 1)
    n_blocks = n_blocks or max(B * max_pages, max_pages + 4)
    k = torch.randn(n_blocks, bs, H_kv, D, generator=gen).to(dtype)
    v = torch.randn(n_blocks, bs, H_kv, D, generator=gen).to(dtype)
    q = torch.randn(B, H, D, generator=gen).to(dtype)
    table = torch.zeros(B, max_pages, dtype=torch.int32)
    for row, n in enumerate(pages):
        if n:
            table[row, :n] = torch.randperm(n_blocks, generator=gen)[:n].to(torch.int32)
    return q, k, v, table, torch.tensor(lengths, dtype=torch.int32)


def _sdpa_f64(q, k, v, table, seqlen, scale):
    B, H, D = q.shape
    H_kv = k.shape[2]
    out = torch.zeros(B, H, D, dtype=torch.float64)
    for b in range(B):
        n = int(seqlen[b])
        if n == 0:
            continue
        kk, vv = dense_kv(k, v, table[b], n)
        out[b] = F.scaled_dot_product_attention(
            q[b].double().view(1, H, 1, D), kk.double().permute(1, 0, 2).unsqueeze(0),
            vv.double().permute(1, 0, 2).unsqueeze(0), scale=scale, enable_gqa=H != H_kv,
        ).view(H, D)
    return out


CASES = [
    (1, 2, 1, 8, 16, [1]), (2, 4, 2, 8, 16, [15, 16]), (1, 4, 2, 16, 16, [17]),
    (2, 4, 4, 8, 16, [32, 0]), (2, 4, 2, 16, 32, [100, 33]), (3, 2, 2, 8, 32, [16, 17, 15]),
    (2, 16, 8, 128, 16, [300, 77]),
]


@pytest.mark.parametrize("B,H,H_kv,D,bs,lengths", CASES)
def test_both_oracles_match_float64_sdpa(B, H, H_kv, D, bs, lengths):
    q, k, v, table, seqlen = _build(B, H, H_kv, D, bs, lengths, seed=3)
    scale = 1.0 / math.sqrt(D)
    ref = _sdpa_f64(q, k, v, table, seqlen, scale)
    torch.testing.assert_close(dense_decode_f64(q, k, v, table, seqlen).double(), ref, atol=1e-6, rtol=0)
    torch.testing.assert_close(reference_paged_decode(q, k, v, table, seqlen).double(), ref, atol=1e-5, rtol=0)


def test_explicit_scale_and_duplicated_blocks():
    """Repeated block ids and an unused table tail of -999 (reference
    tests/unit/test_triton_decode.py:147-169)."""
    q, k, v, _, _ = _build(2, 4, 2, 8, 16, [50, 64], seed=7, n_blocks=6)
    table = torch.tensor([[3, 0, 3, 5, -999, -999], [5, 1, 4, 0, -999, -999]], dtype=torch.int32)
    seqlen = torch.tensor([50, 64], dtype=torch.int32)
    for scale in (None, 0.375):
        s = 1.0 / math.sqrt(8) if scale is None else scale
        ref = _sdpa_f64(q, k, v, table, seqlen, s)
        torch.testing.assert_close(dense_decode_f64(q, k, v, table, seqlen, scale).double(), ref, atol=1e-6, rtol=0)
        torch.testing.assert_close(reference_paged_decode(q, k, v, table, seqlen, scale=scale).double(), ref,
                                   atol=1e-5, rtol=0)


def test_closed_forms():
    q, k, v, table, seqlen = _build(3, 4, 2, 8, 16, [0, 1, 20], seed=11)
    # equal keys in row 2: softmax is uniform, the result is the mean of V
    blk = table[2, :2].long()
    k[blk] = 1.0
    for fn in (dense_decode_f64, reference_paged_decode):
        out = fn(q, k, v, table, seqlen)
        assert not out[0].any(), "an empty row decodes to exact zeros"
        b0 = int(table[1, 0])
        for h in range(4):
            assert torch.allclose(out[1, h], v[b0, 0, h // 2], atol=1e-6), "one token returns v"
        kk, vv = dense_kv(k, v, table[2], 20)
        for h in range(4):
            assert torch.allclose(out[2, h], vv[:, h // 2].mean(0), atol=1e-5)


def test_gqa_head_map_is_h_div_group():
    """Heads 0,1 read KV head 0 and heads 2,3 read KV head 1: zeroing KV head 1's V must
    zero exactly heads 2 and 3."""
    q, k, v, table, seqlen = _build(1, 4, 2, 8, 16, [9], seed=5)
    v[:, :, 1] = 0.0
    for fn in (dense_decode_f64, reference_paged_decode):
        out = fn(q, k, v, table, seqlen)
        assert out[0, 2:].abs().max() == 0 and out[0, :2].abs().max() > 0


def test_a_planted_scale_mistake_fails_the_library_pin():
    q, k, v, table, seqlen = _build(2, 4, 2, 16, 16, [40, 9], seed=2)
    ref = _sdpa_f64(q, k, v, table, seqlen, 1.0 / math.sqrt(16))
    wrong = dense_decode_f64(q, k, v, table, seqlen, scale=1.0 / 16)
    assert (wrong.double() - ref).abs().max() > 1e-3
