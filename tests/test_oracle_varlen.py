"""Pin the packed-prefill oracles: longhand vs SDPA per segment vs brute force, plus the
reference's isolation invariants."""

from __future__ import annotations

import pytest
import torch

from oracle.varlen import brute_force_varlen, longhand_varlen, sdpa_varlen


def _packed(lengths, H, H_kv, D, seed=0):
    gen = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    q = torch.randn(T, H, D, generator=gen)
    k = torch.randn(T, H_kv, D, generator=gen)
    v = torch.randn(T, H_kv, D, generator=gen)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return q, k, v, cu


@pytest.mark.parametrize("causal", [True, False])
def test_brute_force_pins_both_formulations(causal):
    q, k, v, cu = _packed([1, 5, 3], 4, 2, 8, seed=1)
    ref = brute_force_varlen(q, k, v, cu, causal=causal)
    torch.testing.assert_close(longhand_varlen(q, k, v, cu, causal=causal, dtype=torch.float64), ref,
                               atol=1e-10, rtol=0)
    torch.testing.assert_close(sdpa_varlen(q.double(), k.double(), v.double(), cu, causal=causal), ref,
                               atol=1e-10, rtol=0)


@pytest.mark.parametrize("lengths", [[1], [17], [1, 17, 128, 300], [1, 1, 17, 128, 3, 64, 200]])
@pytest.mark.parametrize("H,H_kv", [(8, 4), (8, 1), (16, 8)])
def test_longhand_matches_sdpa(lengths, H, H_kv):
    q, k, v, cu = _packed(lengths, H, H_kv, 64, seed=2)
    torch.testing.assert_close(longhand_varlen(q, k, v, cu), sdpa_varlen(q, k, v, cu), atol=1e-5, rtol=0)


def test_first_token_of_a_causal_segment_returns_its_own_value():
    q, k, v, cu = _packed([4, 6], 4, 2, 16, seed=3)
    out = longhand_varlen(q, k, v, cu)
    for start in cu[:-1]:
        for h in range(4):
            torch.testing.assert_close(out[start, h], v[start, h // 2])


def test_segment_isolation():
    q, k, v, cu = _packed([17, 1, 128], 8, 4, 32, seed=5)
    before = longhand_varlen(q, k, v, cu)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[:17] = torch.randn(17, 8, 32)
    k2[:17] = torch.randn(17, 4, 32)
    after = longhand_varlen(q2, k2, v2, cu)
    assert not torch.equal(after[:17], before[:17])
    assert torch.equal(after[17:], before[17:])


def test_a_planted_mask_mistake_fails_brute_force():
    """An off-by-one causal mask (letting token i see i+1) must fail the pin."""
    q, k, v, cu = _packed([6], 2, 1, 8, seed=6)
    ref = brute_force_varlen(q, k, v, cu)
    qs, ks, vs = q.double().transpose(0, 1), k.double().transpose(0, 1).repeat(2, 1, 1), v.double().transpose(0, 1).repeat(2, 1, 1)
    s = qs @ ks.transpose(-1, -2) / 8 ** 0.5
    s = s.masked_fill(~torch.ones(6, 6, dtype=torch.bool).tril(1), float("-inf"))
    wrong = (torch.softmax(s, -1) @ vs).transpose(0, 1)
    assert (wrong - ref).abs().max() > 1e-3
