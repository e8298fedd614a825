"""Pin the packed-prefill oracles: longhand vs SDPA per segment vs brute force, plus the
reference's isolation invariants."""

from __future__ import annotations

import pytest
import torch

from oracle.varlen import brute_force_varlen, longhand_varlen, sdpa_varlen, varlen_error_bound


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


def _emulated_kernel(q, k, v, cu, *, bits=8, scale_error=1.0, drop_diagonal=False, sum_rounded=True):
    """A float64 emulation of a kernel that rounds P to a ``bits``-bit significand before the
    PV product (bits=8: bf16) and rounds the output to bf16, with mistakes to plant."""
    D = q.shape[-1]
    group = q.size(1) // k.size(1)
    outs = []
    for start, end in zip(cu, cu[1:]):
        n = end - start
        qs = q[start:end].double().transpose(0, 1)
        ks = k[start:end].double().transpose(0, 1).repeat_interleave(group, dim=0)
        vs = v[start:end].double().transpose(0, 1).repeat_interleave(group, dim=0)
        s = qs @ ks.transpose(-1, -2) * (scale_error / D ** 0.5)
        mask = torch.ones(n, n, dtype=torch.bool).tril(-1 if drop_diagonal else 0)
        mask[0, 0] = True  # row 0 keeps its one key
        s = s.masked_fill(~mask, float("-inf"))
        p = torch.exp(s - s.amax(-1, keepdim=True))
        mant, expo = torch.frexp(p)
        p16 = torch.ldexp(torch.round(mant * 2.0 ** bits) / 2.0 ** bits, expo)
        o = (p16 @ vs) / (p16 if sum_rounded else p).sum(-1, keepdim=True)
        outs.append(o.transpose(0, 1))
    return torch.cat(outs).to(torch.bfloat16).float()


BOUND_CASE = ([1, 2, 3, 5, 17, 64, 130], 8, 2, 64)


@pytest.mark.parametrize("sum_rounded", [True, False], ids=["sum-of-rounded-p", "sum-of-fp32-p"])
def test_error_bound_holds_for_a_16_bit_p_kernel_and_is_not_vacuous(sum_rounded):
    lengths, H, H_kv, D = BOUND_CASE
    worst = 0.0
    for seed in range(3):
        q, k, v, cu = _packed(lengths, H, H_kv, D, seed=40 + seed)
        q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
        ref, bound = varlen_error_bound(q, k, v, cu)
        torch.testing.assert_close(ref, longhand_varlen(q, k, v, cu), atol=1e-5, rtol=0)
        err = (_emulated_kernel(q, k, v, cu, sum_rounded=sum_rounded) - ref).abs()
        assert (err <= bound).all()
        worst = max(worst, (err / bound).max().item())
    assert worst > 0.3, f"the bound is loose by {1 / worst:.1f}x on this case"


@pytest.mark.parametrize("mistake", [dict(bits=6), dict(scale_error=1.01), dict(drop_diagonal=True)],
                         ids=["p-rounded-to-6-bits", "scale-off-by-1pc", "diagonal-key-dropped"])
def test_error_bound_catches_planted_mistakes(mistake):
    lengths, H, H_kv, D = BOUND_CASE
    q, k, v, cu = _packed(lengths, H, H_kv, D, seed=40)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    ref, bound = varlen_error_bound(q, k, v, cu)
    err = (_emulated_kernel(q, k, v, cu, **mistake) - ref).abs()
    assert (err > bound).any()


def test_error_bound_on_one_key_rows():
    """A row that sees one key returns that key's v, and its bound is the two roundings
    (output and probability, each ``u |v|``) plus fp32 slack of order 1e-5 relative."""
    q, k, v, cu = _packed([1, 1, 1], 4, 2, 16, seed=9)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    ref, bound = varlen_error_bound(q, k, v, cu)
    assert torch.equal(ref, v.float().repeat_interleave(2, dim=1))
    u = 2.0 ** -8
    slack = (bound - (2 * u + 2 * u * u) * ref.abs()) / ref.abs()
    assert (slack >= 0).all() and (slack <= 5e-5).all()
