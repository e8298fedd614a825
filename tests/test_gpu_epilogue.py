"""The fused decode-step epilogue (q/k RMSNorm + RoPE + paged K/V write, one HIP launch)
against the reference's tensor-op chain run on the same device.

The chain is the reference's (``model/layers.py:342-350`` RMSNorm, ``:59-89``
``apply_rotary_emb``, ``model/paged.py:503-520`` the write), restated by
``miattn.qwen3.rms_norm`` / ``apply_rope`` and ``PagedPool.write_slots``. The kernel rounds
each step to the activation dtype as those ops do, so outputs are equal except where the
fp32 sum of squares, accumulated in another order than torch's reduction, crosses a
rounding boundary of the mean: a few elements may then differ by one or two ulps (1/128
relative in bf16). V is a copy: bit-exact.
"""

from __future__ import annotations

import pytest
import torch

from miattn import PagedPool
from miattn.qwen3 import apply_rope, rms_norm, rope_table

pytestmark = pytest.mark.gpu


def _case(B, H, H_kv, D, dtype, seed, n_blocks=64, bs=16, n_pos=4096, slot_dtype=torch.int64):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(B, (H + 2 * H_kv) * D, generator=g) * 2.0).to(dtype).cuda()
    qn = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype).cuda()
    kn = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype).cuda()
    cos, sin = rope_table(D, 1e6, n_pos, "cuda", dtype)
    pos = torch.randint(0, n_pos, (B,), generator=g).cuda()
    slots = torch.randperm(n_blocks * bs, generator=g)[:B].to(slot_dtype).cuda()
    return qkv, qn, kn, cos, sin, pos, slots


def _reference(pool_ref, layer, qkv, qn, kn, cos, sin, pos, slots, H, H_kv, D, eps):
    B = qkv.shape[0]
    q = qkv[:, : H * D].view(B, 1, H, D)
    k = qkv[:, H * D:(H + H_kv) * D].view(B, 1, H_kv, D)
    v = qkv[:, (H + H_kv) * D:].view(B, 1, H_kv, D)
    q, k = rms_norm(q, qn, eps), rms_norm(k, kn, eps)
    c, s = cos[pos].unsqueeze(1), sin[pos].unsqueeze(1)
    q, k = apply_rope(q, c, s), apply_rope(k, c, s)
    pool_ref.write_slots(layer, slots, k[:, 0], v[:, 0])
    return q[:, 0]


def _ulps(a, b, dtype):
    # distance in units of the dtype's last place at b's magnitude
    eps = torch.finfo(dtype).eps
    scale = torch.clamp(b.float().abs(), min=torch.finfo(dtype).tiny)
    return ((a.float() - b.float()).abs() / (scale * eps)).max().item()


@pytest.mark.parametrize("B,H,H_kv,D", [(32, 16, 8, 128), (5, 8, 2, 256), (7, 4, 4, 64), (1, 16, 8, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_epilogue_matches_the_reference_op_chain(B, H, H_kv, D, dtype, slot_dtype):
    eps = 1e-6
    qkv, qn, kn, cos, sin, pos, slots = _case(B, H, H_kv, D, dtype, seed=B * 7 + D, slot_dtype=slot_dtype)
    pool = PagedPool(2, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H, strict_writes=True)
    ref = PagedPool(2, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H, strict_writes=True)
    q = pool.write_qk_norm_rope(1, slots, qkv, qn, kn, cos, sin, pos, eps)
    q_ref = _reference(ref, 1, qkv, qn, kn, cos, sin, pos, slots, H, H_kv, D, eps)
    torch.cuda.synchronize()
    assert q.shape == (B, H, D) and q.is_contiguous()
    assert torch.equal(pool.values[1], ref.values[1])  # v: a copy
    assert torch.equal(pool.keys[0], ref.keys[0]) and torch.equal(pool.values[0], ref.values[0])  # other layer untouched
    for got, want in ((q, q_ref), (pool.keys[1], ref.keys[1])):
        same = (got == want).float().mean().item()
        assert same > 0.999, f"only {same:.4%} of elements equal"
        assert _ulps(got, want, dtype) <= 2.0


def test_epilogue_rejects_bad_rows_without_writing():
    H, H_kv, D, dtype = 16, 8, 128, torch.bfloat16
    qkv, qn, kn, cos, sin, pos, slots = _case(4, H, H_kv, D, dtype, seed=3)
    pool = PagedPool(1, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H)
    slots[2] = pool.n_slots  # outside the pool
    pool.write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos, 1e-6)
    with pytest.raises(IndexError):
        pool.check_writes()
    written = (pool.keys[0].view(pool.n_slots, -1) != 0).any(1)
    assert written.sum().item() == 3 and not written[slots[[0, 1, 3]].cpu()].logical_not().any()
    # the rejected row's q is zero-filled rather than left as whatever the allocation held
    q = pool.write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos, 1e-6)
    with pytest.raises(IndexError):
        pool.check_writes()
    assert not q[2].any() and q[[0, 1, 3]].abs().amax(-1).gt(0).all()
    pos[1] = cos.shape[0]  # outside the RoPE table
    slots[2] = 5
    pool2 = PagedPool(1, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H)
    pool2.write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos, 1e-6)
    with pytest.raises(IndexError):
        pool2.check_writes()


def test_epilogue_idle_rows_write_nothing_and_get_zero_outputs():
    """slot -1 (an idle seat): nothing reaches the pool, no error is reported, and the row's
    q (and packed k / v when asked for) are zeros, not the allocation's old contents."""
    H, H_kv, D, dtype = 16, 8, 128, torch.bfloat16
    qkv, qn, kn, cos, sin, pos, slots = _case(4, H, H_kv, D, dtype, seed=5)
    slots[1] = -1
    pool = PagedPool(1, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H, strict_writes=True)
    k_out = torch.full((4, H_kv, D), 7.0, dtype=dtype, device="cuda")
    v_out = torch.full((4, H_kv, D), 7.0, dtype=dtype, device="cuda")
    q = pool.write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos, 1e-6, k_out=k_out, v_out=v_out)
    torch.cuda.synchronize()
    written = (pool.keys[0].view(pool.n_slots, -1) != 0).any(1)
    assert written.sum().item() == 3
    assert not q[1].any() and not k_out[1].any() and not v_out[1].any()
    for b in (0, 2, 3):
        assert q[b].abs().amax(-1).gt(0).all() and torch.equal(pool.values[0].view(-1, H_kv, D)[slots[b]], v_out[b])


def test_epilogue_validates_shapes():
    H, H_kv, D, dtype = 16, 8, 128, torch.bfloat16
    qkv, qn, kn, cos, sin, pos, slots = _case(4, H, H_kv, D, dtype, seed=4)
    pool = PagedPool(1, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H)
    with pytest.raises(ValueError, match="qkv"):
        pool.write_qk_norm_rope(0, slots, qkv[:, 1:], qn, kn, cos, sin, pos, 1e-6)
    with pytest.raises(ValueError, match="pos"):
        pool.write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos.int(), 1e-6)
    with pytest.raises(ValueError, match="cos/sin"):
        pool.write_qk_norm_rope(0, slots, qkv, qn, kn, cos[:, 1:], sin[:, 1:], pos, 1e-6)


def test_packed_prefill_epilogue_matches_the_tensor_ops():
    """PackedPrefill.write_rope: one launch for a packed group's q/k norm + RoPE at each
    token's request-local position, the group's K/V write and the packed k/v the attention
    reads; against the reference's ops (norms, apply_rotary_emb, write_prefill_slots)."""
    from miattn import PackedPrefill, PagedWriteSink

    H, H_kv, D, dtype, eps = 16, 8, 128, torch.bfloat16, 1e-6
    lengths = [100, 37, 260]
    T = sum(lengths)
    g = torch.Generator().manual_seed(21)
    qkv = (torch.randn(T, (H + 2 * H_kv) * D, generator=g) * 2.0).to(dtype).cuda()
    qn = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype).cuda()
    kn = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype).cuda()
    cos, sin = rope_table(D, 1e6, 4096, "cuda", dtype)
    perm = torch.randperm(64, generator=g).tolist()
    tables, at = [], 0
    for n in lengths:
        nb = (n + 15) // 16
        tables.append(perm[at:at + nb])
        at += nb
    positions = torch.cat([torch.arange(n) for n in lengths]).cuda()
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    pools = [PagedPool(1, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H, strict_writes=True)
             for _ in range(2)]
    packed = PackedPrefill(cu_seqlens=cu, positions=positions,
                           sinks=[PagedWriteSink(pools[0], t, n) for t, n in zip(tables, lengths)])
    q, k, v = packed.write_rope(0, qkv, qn, kn, cos, sin, eps)
    slots = packed.group_slots
    q_ref = _reference(pools[1], 0, qkv, qn, kn, cos, sin, positions, slots, H, H_kv, D, eps)
    torch.cuda.synchronize()
    assert q.shape == (1, T, H, D) and k.shape == (1, T, H_kv, D) and v.shape == (1, T, H_kv, D)
    assert (q[0] == q_ref).float().mean().item() > 0.999 and _ulps(q[0], q_ref, dtype) <= 2.0
    keys, vals = pools[0].keys[0].view(-1, H_kv, D), pools[0].values[0].view(-1, H_kv, D)
    assert torch.equal(keys[slots], k[0]) and torch.equal(vals[slots], v[0])  # packed copies = pool rows
    assert torch.equal(v[0], qkv[:, (H + H_kv) * D:].view(T, H_kv, D))
    ref_keys = pools[1].keys[0].view(-1, H_kv, D)[slots]
    assert (k[0] == ref_keys).float().mean().item() > 0.999 and _ulps(k[0], ref_keys, dtype) <= 2.0
    with pytest.raises(RuntimeError, match="already written"):
        packed.write_rope(0, qkv, qn, kn, cos, sin, eps)


# ---------------------------------------------------------------- decode-step small ops
from miattn.qwen3 import add_rms_norm, silu_mul  # noqa: E402
import torch.nn.functional as F  # noqa: E402


@pytest.mark.parametrize("rows,cols", [(32, 1024), (3, 4096), (5, 200)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_delta", [True, False])
def test_add_rms_norm_matches_the_reference_op_chain(rows, cols, dtype, with_delta):
    g = torch.Generator().manual_seed(rows * cols)
    x = torch.randn(rows, cols, generator=g).to(dtype).cuda()
    d = torch.randn(rows, cols, generator=g).to(dtype).cuda() if with_delta else None
    w = (1.0 + 0.1 * torch.randn(cols, generator=g)).to(dtype).cuda()
    s_ref = x + d if with_delta else x.clone()
    h_ref = rms_norm(s_ref, w, 1e-6)
    xs = x.clone()
    x_out, h = add_rms_norm(xs, d, w, 1e-6)
    torch.cuda.synchronize()
    assert x_out is xs and torch.equal(xs, s_ref)  # the residual add is exact per element
    same = (h == h_ref).float().mean().item()
    assert same > 0.999, f"only {same:.4%} equal"
    assert _ulps(h, h_ref, dtype) <= 2.0


@pytest.mark.parametrize("rows,inter", [(32, 3072), (7, 100)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_silu_mul_matches_the_reference_op_chain(rows, inter, dtype):
    g = torch.Generator().manual_seed(rows + inter)
    gu = (torch.randn(rows, 2 * inter, generator=g) * 3).to(dtype).cuda()
    want = F.silu(gu[:, :inter]) * gu[:, inter:]
    got = silu_mul(gu)
    torch.cuda.synchronize()
    same = (got == want).float().mean().item()
    assert same > 0.999, f"only {same:.4%} equal"
    assert _ulps(got, want, dtype) <= 2.0


def test_decode_step_ops_reject_bad_shapes():
    x = torch.zeros(4, 8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="delta"):
        add_rms_norm(x, x[:, :4].contiguous(), torch.ones(8, dtype=torch.bfloat16, device="cuda"), 1e-6)
    with pytest.raises(ValueError, match="gate_up"):
        silu_mul(torch.zeros(4, 7, dtype=torch.bfloat16, device="cuda"))


def _qwen35_norm(x, w, eps):
    """Qwen3.5's zero-centred q/k norm (reference model/qwen35.py:83-89): fp32 throughout,
    ``x * rsqrt(mean(x^2) + eps) * (1 + w)``, cast back once."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w.float())).to(x.dtype)


def _partial_rope(x, cos, sin, rotary):
    """NeoX rotation of the first ``rotary`` elements, tail passed through (reference
    model/layers.py:91-117, ``apply_rotary_emb_partial``)."""
    return torch.cat([apply_rope(x[..., :rotary], cos, sin), x[..., rotary:]], dim=-1)


@pytest.mark.parametrize("B,H,H_kv,D,rotary", [(32, 8, 2, 256, 64), (3, 8, 2, 256, 128), (4, 16, 8, 128, 64)])
@pytest.mark.parametrize("zero_centred", [False, True], ids=["qwen3-norm", "qwen35-norm"])
def test_partial_rope_and_the_zero_centred_norm(B, H, H_kv, D, rotary, zero_centred):
    """Partial RoPE (Qwen3.5: 64 of 256 head dims rotate) and the zero-centred fp32 q/k
    norm against their tensor-op restatements; the unrotated tail is the normed input."""
    dtype, eps = torch.bfloat16, 1e-6
    qkv, qn, kn, _, _, pos, slots = _case(B, H, H_kv, D, dtype, seed=B + rotary)
    if zero_centred:  # a delta around zero, as the checkpoint's weights are
        qn, kn = qn - 1.0, kn - 1.0
    cos, sin = rope_table(rotary, 1e7, 4096, "cuda", dtype)
    pool = PagedPool(1, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H, strict_writes=True)
    q = pool.write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos, eps, rotary_dim=rotary,
                                zero_centred_norm=zero_centred)
    torch.cuda.synchronize()
    qr = qkv[:, : H * D].view(B, H, D)
    kr = qkv[:, H * D:(H + H_kv) * D].view(B, H_kv, D)
    vr = qkv[:, (H + H_kv) * D:].view(B, H_kv, D)
    norm = (lambda x, w: _qwen35_norm(x, w, eps)) if zero_centred else (lambda x, w: rms_norm(x, w, eps))
    c, s = cos[pos], sin[pos]  # (B, rotary/2); apply_rope inserts the head axis
    q_want = _partial_rope(norm(qr, qn), c, s, rotary)
    k_want = _partial_rope(norm(kr, kn), c, s, rotary)
    flat_k = pool.keys[0].view(-1, H_kv, D)[slots]
    assert torch.equal(pool.values[0].view(-1, H_kv, D)[slots], vr)
    for got, want in ((q, q_want), (flat_k, k_want)):
        same = (got == want).float().mean().item()
        assert same > 0.995, f"only {same:.4%} of elements equal"
        assert _ulps(got, want, dtype) <= 2.0
        # the tail past rotary_dim is the normed input itself
        assert _ulps(got[..., rotary:], want[..., rotary:], dtype) <= 1.0


def test_partial_rope_rejects_unsupported_rotary_dims():
    H, H_kv, D, dtype = 8, 2, 256, torch.bfloat16
    qkv, qn, kn, _, _, pos, slots = _case(2, H, H_kv, D, dtype, seed=9)
    cos, sin = rope_table(96, 1e7, 64, "cuda", dtype)
    pool = PagedPool(1, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H)
    with pytest.raises(ValueError, match="rotary_dim"):
        pool.write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos, 1e-6, rotary_dim=96)
