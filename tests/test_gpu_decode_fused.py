"""The fused decode launch (mi_paged_decode_fused, ``PagedDecodePlan.run_fused``) against the
two launches it replaces: ``PagedPool.write_qk_norm_rope`` (q/k RMSNorm + RoPE + the new
token's K/V write, reference model/layers.py:193-211 and model/paged.py:503-520) followed by
``PagedDecodePlan.run`` (reference model/triton_decode.py:250-328).

The fused kernel recomputes q in the decode workgroups' own lane layout, reproducing the
epilogue's fp32 sum of squares through the same butterfly, and reads the new token's k/v
from registers rather than from the pool: the bar is bit equality of the attention output
and of both pools afterwards, on split-K partial inputs and plain ones, idle rows, refused
rows and rows whose new token is their only token.
"""

from __future__ import annotations

import pytest
import torch

from miattn import PagedPool, paged_decode_plan
from miattn.qwen3 import rope_table
from miattn.rows import Parts

pytestmark = pytest.mark.gpu

H, H_KV, D, BS, EPS = 16, 8, 128, 16, 1e-6


def _case(lengths, *, parts, dtype=torch.bfloat16, seed=0, n_pos=4096, slot_bits=64, idle=(), bad_slot=(),
          heads=(H, H_KV)):
    n_head, n_kv = heads
    width_qkv = (n_head + 2 * n_kv) * D
    g = torch.Generator().manual_seed(seed)
    B = len(lengths)
    need = [max(1, -(-n // BS)) for n in lengths]
    n_blocks = 2 * sum(need) + 8
    perm = torch.randperm(n_blocks, generator=g).tolist()
    width = max(need)
    table = torch.full((B, width), 0, dtype=torch.int32)
    at = 0
    for r, k in enumerate(need):
        table[r, :k] = torch.tensor(perm[at:at + k], dtype=torch.int32)
        at += k
    pools = []
    keys = torch.randn(n_blocks, BS, n_kv, D, generator=g).to(dtype)
    vals = torch.randn(n_blocks, BS, n_kv, D, generator=g).to(dtype)
    for _ in range(2):
        pool = PagedPool(1, n_blocks, BS, n_kv, D, dtype=dtype, device="cuda", n_head=n_head)
        pool.keys[0].copy_(keys)
        pool.values[0].copy_(vals)
        pools.append(pool)
    seqlen = torch.tensor(lengths, dtype=torch.int32)
    pos = seqlen.to(torch.int64) - 1
    slots = torch.tensor([int(table[r, p // BS]) * BS + p % BS if p >= 0 else -1 for r, p in enumerate(pos.tolist())],
                         dtype=torch.int64)
    for r in idle:
        slots[r], pos[r], seqlen[r] = -1, -1, 0
    for r in bad_slot:
        slots[r] = n_blocks * BS + 3
    if parts:
        qkv = Parts((torch.randn(parts, B, width_qkv, generator=g) * 2.0).cuda(), dtype)
    else:
        qkv = (torch.randn(B, width_qkv, generator=g) * 2.0).to(dtype).cuda()
    qn = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype).cuda()
    kn = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype).cuda()
    cos, sin = rope_table(D, 1e6, n_pos, "cuda", dtype)
    slot_dtype = torch.int32 if slot_bits == 32 else torch.int64
    return (pools, table.cuda(), seqlen.cuda(), pos.cuda(), slots.to(slot_dtype).cuda(), qkv, qn, kn, cos, sin)


def _both(case):
    pools, table, seqlen, pos, slots, qkv, qn, kn, cos, sin = case
    B = table.shape[0]
    q0 = torch.zeros(B, pools[0].n_head, D, dtype=pools[0].dtype, device="cuda")
    plan_a = paged_decode_plan(q0, pools[0].keys, pools[0].values, table, seqlen)
    plan_b = paged_decode_plan(q0, pools[1].keys, pools[1].values, table, seqlen)
    q = pools[0].write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos, EPS)
    out_a = plan_a.run(0, q)
    assert plan_b.fused_supported(pools[1].dtype, 2 * cos.shape[1])
    out_b = plan_b.run_fused(0, qkv, qn, kn, cos, sin, pos, slots, EPS, error_word=pools[1].write_error_word)
    torch.cuda.synchronize()
    return pools, out_a, out_b


def _assert_same(pools, out_a, out_b):
    assert torch.isfinite(out_a.float()).all()
    assert torch.equal(out_a, out_b), f"{int((out_a != out_b).sum())} output elements differ"
    assert torch.equal(pools[0].keys[0], pools[1].keys[0])
    assert torch.equal(pools[0].values[0], pools[1].values[0])


@pytest.mark.parametrize("parts", [0, 1, 2, 8], ids=["plain", "parts1", "parts2", "parts8"])
def test_fused_equals_epilogue_then_decode_config2_lengths(parts):
    """B = 32 rows with lengths U[128, 2048] (config 2's shape), the decode step's layout:
    each row's new token at seqlen - 1."""
    g = torch.Generator().manual_seed(3)
    lengths = torch.randint(128, 2049, (32,), generator=g).tolist()
    pools, out_a, out_b = _both(_case(lengths, parts=parts, seed=parts))
    _assert_same(pools, out_a, out_b)
    pools[0].check_writes()
    pools[1].check_writes()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("slot_bits", [32, 64])
def test_fused_short_rows_idle_rows_and_dtypes(dtype, slot_bits):
    """Rows of 1 token (the new token is the whole row: the only split is the last one), rows
    ending on a block boundary and one past it, and idle rows (slot -1, seqlen 0)."""
    lengths = [1, 2, 15, 16, 17, 33, 300, 1, 64, 129]
    pools, out_a, out_b = _both(_case(lengths, parts=2, dtype=dtype, seed=7, slot_bits=slot_bits, idle=(3, 8)))
    _assert_same(pools, out_a, out_b)
    assert not out_b[3].any() and not out_b[8].any()


@pytest.mark.parametrize("bad", ["position", "slot"])
def test_fused_refused_row_is_reported_and_matches(bad):
    """A row whose position is outside the RoPE table, or whose slot is outside the pool, is
    written by neither form, attends with q = 0 in both, and is reported by both."""
    lengths = [40, 700, 90, 1200]
    if bad == "position":
        case = _case(lengths, parts=2, seed=11, n_pos=1000)       # row 3's position 1199 is past the table
    else:
        case = _case(lengths, parts=2, seed=11, bad_slot=(1,))
    pools, out_a, out_b = _both(case)
    _assert_same(pools, out_a, out_b)
    for pool in pools:
        with pytest.raises(IndexError):
            pool.check_writes()


def test_fused_rejects_shapes_it_does_not_cover():
    pools, table, seqlen, pos, slots, qkv, qn, kn, cos, sin = _case([20, 30], parts=0, seed=2)
    q0 = torch.zeros(2, H, D, dtype=torch.bfloat16, device="cuda")
    plan = paged_decode_plan(q0, pools[1].keys, pools[1].values, table, seqlen)
    assert not plan.fused_supported(torch.bfloat16, 64)
    with pytest.raises(ValueError, match="whole-head RoPE"):
        plan.run_fused(0, qkv, qn, kn, cos[:, :32].contiguous(), sin[:, :32].contiguous(), pos, slots, EPS)
    with pytest.raises(ValueError, match="int64"):
        plan.run_fused(0, qkv, qn, kn, cos, sin, pos.int(), slots, EPS)


@pytest.mark.parametrize("heads", [(16, 16), (32, 4), (8, 2), (64, 8)], ids=["mha16", "gqa8-4kv", "gqa4-2kv", "gqa8-8kv"])
def test_fused_other_head_groupings(heads):
    """Other GQA groupings at head_dim 128: the workgroup's KV heads and query heads per lane
    change, and with them which q heads each lane normalises and rotates; bit-equal to the two
    launches."""
    pools, out_a, out_b = _both(_case([5, 700, 33, 1500, 129], parts=2, seed=13, heads=heads))
    _assert_same(pools, out_a, out_b)
