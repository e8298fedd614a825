"""KV slot write on the HIP kernel: bit-exact against the CPU oracle loops (reference
tests/unit/test_paged_kv.py:99-217,440-542, against this build)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from miattn import PackedPrefill, PagedKV, PagedPool, PagedWriteSink
from miattn import workloads as W
from oracle import slots as S

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "slot_kats.json").read_text())
H_KV, D = 2, 4


def _np(t):
    return t.cpu().float().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64], ids=["i32", "i64"])
@pytest.mark.parametrize("layout", ["contiguous", "sink-permuted", "strided-d"])
def test_write_slots_is_bit_exact(dtype, slot_dtype, layout, cuda):
    n_blocks, bs, H_kv, D_ = 64, 16, 8, 128
    pool = PagedPool(1, n_blocks, bs, H_kv, D_, dtype=dtype, device=cuda)
    gen = torch.Generator().manual_seed(3)
    n = 300
    if layout == "contiguous":
        k = torch.randn(n, H_kv, D_, generator=gen).to(dtype)
        v = torch.randn(n, H_kv, D_, generator=gen).to(dtype)
    elif layout == "sink-permuted":  # (1, H, L, D)[0].permute(1, 0, 2), the sink's view
        k = torch.randn(H_kv, n, D_, generator=gen).to(dtype).permute(1, 0, 2)
        v = torch.randn(H_kv, n, D_, generator=gen).to(dtype).permute(1, 0, 2)
    else:  # every other element of a wider buffer: not 16-byte vectorisable
        k = torch.randn(n, H_kv, 2 * D_, generator=gen).to(dtype)[..., ::2]
        v = torch.randn(n, H_kv, 2 * D_, generator=gen).to(dtype)[..., ::2]
    slots = torch.randperm(n_blocks * bs, generator=gen)[:n].to(slot_dtype)
    pool.write_slots(0, slots.to(cuda), k.to(cuda), v.to(cuda))
    pool.check_writes()
    ref_k = np.zeros((n_blocks * bs, H_kv, D_), dtype=_np(k[:1]).dtype)
    ref_v = np.zeros_like(ref_k)
    ref_k[slots.numpy()] = _np(k.contiguous())
    ref_v[slots.numpy()] = _np(v.contiguous())
    assert np.array_equal(_np(pool.keys[0]).reshape(-1, H_kv, D_), ref_k)
    assert np.array_equal(_np(pool.values[0]).reshape(-1, H_kv, D_), ref_v)


def test_prefill_known_answers_and_per_block_reference(cuda):
    case = KATS["prefill_shuffled_table"]
    bs, table, n = case["block_size"], case["block_table"], case["length"]
    pool = PagedPool(2, 8, bs, H_KV, D, device=cuda, n_head=4)
    gen = torch.Generator().manual_seed(71)
    k = torch.randn(1, H_KV, n, D, generator=gen)[0].permute(1, 0, 2)
    v = torch.randn(1, H_KV, n, D, generator=gen)[0].permute(1, 0, 2)
    for layer in range(2):
        pool.write_prefill(layer, table, 0, k.to(cuda), v.to(cuda))
    ref = np.zeros((8, bs, H_KV, D), np.float32)
    S.write_blocks(ref, table, 0, k.contiguous().numpy())
    for layer in range(2):
        assert np.array_equal(pool.keys[layer].cpu().numpy(), ref)
    for token, blk, off in case["token_to_block_offset"]:
        assert torch.equal(pool.keys[0][blk, off].cpu(), k[token])
        assert torch.equal(pool.values[0][blk, off].cpu(), v[token])
    for blk in case["untouched_blocks"]:
        assert not pool.keys[0][blk].any()


def test_chunked_append(cuda):
    case = KATS["chunked_append"]
    bs, table = case["block_size"], case["block_table"]
    pool = PagedPool(1, 8, bs, H_KV, D, device=cuda)
    chunks = [torch.randn(n, H_KV, D) for _, n in case["chunks"]]
    for (start, _), c in zip(case["chunks"], chunks):
        pool.write_prefill(0, table, start, c.to(cuda), (c * 2).to(cuda))
    total = sum(n for _, n in case["chunks"])
    got = S.gather_tokens(pool.keys[0].cpu().numpy(), table, total)
    assert np.array_equal(got, torch.cat(chunks).numpy())


def test_decode_container_write_matches_per_row_reference(cuda):
    case = KATS["decode_rows"]
    pool = PagedPool(1, 8, case["block_size"], H_KV, D, device=cuda, n_head=4)
    kv = PagedKV(pool, case["block_tables"], case["positions"], rope_len=64, n_head=4)
    k = torch.randn(2, H_KV, 1, D)
    v = torch.randn(2, H_KV, 1, D)
    kv.write(0, k.to(cuda), v.to(cuda))
    ref_k = np.zeros((8, case["block_size"], H_KV, D), np.float32)
    ref_v = np.zeros_like(ref_k)
    for row, (table, pos) in enumerate(zip(case["block_tables"], case["positions"])):
        S.write_tokens(ref_k, table, [pos], k[row:row + 1, :, 0].numpy())
        S.write_tokens(ref_v, table, [pos], v[row:row + 1, :, 0].numpy())
    assert np.array_equal(pool.keys[0].cpu().numpy(), ref_k)
    assert np.array_equal(pool.values[0].cpu().numpy(), ref_v)


def test_boundary_slot_and_rebuilt_container(cuda):
    case = KATS["decode_block_boundary"]
    pool = PagedPool(1, 8, 16, H_KV, D, device=cuda, n_head=4)
    kv = PagedKV(pool, [case["block_table"]], [case["position"]], rope_len=64, n_head=4)
    before = pool.keys[0].clone()
    k = torch.randn(1, H_KV, 1, D, device=cuda)
    kv.write(0, k, torch.randn_like(k))
    flat = pool.keys[0].view(-1, H_KV, D)
    assert torch.equal(flat[case["slot"]], k[0, :, 0])
    changed = (pool.keys[0] != before).any(-1).any(-1).view(-1).nonzero().view(-1).tolist()
    assert changed == [case["slot"]]
    for table, pos, slot in KATS["rebuilt_container"]["cases"]:
        kk = torch.randn(1, H_KV, 1, D, device=cuda)
        PagedKV(pool, [table], [pos], rope_len=64, n_head=4).write(0, kk, torch.zeros_like(kk))
        assert torch.equal(flat[slot], kk[0, :, 0])


def test_out_of_range_slot_is_skipped_and_reported(cuda):
    pool = PagedPool(1, 4, 16, H_KV, D, device=cuda)
    k = torch.randn(2, H_KV, D, device=cuda)
    pool.write_slots(0, torch.tensor([0, 10_000], device=cuda), k, k)
    assert torch.equal(pool.keys[0].view(-1, H_KV, D)[0], k[0])
    assert not pool.keys[0].view(-1, H_KV, D)[1:].any(), "nothing else was written"
    with pytest.raises(IndexError, match="token 1"):
        pool.check_writes()
    pool.check_writes()  # the error word was cleared
    strict = PagedPool(1, 4, 16, H_KV, D, device=cuda, strict_writes=True)
    with pytest.raises(IndexError):
        strict.write_slots(0, torch.tensor([-1, 3], device=cuda), k, k)


def test_write_past_the_block_table_raises_before_touching_the_pool(cuda):
    pool = PagedPool(1, 4, 16, H_KV, D, device=cuda, n_head=4)
    kv = PagedKV(pool, [[0]], [16], rope_len=32, n_head=4)
    before = pool.keys[0].clone()
    k = torch.randn(1, H_KV, 1, D, device=cuda)
    with pytest.raises(IndexError, match="block table has 1 blocks"):
        kv.write(0, k, k)
    assert torch.equal(pool.keys[0], before)


def test_config3_packed_group_write_is_bit_exact(cuda):
    """Config 3: 8 prompts through one packed slot-write launch per layer, equal to the
    per-request sink loop and to the numpy oracle."""
    inp = W.prefill_config3()
    pool_a = PagedPool(2, inp.n_blocks, inp.block_size, 8, 128, dtype=torch.bfloat16, device=cuda, n_head=16)
    pool_b = PagedPool(2, inp.n_blocks, inp.block_size, 8, 128, dtype=torch.bfloat16, device=cuda, n_head=16)
    sinks_a = [PagedWriteSink(pool_a, t, n) for t, n in zip(inp.tables, inp.lengths)]
    sinks_b = [PagedWriteSink(pool_b, t, n) for t, n in zip(inp.tables, inp.lengths)]
    positions = torch.cat([torch.arange(n) for n in inp.lengths]).to(cuda)
    packed = PackedPrefill(cu_seqlens=inp.cu_seqlens, positions=positions, sinks=sinks_a)
    assert packed.group_slots is not None
    k = inp.k.to(cuda).unsqueeze(0)
    v = inp.v.to(cuda).unsqueeze(0)
    for layer in range(2):
        packed.write(layer, k, v)
        start = 0
        for sink, end in zip(sinks_b, inp.cu_seqlens[1:]):
            sink.set_kv(layer, (k[0, start:end].transpose(0, 1).unsqueeze(0), v[0, start:end].transpose(0, 1).unsqueeze(0)))
            start = end
    for layer in range(2):
        assert torch.equal(pool_a.keys[layer], pool_b.keys[layer])
        assert torch.equal(pool_a.values[layer], pool_b.values[layer])
    got = pool_a.keys[1].view(-1, 8, 128)[inp.slots.to(cuda)].cpu()
    assert torch.equal(got, inp.k)
    with pytest.raises(RuntimeError, match="already written"):
        packed.write(0, k, v)
