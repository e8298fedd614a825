"""Host-side contracts of the drop-in modules on a CPU-only host: validation messages,
exception types, the device-type dispatch and the no-fallback rule for HIP entry points
(reference tests/unit/test_triton_decode.py:405-460, tests/unit/test_attention_varlen.py:
343-449, tests/unit/test_paged_kv.py:134-183,257-287,521-542,
tests/unit/test_packed_prefill.py:86-158). Host pools and the host prefill arm are
built and used on ``cpu`` the way the reference's own CPU tests build them."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

import miattn
from miattn import (HipVarlen, PackedPrefill, PagedKV, PagedPool, PagedWriteSink, SdpaVarlen, backend_for,
                    paged_decode)
from miattn import decode as decode_mod


def _inputs(H=4, H_kv=2, D=8, lengths=(17, 5)):
    B = len(lengths)
    q = torch.randn(B, H, D)
    k = torch.randn(4, 16, H_kv, D)
    v = torch.randn(4, 16, H_kv, D)
    table = torch.zeros(B, 2, dtype=torch.int32)
    return q, k, v, table, torch.tensor(lengths, dtype=torch.int32)


def test_paged_decode_never_falls_back_to_the_cpu():
    with pytest.raises(RuntimeError, match="CUDA"):
        paged_decode(*_inputs())


def test_paged_decode_raises_when_the_library_is_unavailable(monkeypatch):
    monkeypatch.setattr(decode_mod, "TRITON_AVAILABLE", False)
    with pytest.raises(RuntimeError, match="Triton"):
        decode_mod.paged_decode(*_inputs())


@pytest.mark.parametrize(
    "mutate,match",
    [
        (lambda a: (a[0][0], *a[1:]), "must be \\(B, H, D\\)"),
        (lambda a: (a[0], a[1].double(), a[2].double(), a[3], a[4]), "share one dtype"),
        (lambda a: (a[0], a[1], a[2], a[3].long(), a[4]), "int32"),
        (lambda a: (a[0], a[1], a[2], a[3], a[4].float()), "int32 or int64"),
        (lambda a: (a[0], a[1], a[2], a[3], torch.tensor([99, 1], dtype=torch.int32)), "capacity"),
        (lambda a: (a[0], a[1], a[2], a[3], torch.tensor([-1, 1], dtype=torch.int32)), ">= 0"),
        (lambda a: (a[0][:, :3], a[1], a[2], a[3], a[4]), "multiple of n_kv_head"),
        (lambda a: (a[0], a[1][:, :12].contiguous(), a[2][:, :12].contiguous(), a[3], a[4]), "power of two"),
        (lambda a: (a[0][..., :4], a[1], a[2], a[3], a[4]), "head_dim"),
    ],
)
def test_decode_validation_errors_are_value_errors(mutate, match):
    args = mutate(_inputs())
    with pytest.raises(ValueError, match=match):
        decode_mod._check(*args)


def test_varlen_validation_precedes_the_device_check():
    q = torch.randn(8, 8, 128).bfloat16()
    k = torch.randn(8, 4, 128).bfloat16()
    cases = [([1, 3, 8], 5, "must start at 0"), ([0, 5, 3, 8], 5, "strictly increasing"),
             ([0, 4, 7], 4, "must end at"), ([0, 4, 8], 5, "max_seqlen"), ([0, 4, 4, 8], 4, "strictly increasing"),
             ([0], 0, "needs n_seqs")]
    for cu, ms, match in cases:
        with pytest.raises(ValueError, match=match):
            HipVarlen().prefill_varlen(q, k, k, cu_seqlens=cu, max_seqlen=ms)
    with pytest.raises(ValueError, match="1-D"):
        HipVarlen().prefill_varlen(q, k, k, cu_seqlens=torch.tensor([[0, 8]]), max_seqlen=8)
    with pytest.raises(ValueError, match="integers"):
        HipVarlen().prefill_varlen(q, k, k, cu_seqlens=torch.tensor([0.0, 8.0]), max_seqlen=8)
    with pytest.raises(ValueError, match="3-D"):
        HipVarlen().prefill_varlen(q[None], k[None], k[None], cu_seqlens=[0, 8], max_seqlen=8)
    with pytest.raises(ValueError, match="multiple of n_kv_head"):
        HipVarlen().prefill_varlen(q, k[:, :3], k[:, :3], cu_seqlens=[0, 8], max_seqlen=8)
    with pytest.raises(ValueError, match="share head_dim"):
        HipVarlen().prefill_varlen(q, k[..., :64], k[..., :64], cu_seqlens=[0, 8], max_seqlen=8)
    with pytest.raises(ValueError, match="share one dtype"):
        HipVarlen().prefill_varlen(q, k.float(), k.float(), cu_seqlens=[0, 8], max_seqlen=8)
    with pytest.raises(ValueError, match="floating-point"):
        HipVarlen().prefill_varlen(q.int(), k.int(), k.int(), cu_seqlens=[0, 8], max_seqlen=8)
    # a valid call with CPU tensors is refused, never computed
    with pytest.raises(RuntimeError, match="CUDA"):
        HipVarlen().prefill_varlen(q, k, k, cu_seqlens=[0, 8], max_seqlen=8)


def test_backend_selection_is_by_device_type():
    assert isinstance(backend_for("cpu"), SdpaVarlen) and backend_for("cpu").name == "sdpa-varlen"
    assert isinstance(backend_for(torch.device("mps")), SdpaVarlen)
    with pytest.raises(ValueError, match="no packed-prefill backend"):
        backend_for("meta")
    assert miattn.FlashVarlen is HipVarlen


def test_host_pool_write_validation():
    pool = PagedPool(2, 4, 16, 2, 4, n_head=4)
    k = torch.randn(2, 2, 4)
    slots = torch.tensor([0, 1])
    with pytest.raises(ValueError, match="one entry per token"):
        pool.write_slots(0, slots[:1], k, k)
    with pytest.raises(ValueError, match="integer tensor"):
        pool.write_slots(0, slots.float(), k, k)
    with pytest.raises(ValueError, match="k/v shapes differ"):
        pool.write_slots(0, slots, k, k[:1])
    with pytest.raises(ValueError, match="head shape"):
        pool.write_slots(0, slots, k[:, :, :2], k[:, :, :2])
    with pytest.raises(IndexError, match="outside the pool's"):
        pool.write_slots(2, slots, k, k)
    with pytest.raises((IndexError, RuntimeError)):
        pool.write_slots(0, torch.tensor([0, 10_000]), k, k)
    with pytest.raises(IndexError):
        pool.write_prefill(0, [0], 0, torch.randn(17, 2, 4), torch.randn(17, 2, 4))
    with pytest.raises(IndexError):
        pool.write_prefill(0, [pool.n_blocks], 0, k, k)
    with pytest.raises(ValueError):
        pool.write_prefill(0, [0], 0, k[:, :, :2], k)
    pool.check_writes()  # host pools raise at the write; nothing pending


def test_host_pool_writes_the_reference_known_answers():
    """Slots of the reference's shuffled-table and block-boundary cases on a host pool
    (tests/golden/slot_kats.json; reference tests/unit/test_paged_kv.py:134-158,464-478)."""
    kats = json.loads((Path(__file__).parent / "golden" / "slot_kats.json").read_text())
    case = kats["prefill_shuffled_table"]
    bs, table = case["block_size"], case["block_table"]
    pool = PagedPool(1, 8, bs, 2, 4)
    k = torch.randn(case["length"], 2, 4)
    v = torch.randn(case["length"], 2, 4)
    pool.write_prefill(0, table, case["start"], k, v)
    for t, block, offset in case["token_to_block_offset"]:
        assert torch.equal(pool.keys[0][block, offset], k[t]) and torch.equal(pool.values[0][block, offset], v[t])
    for block in case["untouched_blocks"]:
        assert not pool.keys[0][block].any() and not pool.values[0][block].any()
    edge = kats["decode_block_boundary"]
    slots = PagedPool(1, 8, edge["block_size"], 2, 4).slot_ids(edge["block_table"], edge["position"], 1)
    assert slots.tolist() == [edge["slot"]]
    # int32 slot ids are accepted, as int64 are; the pool's flat view receives every row
    pool.write_slots(0, torch.tensor([3, 17], dtype=torch.int32), k[:2], v[:2])
    flat = pool.keys[0].view(-1, 2, 4)
    assert torch.equal(flat[3], k[0]) and torch.equal(flat[17], k[1])


def test_host_chunked_append_continues_a_request():
    """A second chunk from start=21 lands after the first (reference
    tests/unit/test_paged_kv.py:161-183)."""
    pool = PagedPool(1, 6, 16, 2, 4)
    table = [4, 1, 3]
    first, second = torch.randn(21, 2, 4), torch.randn(19, 2, 4)
    pool.write_prefill(0, table, 0, first, first)
    pool.write_prefill(0, table, 21, second, second)
    whole = torch.cat([first, second])
    logical = pool.keys[0][torch.tensor(table)].reshape(-1, 2, 4)[:40]
    assert torch.equal(logical, whole)


def test_sdpa_arm_matches_the_longhand_oracle_and_isolates_segments():
    from oracle.varlen import longhand_varlen

    gen = torch.Generator().manual_seed(3)
    cu = [0, 5, 6, 30]
    q = torch.randn(30, 4, 16, generator=gen)
    k = torch.randn(30, 2, 16, generator=gen)
    v = torch.randn(30, 2, 16, generator=gen)
    out = SdpaVarlen().prefill_varlen(q, k, v, cu_seqlens=cu, max_seqlen=24)
    assert (out - longhand_varlen(q, k, v, cu)).abs().max().item() < 1e-5
    k2 = k.clone()
    k2[:5] += 1.0  # segment 0 only
    out2 = SdpaVarlen().prefill_varlen(q, k2, v, cu_seqlens=torch.tensor(cu), max_seqlen=24)
    assert torch.equal(out2[5:], out[5:])
    with pytest.raises(ValueError, match="max_seqlen"):
        SdpaVarlen().prefill_varlen(q, k, v, cu_seqlens=cu, max_seqlen=23)


def test_packed_prefill_on_the_host_writes_through_paged_sinks():
    """PackedPrefill on cpu picks the SDPA arm and writes each request through its sink
    (reference tests/unit/test_packed_prefill.py:86-126)."""
    pool = PagedPool(2, 8, 16, 2, 8, n_head=4)
    lengths, tables = [5, 20], [[6], [2, 0]]
    sinks = [PagedWriteSink(pool, t, n) for t, n in zip(tables, lengths)]
    packed = PackedPrefill(cu_seqlens=[0, 5, 25], positions=torch.tensor(list(range(5)) + list(range(20))),
                           sinks=sinks)
    assert packed.backend_name == "sdpa-varlen" and packed.group_slots is not None
    k = torch.randn(1, 25, 2, 8)
    v = torch.randn(1, 25, 2, 8)
    packed.write(1, k, v)
    assert torch.equal(pool.keys[1][6, :5], k[0, :5])
    assert torch.equal(pool.keys[1][2], k[0, 5:21]) and torch.equal(pool.values[1][0, :4], v[0, 21:])
    with pytest.raises(RuntimeError, match="already written"):
        packed.write(1, k, v)
    q = torch.randn(1, 25, 4, 8)
    y = packed.attend(q, k, v)
    assert y.shape == (1, 25, 4, 8)


def test_paged_kv_rejects_a_cpu_pool():
    pool = PagedPool(1, 4, 16, 2, 4)
    with pytest.raises(ValueError, match="CUDA"):
        PagedKV(pool, [[0]], [3], rope_len=16)


def test_packed_prefill_validation():
    pos = torch.arange(4)
    with pytest.raises(ValueError, match="start at 0"):
        PackedPrefill(cu_seqlens=[1, 4], positions=pos, sinks=[object()], backend=object())
    with pytest.raises(ValueError, match="strictly increasing"):
        PackedPrefill(cu_seqlens=[0, 2, 2, 4], positions=pos, sinks=[object()] * 3, backend=object())
    with pytest.raises(ValueError, match="one sink per request"):
        PackedPrefill(cu_seqlens=[0, 4], positions=pos, sinks=[], backend=object())
    with pytest.raises(ValueError, match="request-local"):
        PackedPrefill(cu_seqlens=[0, 2, 4], positions=pos, sinks=[object()] * 2, backend=object())
    p = PackedPrefill(cu_seqlens=[0, 2, 4], positions=torch.tensor([0, 1, 0, 1]), sinks=[object()] * 2,
                      backend=object())
    assert p.max_seqlen == 2 and p.last_token_index.tolist() == [1, 3] and p.n_seqs == 2


def test_availability_flag_is_exported():
    assert miattn.TRITON_AVAILABLE is miattn.HIP_AVAILABLE


# ---------------------------------------------------------------- decode-step host helpers
def test_glu_weight_interleaves_gate_and_up_rows_by_16():
    from miattn.rows import glu_weight

    wg = torch.arange(48 * 4, dtype=torch.float32).view(48, 4)
    wu = -wg - 1
    w = glu_weight(wg, wu)
    assert w.shape == (96, 4)
    for t in range(3):
        assert torch.equal(w[32 * t:32 * t + 16], wg[16 * t:16 * t + 16])
        assert torch.equal(w[32 * t + 16:32 * t + 32], wu[16 * t:16 * t + 16])
    with pytest.raises(ValueError, match="inter % 16"):
        glu_weight(wg[:40], wu[:40])


def test_parts_hold_split_partials_and_sum_them_in_order():
    from miattn.rows import Parts

    data = torch.tensor([[[1e8, 1.0]], [[-1e8, 1.0]], [[1.0, 1.0]]], dtype=torch.float32)
    p = Parts(data, torch.bfloat16)
    assert p.shape == (1, 2) and p.n_parts == 3
    # split order: (1e8 + -1e8) + 1 = 1 exactly, where another order could lose the 1
    assert torch.equal(p.value(), torch.tensor([[1.0, 3.0]], dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="fp32"):
        Parts(data.double(), torch.bfloat16)


def test_rows_gemm_takes_only_device_tensors_of_its_shapes():
    from miattn.rows import rows_supported

    x = torch.zeros(4, 1024, dtype=torch.bfloat16)
    w = torch.zeros(64, 1024, dtype=torch.bfloat16)
    assert not rows_supported(x, w)  # host tensors: the product path is the HIP launch only
