"""Host-side contracts of the drop-in modules on a CPU-only host: validation messages,
exception types and the no-fallback rule (reference tests/unit/test_triton_decode.py:
405-460, tests/unit/test_attention_varlen.py:343-428, tests/unit/test_paged_kv.py:
257-270,521-542, tests/unit/test_block_manager.py)."""

from __future__ import annotations

import pytest
import torch

import miattn
from miattn import BlockManager, HipVarlen, PackedPrefill, PagedKV, PagedPool, backend_for, paged_decode
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
        decode_mod._validate(*args)


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
    with pytest.raises(ValueError, match="no packed-prefill backend"):
        backend_for("cpu")
    with pytest.raises(ValueError, match="no packed-prefill backend"):
        backend_for("meta")


def test_pool_write_validation_and_no_cpu_write():
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
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pool.write_slots(0, slots, k, k)
    with pytest.raises(IndexError):
        pool.write_prefill(0, [0], 0, torch.randn(17, 2, 4), torch.randn(17, 2, 4))
    with pytest.raises(IndexError):
        pool.write_prefill(0, [pool.n_blocks], 0, k, k)
    with pytest.raises(ValueError):
        pool.write_prefill(0, [0], 0, k[:, :, :2], k)


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


def test_block_manager_contract():
    m = BlockManager(4, 16)
    assert m.reserve(2) == [0, 1]
    assert m.reserve(3) is None and m.in_use == 2
    assert m.reserve(0) == []
    with pytest.raises(ValueError, match="duplicate"):
        m.free([0, 0])
    with pytest.raises(ValueError, match="not allocated"):
        m.free([3])
    assert m.in_use == 2, "a refused free changes nothing"
    m.free([1])
    assert m.reserve(2) == [1, 2]
    assert m.peak == 3
    assert m.blocks_for(0, 0) == 1 and m.blocks_for(16, 0) == 1 and m.blocks_for(16, 1) == 2
    stats = m.stats()
    assert stats["alloc_calls"] == 2 and stats["free_calls"] == 1 and stats["free"] == 1
    with pytest.raises(ValueError):
        BlockManager(0, 16)
    with pytest.raises(ValueError):
        m.reserve(-1)


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
