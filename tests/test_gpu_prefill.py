"""Packed varlen prefill on the HIP MFMA kernel vs the CPU oracles (the reference's
varlen tests, reference tests/unit/test_attention_varlen.py:122-544, against this build).

Bars: bf16/fp16 max|delta| <= 2e-2 against the fp32 longhand oracle on the small cases, a
per-element bound derived from the kernels' rounding on config 3 at full size; bitwise packing
invariance and segment isolation (the kernel's per-tile arithmetic does not depend on the
other segments of the pack). Every case runs on the library's default kernel choice and
on each kernel it can be asked for (``HipVarlen(kernel="ring" | "staged" | "duo" | "tall")``).
"""

from __future__ import annotations

import functools

import pytest
import torch

from miattn import HipVarlen, _lib, backend_for
from miattn import workloads as W
from miattn.varlen import check_prefill_errors
from oracle.varlen import UNIT_ROUNDOFF, longhand_varlen, varlen_error_bound

pytestmark = pytest.mark.gpu

LENGTH_SETS = [
    pytest.param([1], id="1seg-len1"),
    pytest.param([17], id="1seg-len17"),
    pytest.param([128], id="1seg-len128"),
    pytest.param([1517], id="1seg-len1517"),
    pytest.param([1, 17], id="2seg-1-17"),
    pytest.param([128, 1517], id="2seg-128-1517"),
    pytest.param([1, 17, 128, 1517], id="4seg"),
    pytest.param([1, 1, 17, 128, 1517, 3, 64, 200], id="8seg-mixed"),
]


def _packed(lengths, H, H_kv, D, *, dtype=torch.bfloat16, seed=0):
    gen = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    q = torch.randn(T, H, D, generator=gen).to(dtype)
    k = torch.randn(T, H_kv, D, generator=gen).to(dtype)
    v = torch.randn(T, H_kv, D, generator=gen).to(dtype)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return q, k, v, cu, max(lengths)


KERNELS = [pytest.param(None, id="default"), pytest.param("ring", id="ring"), pytest.param("staged", id="staged"),
           pytest.param("duo", id="duo"), pytest.param("tall", id="tall")]


def _run(q, k, v, cu, max_seqlen, dev, kernel=None, **kw):
    out = HipVarlen(kernel).prefill_varlen(q.to(dev), k.to(dev), v.to(dev), cu_seqlens=cu, max_seqlen=max_seqlen,
                                           **kw)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("H,H_kv", [(8, 4), (8, 1), (16, 8)], ids=["gqa2", "gqa8", "qwen3"])
@pytest.mark.parametrize("lengths", LENGTH_SETS)
def test_matches_the_per_segment_oracle(lengths, H, H_kv, kernel, cuda):
    q, k, v, cu, ms = _packed(lengths, H, H_kv, 128)
    out = _run(q, k, v, cu, ms, cuda, kernel)
    ref = longhand_varlen(q, k, v, cu)
    assert out.shape == (sum(lengths), H, 128) and out.dtype == torch.bfloat16
    assert torch.isfinite(out).all()
    assert (out.float() - ref).abs().max().item() <= 2e-2


@pytest.mark.parametrize("D,kernel", [(64, None), (64, "ring"), (64, "staged"), (64, "duo"), (64, "tall"),
                                      (128, None), (128, "ring"), (128, "staged"), (128, "duo"), (128, "tall"),
                                      (256, None), (256, "staged"), (256, "duo")])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_head_dims_and_dtypes(D, kernel, dtype, cuda):
    q, k, v, cu, ms = _packed([1, 33, 128, 300], 8, 4, D, dtype=dtype, seed=2)
    out = _run(q, k, v, cu, ms, cuda, kernel)
    assert out.dtype == dtype
    assert (out.float() - longhand_varlen(q, k, v, cu)).abs().max().item() <= 2e-2


@pytest.mark.parametrize("kernel", [pytest.param(None, id="default"), pytest.param("ring", id="ring"),
                                    pytest.param("duo", id="duo"), pytest.param("tall", id="tall")])
@pytest.mark.parametrize("lengths,H,H_kv,D,dtype", [
    pytest.param([2100], 8, 4, 128, torch.bfloat16, id="split-2100-gqa2"),
    pytest.param([2100], 2, 1, 128, torch.bfloat16, id="split-2100-h2"),
    pytest.param([1, 17, 2048, 300], 16, 8, 128, torch.bfloat16, id="qwen3-4seg"),
    pytest.param([2049, 33], 8, 1, 64, torch.float16, id="d64-fp16-gqa8"),
    pytest.param([4500], 4, 2, 128, torch.bfloat16, id="split-4500-4way"),
])
def test_long_segments_and_split_pieces(lengths, H, H_kv, D, dtype, kernel, cuda):
    """Long segments; when the launch underfills the chip the longest tiles' key ranges
    are split into pieces whose partials a second launch merges."""
    q, k, v, cu, ms = _packed(lengths, H, H_kv, D, dtype=dtype, seed=7)
    out = _run(q, k, v, cu, ms, cuda, kernel)
    assert out.dtype == dtype and torch.isfinite(out).all()
    assert (out.float() - longhand_varlen(q, k, v, cu)).abs().max().item() <= 2e-2


@pytest.mark.parametrize("kernel", [pytest.param(None, id="default"), pytest.param("duo", id="duo"),
                                    pytest.param("staged", id="staged")])
@pytest.mark.parametrize("lengths", [pytest.param([1500], id="split-1500"), pytest.param([900, 3], id="split-900")])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "non-causal"])
def test_head_dim_256_split_pieces(lengths, causal, kernel, cuda):
    """Head_dim 256 on a launch too small to fill the chip (H 8 / H_kv 2): the schedule
    splits the longest tiles' key ranges and the merge launch folds the pieces. Without the
    causal mask every tile runs the whole key range, so the last tiles are split too and
    no step is a diagonal one."""
    q, k, v, cu, ms = _packed(lengths, 8, 2, 256, seed=13)
    out = _run(q, k, v, cu, ms, cuda, kernel, causal=causal)
    assert torch.isfinite(out).all()
    assert (out.float() - longhand_varlen(q, k, v, cu, causal=causal)).abs().max().item() <= 2e-2


@pytest.mark.parametrize("D", [128, 256])
def test_default_kernel_past_255_heads(D, cuda):
    """256 query heads (beyond the duo kernel's item word): the default schedule runs the
    ring kernel at head_dim 128 and the register-staged kernel at 256."""
    q, k, v, cu, ms = _packed([70, 5, 130], 256, 8, D, seed=17)
    out = _run(q, k, v, cu, ms, cuda)
    assert (out.float() - longhand_varlen(q, k, v, cu)).abs().max().item() <= 2e-2


@pytest.mark.parametrize("kernel", KERNELS)
def test_many_short_segments(kernel, cuda):
    """150 short segments (1-89 tokens) in one pack: every tile of every segment gets its
    own schedule entry, and no query sees another segment's keys."""
    gen = torch.Generator().manual_seed(71)
    lengths = torch.randint(1, 90, (150,), generator=gen).tolist()
    q, k, v, cu, ms = _packed(lengths, 8, 4, 128, seed=11)
    out = _run(q, k, v, cu, ms, cuda, kernel)
    assert (out.float() - longhand_varlen(q, k, v, cu)).abs().max().item() <= 2e-2


@pytest.mark.parametrize("kernel", KERNELS)
def test_long_non_causal(kernel, cuda):
    q, k, v, cu, ms = _packed([2050, 70], 8, 4, 128, seed=8)
    out = _run(q, k, v, cu, ms, cuda, kernel, causal=False)
    assert (out.float() - longhand_varlen(q, k, v, cu, causal=False)).abs().max().item() <= 2e-2


@pytest.mark.parametrize("kernel", KERNELS)
def test_non_causal_and_custom_scale(kernel, cuda):
    q, k, v, cu, ms = _packed([17, 64, 200], 8, 1, 128, seed=4)
    out = _run(q, k, v, cu, ms, cuda, kernel, causal=False)
    assert (out.float() - longhand_varlen(q, k, v, cu, causal=False)).abs().max().item() <= 2e-2
    out = _run(q, k, v, cu, ms, cuda, kernel, softmax_scale=0.37)
    assert (out.float() - longhand_varlen(q, k, v, cu, scale=0.37)).abs().max().item() <= 2e-2


@pytest.mark.parametrize("kernel", KERNELS)
def test_packed_equals_one_at_a_time_bitwise(kernel, cuda):
    lengths = [17, 1, 128, 333]
    q, k, v, cu, ms = _packed(lengths, 16, 8, 128, seed=3)
    packed = _run(q, k, v, cu, ms, cuda, kernel)
    single = torch.cat([_run(q[s:e], k[s:e], v[s:e], [0, e - s], e - s, cuda, kernel) for s, e in zip(cu, cu[1:])])
    if kernel == "tall":
        # the tall schedule's split cap depends on the whole batch, so a packed and a
        # one-segment launch may cut a tile's key range differently: the pieces' fp32 sums
        # then differ in order, which moves an output by at most one ulp (a slice or offset
        # bug moves it by far more); tiles that neither launch splits stay bitwise
        ulp = torch.maximum(packed.float().abs(), single.float().abs()) * 2.0 ** -8
        assert ((packed.float() - single.float()).abs() <= ulp + 1e-6).all()
    else:
        assert torch.equal(packed, single)


@pytest.mark.parametrize("kernel", KERNELS)
def test_changing_segment_zero_leaves_the_others_bitwise(kernel, cuda):
    lengths = [17, 1, 128]
    q, k, v, cu, ms = _packed(lengths, 8, 4, 128, seed=5)
    before = _run(q, k, v, cu, ms, cuda, kernel)
    gen = torch.Generator().manual_seed(99)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[:17] = torch.randn(17, 8, 128, generator=gen).bfloat16()
    k2[:17] = torch.randn(17, 4, 128, generator=gen).bfloat16()
    v2[:17] = torch.randn(17, 4, 128, generator=gen).bfloat16()
    after = _run(q2, k2, v2, cu, ms, cuda, kernel)
    assert not torch.equal(after[:17], before[:17])
    assert torch.equal(after[17:], before[17:])


# Config 3 at full size against a per-element bound derived from the kernels' arithmetic
# (oracle.varlen.varlen_error_bound): output rounding u|o|, the probabilities rounded to the
# input dtype before the PV MFMA (u times the probability-weighted |v| or spread of v), and
# fp32 slack, with u = 2^-8 (bf16) or 2^-11 (fp16), the unit roundoff of round-to-nearest
# into an 8- or 11-bit significand. A 16-bit-P emulation reaches 0.6-0.7 of it; P rounded to
# 6 bits, a 1% scale error or a dropped key exceed it (tests/test_oracle_varlen.py). fp16
# also keeps the north-star bar: <= 1e-3 beyond the output's own rounding.
FP16_EXCESS_BAR = 1e-3


@functools.lru_cache(maxsize=2)
def _config3(dtype, H, H_kv, D):
    inp = W.prefill_config3(H=H, H_kv=H_kv, D=D, dtype=dtype)
    ref, bound = varlen_error_bound(inp.q, inp.k, inp.v, inp.cu_seqlens)
    return inp, ref, bound


def _check_config3(kernel, dtype, H, H_kv, D, cuda):
    inp, ref, bound = _config3(dtype, H, H_kv, D)
    out = _run(inp.q, inp.k, inp.v, inp.cu_seqlens, max(inp.lengths), cuda, kernel).float()
    err = (out - ref).abs()
    ratio = (err / bound).max().item()
    print(f"config 3 H{H}/{H_kv} D{D} ({kernel}, {dtype}): max|delta| {err.max().item():.3e}, "
          f"max |delta|/bound {ratio:.3f}")
    assert torch.isfinite(out).all()
    assert (err <= bound).all(), f"{int((err > bound).sum())} elements beyond the derived bound (max ratio {ratio:.3f})"
    if dtype == torch.float16:
        assert (err - ref.abs() * UNIT_ROUNDOFF[dtype]).max().item() <= FP16_EXCESS_BAR


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("kernel", KERNELS)
def test_config3_full_size(kernel, dtype, cuda):
    _check_config3(kernel, dtype, 16, 8, 128, cuda)


@pytest.mark.parametrize("kernel", [pytest.param(None, id="default"), pytest.param("duo", id="duo"),
                                    pytest.param("staged", id="staged")])
def test_config3_qwen35_shape(kernel, cuda):
    """Config 3's lengths at the Qwen3.5 attention shape (H 8 / H_kv 2 / head_dim 256), on
    every kernel that takes head_dim 256 (the default there is the duo kernel at one
    workgroup per CU)."""
    _check_config3(kernel, torch.bfloat16, 8, 2, 256, cuda)


def test_error_surface(cuda):
    q, k, v, cu, ms = _packed([4, 4], 8, 4, 128, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="fp16/bf16"):
        HipVarlen().prefill_varlen(q.to(cuda), k.to(cuda), v.to(cuda), cu_seqlens=cu, max_seqlen=ms)
    qb, kb, vb = q.bfloat16(), k.bfloat16(), v.bfloat16()
    with pytest.raises(RuntimeError, match="CUDA"):
        HipVarlen().prefill_varlen(qb, kb, vb, cu_seqlens=cu, max_seqlen=ms)
    for bad_cu, bad_ms, match in (([1, 3, 8], 5, "must start at 0"), ([0, 5, 3, 8], 5, "strictly increasing"),
                                  ([0, 4, 7], 4, "must end at"), ([0, 4, 8], 5, "max_seqlen")):
        with pytest.raises(ValueError, match=match):
            HipVarlen().prefill_varlen(qb.to(cuda), kb.to(cuda), vb.to(cuda), cu_seqlens=bad_cu, max_seqlen=bad_ms)
    with pytest.raises(ValueError, match="unknown prefill kernel"):
        HipVarlen("fast")
    with pytest.raises(ValueError, match="head_dim 64 or 128"):
        q256 = torch.zeros(8, 8, 256, dtype=torch.bfloat16, device=cuda)
        k256 = torch.zeros(8, 4, 256, dtype=torch.bfloat16, device=cuda)
        HipVarlen("ring").prefill_varlen(q256, k256, k256, cu_seqlens=[0, 8], max_seqlen=8)
    assert backend_for("cuda").name == "hip-mfma-varlen"
    assert isinstance(backend_for(torch.device("cuda:0")), HipVarlen)


@pytest.mark.parametrize("lengths,H,H_kv", [
    pytest.param([1742, 110, 658, 364, 390, 450, 152, 445], 16, 8, id="config3-per-xcd-lists"),
    pytest.param([300, 47, 1000], 8, 2, id="one-list"),
])
@pytest.mark.parametrize("kernel", ["duo", "tall"])
def test_persistent_kernels_are_stable_across_calls_and_graph_replays(lengths, H, H_kv, kernel, cuda):
    """The persistent kernels' workgroups each work through a list of items with the next
    item's loads in flight during the current one's epilogue (and, in the tall kernel, split
    pieces merged through counters that every launch must leave at zero): every call must
    compute every item (outputs match the oracle) and give the same bits call after call,
    eager and replayed from a HIP graph."""
    q, k, v, cu, ms = _packed(lengths, H, H_kv, 128, seed=11)
    qd, kd, vd = q.to(cuda), k.to(cuda), v.to(cuda)
    be = HipVarlen(kernel, strict=True)
    first = be.prefill_varlen(qd, kd, vd, cu_seqlens=cu, max_seqlen=ms)
    torch.cuda.synchronize()
    assert (first.float().cpu() - longhand_varlen(q, k, v, cu)).abs().max().item() <= 2e-2
    for _ in range(3):
        again = be.prefill_varlen(qd, kd, vd, cu_seqlens=cu, max_seqlen=ms)
        torch.cuda.synchronize()
        assert torch.equal(again, first)
    stream = torch.cuda.Stream()
    outs = []
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(2):
                outs.append(be.prefill_varlen(qd, kd, vd, cu_seqlens=cu, max_seqlen=ms))
    for _ in range(3):
        for o in outs:
            o.zero_()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(o, first) for o in outs)


@pytest.mark.parametrize("kernel,D,H,H_kv,lengths,code", [
    pytest.param("tall", 128, 16, 8, [1742, 110, 658], 1, id="tall-owner-wait"),
    pytest.param("duo", 256, 8, 2, [700, 90], 2, id="duo256-pair-wait"),
])
def test_a_bounded_wait_that_gives_up_is_reported(kernel, D, H, H_kv, lengths, code, cuda):
    """The kernels' bounded waits (a tall owner for its producer pieces, a head_dim 256 duo
    wave for its partner) are forced to give up at once from the host (wait limit 0): the
    launch still ends normally, the error word carries the kernel's code, and
    check_prefill_errors raises. With the limit restored the same call is correct again
    (the tall counters are back at zero)."""
    q, k, v, cu, ms = _packed(lengths, H, H_kv, D, seed=21)
    qd, kd, vd = q.to(cuda), k.to(cuda), v.to(cuda)
    be = HipVarlen(kernel)
    check_prefill_errors(cuda)  # nothing pending
    previous = _lib.lib.mi_prefill_wait_limit(0)
    try:
        be.prefill_varlen(qd, kd, vd, cu_seqlens=cu, max_seqlen=ms)
        torch.cuda.synchronize()
    finally:
        _lib.lib.mi_prefill_wait_limit(previous)
    with pytest.raises(RuntimeError, match="gave up waiting"):
        check_prefill_errors(cuda)
    check_prefill_errors(cuda)  # cleared by the raise
    out = be.prefill_varlen(qd, kd, vd, cu_seqlens=cu, max_seqlen=ms)
    torch.cuda.synchronize()
    check_prefill_errors(cuda)
    assert (out.float().cpu() - longhand_varlen(q, k, v, cu)).abs().max().item() <= 2e-2
