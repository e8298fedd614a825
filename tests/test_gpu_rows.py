"""The decode-step rows GEMM (``mi_rows_gemm``, ``miattn.rows.rows_linear``) against a float64
product of the same bf16/fp16 operands, and the ops that consume its split-K partial sums
against the same ops fed the summed, rounded projection.

``nn.Linear`` rounds an fp32-accumulated dot product once to the activation dtype; the kernel
does the same with another fp32 summation order, so a plain output lies within one unit in
the last place of the exactly rounded product, and the fp32 partial sums, added in float64,
lie within fp32 accumulation error (K products) of the exact product. A consumer fed
:class:`Parts` sums them in split order and rounds once before its op chain, which
``Parts.value()`` restates in torch: the results are bit-identical.
"""

from __future__ import annotations

import pytest
import torch

from miattn import PagedPool
import torch.nn.functional as F

from miattn.qwen3 import (add_rms_norm, decode_step_begin, greedy_advance, greedy_advance_tiles, rms_norm,
                          rope_table, silu_mul)
from miattn.rows import Parts, argmax_rows, glu_weight, rows_linear, rows_supported, rows_swiglu, rows_tile_best

pytestmark = pytest.mark.gpu


def _operands(M, N, K, dtype, seed, lda=None):
    g = torch.Generator().manual_seed(seed)
    lda = lda or K
    a_full = torch.randn(M, lda, generator=g).to(dtype).cuda()
    w = (torch.randn(N, K, generator=g) * 0.05).to(dtype).cuda()
    return a_full[:, :K], w


@pytest.mark.parametrize(
    "M,N,K,n_split,dtype",
    [
        (32, 4096, 1024, None, torch.bfloat16),   # q/k/v (stacked) at the Qwen3-0.6B shape
        (32, 1024, 2048, None, torch.bfloat16),   # o_proj
        (32, 6144, 1024, None, torch.bfloat16),   # gate/up (stacked)
        (32, 1024, 3072, None, torch.bfloat16),   # down_proj
        (32, 8208, 1024, 1, torch.bfloat16),      # lm_head-like, N not a multiple of 32 tiles of 1024
        (5, 100, 1024, 1, torch.bfloat16),
        (17, 1000, 2048, 4, torch.float16),
        (1, 33, 256, 1, torch.bfloat16),
        (3, 64, 3072, 12, torch.bfloat16),
        (32, 4096, 1024, 1, torch.float16),
        (31, 96, 512, 2, torch.bfloat16),
    ],
)
def test_rows_gemm_matches_the_exact_product(M, N, K, n_split, dtype):
    a, w = _operands(M, N, K, dtype, seed=M * 131 + N + K)
    exact = a.double() @ w.double().t()
    got = rows_linear(a, w, n_split=n_split)
    torch.cuda.synchronize()
    scale = exact.abs().max().item()
    if isinstance(got, Parts):
        assert n_split != 1 and got.shape == (M, N) and got.dtype == dtype
        total = got.data.double().sum(0)
        assert (total - exact).abs().max().item() <= 1e-5 * scale
        got = got.value()
    assert got.shape == (M, N) and got.dtype == dtype
    # one ulp of the dtype at each element's magnitude (the exact product rounded once is
    # within half an ulp; the fp32 sum order moves it by far less than the other half)
    ulp = torch.finfo(dtype).eps * exact.abs().clamp(min=scale * 1e-3)
    assert ((got.double() - exact).abs() <= ulp).all()


def test_rows_gemm_row_strides_and_a_reused_output():
    a, w = _operands(8, 256, 1024, torch.bfloat16, seed=5, lda=1024 + 64)
    assert a.stride(0) == 1088
    want = rows_linear(a.contiguous(), w, n_split=1)
    for _ in range(2):
        got = rows_linear(a, w, n_split=1)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_rows_linear_rejects_what_it_does_not_take():
    w = torch.zeros(64, 1024, dtype=torch.bfloat16, device="cuda")
    for bad_a in (torch.zeros(33, 1024, dtype=torch.bfloat16, device="cuda"),
                  torch.zeros(4, 1000, dtype=torch.bfloat16, device="cuda"),
                  torch.zeros(4, 1024, dtype=torch.float32, device="cuda")):
        assert not rows_supported(bad_a, w)
        with pytest.raises(ValueError, match="rows_linear"):
            rows_linear(bad_a, w)
    with pytest.raises(ValueError, match="n_split"):
        rows_linear(torch.zeros(4, 1024, dtype=torch.bfloat16, device="cuda"), w, n_split=3)


def _parts(M, N, S, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return Parts((torch.randn(S, M, N, generator=g) * scale).cuda(), dtype)


@pytest.mark.parametrize("S", [2, 6])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_add_rms_norm_takes_partial_sums(S, dtype):
    g = torch.Generator().manual_seed(S)
    x = torch.randn(32, 1024, generator=g).to(dtype).cuda()
    w = (1.0 + 0.1 * torch.randn(1024, generator=g)).to(dtype).cuda()
    d = _parts(32, 1024, S, dtype, seed=S + 1)
    x1, h1 = add_rms_norm(x.clone(), d, w, 1e-6)
    x2, h2 = add_rms_norm(x.clone(), d.value(), w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(x1, x2) and torch.equal(h1, h2)


@pytest.mark.parametrize("S", [2, 4])
def test_silu_mul_takes_partial_sums(S):
    gu = _parts(32, 2 * 3072, S, torch.bfloat16, seed=7 + S, scale=2.0)
    got = silu_mul(gu)
    want = silu_mul(gu.value())
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("S", [1, 2])
@pytest.mark.parametrize("B,H,H_kv,D", [(32, 16, 8, 128), (5, 8, 2, 256)])
def test_epilogue_takes_partial_sums(S, B, H, H_kv, D):
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(B + D + S)
    qkv = _parts(B, (H + 2 * H_kv) * D, S, dtype, seed=B * D + S, scale=2.0)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype).cuda()
    kn = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype).cuda()
    cos, sin = rope_table(D, 1e6, 4096, "cuda", dtype)
    pos = torch.randint(0, 4096, (B,), generator=g).cuda()
    slots = torch.randperm(64 * 16, generator=g)[:B].cuda()
    pools = [PagedPool(1, 64, 16, H_kv, D, dtype=dtype, device="cuda", n_head=H, strict_writes=True)
             for _ in range(2)]
    q1 = pools[0].write_qk_norm_rope(0, slots, qkv, qn, kn, cos, sin, pos, 1e-6)
    q2 = pools[1].write_qk_norm_rope(0, slots, qkv.value(), qn, kn, cos, sin, pos, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(pools[0].keys[0], pools[1].keys[0])
    assert torch.equal(pools[0].values[0], pools[1].values[0])


@pytest.mark.parametrize("rows,cols,dtype", [(32, 151936, torch.bfloat16), (3, 1000, torch.float16),
                                             (5, 8193, torch.float32), (1, 7, torch.bfloat16)])
def test_argmax_rows_is_torch_argmax(rows, cols, dtype):
    g = torch.Generator().manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    # planted ties: two equal maxima (the first wins), a row of equal values, a NaN after a max
    x[0, cols // 3] = 100.0
    x[0, cols - 1] = 100.0
    if rows > 1:
        x[1] = 0.5
    if rows > 2:
        x[2, 0] = 50.0
        x[2, cols // 2] = float("nan")
        x[2, cols - 1] = float("nan")
    got = argmax_rows(x.cuda())
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), x.argmax(-1))


def test_argmax_rows_on_a_strided_view():
    x = torch.randn(4, 300, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    view = x.cuda()[:, 5:290]  # rows 600 bytes apart, not 16-byte aligned: the scalar walk
    assert torch.equal(argmax_rows(view).cpu(), x[:, 5:290].argmax(-1))


@pytest.mark.parametrize("M,inter,K,dtype", [(32, 3072, 1024, torch.bfloat16), (7, 48, 512, torch.float16),
                                             (1, 16, 256, torch.bfloat16)])
def test_swiglu_launch_equals_projection_then_silu_mul(M, inter, K, dtype):
    g = torch.Generator().manual_seed(M + inter)
    x = torch.randn(M, K, generator=g).to(dtype).cuda()
    wg = (torch.randn(inter, K, generator=g) * 0.05).to(dtype).cuda()
    wu = (torch.randn(inter, K, generator=g) * 0.05).to(dtype).cuda()
    got = rows_swiglu(x, glu_weight(wg, wu))
    # the same dot products through the plain launch, then the separate SiLU * up op
    want = silu_mul(rows_linear(x, torch.cat([wg, wu], 0), n_split=1))
    exact_g = (x.double() @ wg.double().t()).to(dtype)
    exact_u = (x.double() @ wu.double().t()).to(dtype)
    ref = F.silu(exact_g) * exact_u  # the reference's ops on correctly rounded projections
    torch.cuda.synchronize()
    assert got.shape == (M, inter) and got.dtype == dtype
    assert torch.equal(got, want)
    # within the projections' own rounding of the op chain on exactly rounded projections
    assert ((got.float() - ref.float()).abs() <= 0.02 * ref.float().abs() + 1e-3).all()



def test_decode_step_begin_matches_the_tensor_ops():
    g = torch.Generator().manual_seed(11)
    B, C, V, bs, mb = 6, 1024, 1000, 16, 9
    embed = torch.randn(V, C, generator=g).to(torch.bfloat16).cuda()
    w = (1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16).cuda()
    tokens = torch.randint(0, V, (B,), generator=g).cuda()
    pos = torch.randint(0, mb * bs, (B,), generator=g).cuda()
    table = torch.randperm(64, generator=g)[: B * mb].view(B, mb).to(torch.int32).cuda()
    seqlen = torch.zeros(B, dtype=torch.int32, device="cuda")
    slots = torch.zeros(B, dtype=torch.int64, device="cuda")
    x = torch.empty(B, C, dtype=torch.bfloat16, device="cuda")
    h = torch.empty_like(x)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    decode_step_begin(tokens, pos, table, bs, embed, w, 1e-6, seqlen, slots, x, h, err)
    torch.cuda.synchronize()
    assert err.item() == 0
    assert torch.equal(seqlen, (pos + 1).int())
    assert torch.equal(slots, table.long().gather(1, (pos // bs).view(-1, 1)).view(-1) * bs + pos % bs)
    assert torch.equal(x, embed[tokens])
    want = rms_norm(embed[tokens], w, 1e-6)
    assert (h == want).float().mean().item() > 0.999
    # an out-of-range token or position is reported and its row left alone
    tokens[2] = V
    pos[4] = mb * bs
    seqlen.zero_()
    decode_step_begin(tokens, pos, table, bs, embed, w, 1e-6, seqlen, slots, x, h, err)
    torch.cuda.synchronize()
    assert err.item() in (3, 5) and seqlen[2].item() == 0 and seqlen[4].item() == 0 and seqlen[0].item() > 0


def test_greedy_advance_updates_the_step_state():
    g = torch.Generator().manual_seed(12)
    B, V, max_new = 5, 3000, 3
    logits = torch.randn(B, V, generator=g).to(torch.bfloat16).cuda()
    tokens = torch.zeros(B, dtype=torch.int64, device="cuda")
    pos = torch.arange(B, dtype=torch.int64, device="cuda") * 10
    history = torch.full((B, max_new), -1, dtype=torch.int64, device="cuda")
    steps = torch.tensor([0, 1, 2, 3, 0], dtype=torch.int64, device="cuda")  # row 3 is past its history
    greedy_advance(logits, tokens, pos, history, steps)
    torch.cuda.synchronize()
    pick = logits.cpu().argmax(-1)
    assert torch.equal(tokens.cpu(), pick)
    assert torch.equal(pos.cpu(), torch.arange(B) * 10 + 1)
    assert torch.equal(steps.cpu(), torch.tensor([1, 2, 3, 4, 1]))
    h = history.cpu()
    assert h[0, 0] == pick[0] and h[1, 1] == pick[1] and h[2, 2] == pick[2] and h[4, 0] == pick[4]
    assert (h[3] == -1).all() and (h[0, 1:] == -1).all()


@pytest.mark.parametrize("M,N,K", [(32, 151936, 1024), (5, 1000, 512), (3, 70, 256)])
def test_lm_head_tile_picks_give_the_argmax_of_the_logits(M, N, K):
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).cuda()
    w[N // 2] = w[N // 3]  # identical weight rows: equal logits in two tiles, the lower column wins
    x[0] = w[N // 3].float().sign().to(torch.bfloat16)  # row 0's maximum is at that tie
    logits = rows_linear(x, w, n_split=1)
    out = torch.empty_like(logits)
    tiles = rows_tile_best(x, w, out)
    assert torch.equal(out, logits)  # the same products, stored when asked
    tiles_nolog = rows_tile_best(x, w)
    assert torch.equal(tiles, tiles_nolog)
    B = M
    tokens = torch.zeros(B, dtype=torch.int64, device="cuda")
    pos = torch.zeros(B, dtype=torch.int64, device="cuda")
    history = torch.zeros(B, 2, dtype=torch.int64, device="cuda")
    steps = torch.zeros(B, dtype=torch.int64, device="cuda")
    greedy_advance_tiles(tiles, tokens, pos, history, steps)
    torch.cuda.synchronize()
    want = logits.cpu().argmax(-1)
    assert torch.equal(tokens.cpu(), want) and torch.equal(history[:, 0].cpu(), want)
    # each tile's pick is its own first maximum
    t = tiles.cpu()
    vals = t[..., 0].view(torch.float32)
    lg = logits.float().cpu()
    for tile in (0, (N - 1) // 32):
        seg = lg[:, tile * 32:(tile + 1) * 32]
        assert torch.equal(t[:, tile, 1].long(), seg.argmax(-1) + tile * 32)
        assert torch.equal(vals[:, tile], seg.max(-1).values)


def test_tile_picks_follow_torch_on_ties_and_nan():
    # a weight matrix whose products hold exact ties and a NaN: x = e_0, so logits row r
    # are column 0 of w (rows of w scaled per output column)
    K, N = 256, 96
    w = torch.zeros(N, K)
    w[:, 0] = torch.tensor([float(c % 5) for c in range(N)])  # max 4.0 first at column 4, repeats
    w[70, 0] = 4.0
    x = torch.zeros(3, K)
    x[:, 0] = 1.0
    x[2, 0] = -1.0  # row 2: max 0.0 first at column 0
    wb, xb = w.to(torch.bfloat16).cuda(), x.to(torch.bfloat16).cuda()
    wn = wb.clone()
    wn[40, 0] = float("nan")  # a NaN product in tile 1 beats every number
    for weight, want in ((wb, [4, 4, 0]), (wn, [40, 40, 40])):
        tiles = rows_tile_best(xb, weight)
        tokens = torch.zeros(3, dtype=torch.int64, device="cuda")
        greedy_advance_tiles(tiles, tokens, torch.zeros_like(tokens), torch.zeros(3, 1, dtype=torch.int64,
                             device="cuda"), torch.zeros_like(tokens))
        torch.cuda.synchronize()
        assert tokens.cpu().tolist() == want
        assert torch.equal(tokens.cpu(), (xb.float() @ weight.float().t()).to(torch.bfloat16).cpu().argmax(-1))
