"""The C-ABI library loads on a CPU-only host and exports every function the header
declares; host-only entry points (the prefill tile scheduler) are checked here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

import miattn
from miattn import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "miattn.h"


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_without_a_gpu():
    assert miattn.HIP_AVAILABLE, miattn.LOAD_ERROR
    assert _lib.lib.mi_abi_version() == _lib.ABI_VERSION


def test_every_declared_function_is_exported_and_bound():
    declared = _declared_functions()
    assert len(declared) >= 7
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared:
        assert hasattr(handle, name), f"{name} declared in miattn.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes binding"


def test_error_channel_reports_the_last_failure():
    strides = _lib.int64_array([0] * 15)
    rc = _lib.lib.mi_paged_decode(None, None, None, None, None, None, 1, 3, 2, 128, 16, 4, strides,
                                  1.0, 2, None, 0, None)
    assert rc == _lib.MI_ERR_INVALID
    assert "multiple of n_kv_head" in _lib.last_error()
    with pytest.raises(ValueError, match="multiple of n_kv_head"):
        _lib.check(rc, "probe")


KERNELS = {"staged": 0, "ring": 1, "duo": 3}
ROWS = {0: 64, 1: 128, 3: 64}   # query rows per tile
KEYS = {0: 64, 1: 64, 3: 64}    # keys per unit of a tile's work
PER_CU = {0: 2, 1: 1, 3: 2}     # workgroups one CU runs at once


def _kind(kernel, D, lengths=()):
    if kernel is None:  # head_dim 64/128: ring from an 8192-token segment, duo below; 256: duo
        if D in (64, 128):
            return 1 if max(lengths) >= 8192 else 3
        return 3 if D == 256 else 0
    return KERNELS[kernel]


def _schedule(lengths, H=16, H_kv=8, D=128, causal=1, kernel=None):
    """(header, work pieces, merges) of mi_varlen_schedule_for: pieces are (seq, tile,
    split, n_split, slot), merges (seq, tile, n_split, slot)."""
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    host_cu = (ctypes.c_int32 * len(cu))(*cu)
    code = -1 if kernel is None else KERNELS[kernel]
    words = _lib.lib.mi_varlen_schedule_for(host_cu, len(lengths), H, H_kv, D, causal, code, None, 0)
    out = (ctypes.c_int32 * words)()
    assert _lib.lib.mi_varlen_schedule_for(host_cu, len(lengths), H, H_kv, D, causal, code, out, words) == words
    if kernel is None:  # the default entry point makes the same schedule
        same = (ctypes.c_int32 * words)()
        assert _lib.lib.mi_varlen_schedule(host_cu, len(lengths), H, H_kv, D, causal, same, words) == words
        assert list(same) == list(out)
    n_work, n_merge, n_partials, layout = out[0], out[1], out[2], out[3]
    kind = _kind(kernel, D, lengths)
    rows = ROWS[kind]
    if kind == 3:
        return _duo_schedule(out, words, lengths, cu, H, H_kv, D)
    assert layout == (kind << 20) | (D << 8) | rows and words == 4 + 2 * (n_work + n_merge)
    w = [out[i] & 0xFFFFFFFF for i in range(4, words)]
    pieces = [(w[2 * i] >> 16, w[2 * i] & 0xFFFF, w[2 * i + 1] >> 28, ((w[2 * i + 1] >> 24) & 15) + 1,
               w[2 * i + 1] & 0xFFFFFF) for i in range(n_work)]
    merges = [(w[2 * i] >> 16, w[2 * i] & 0xFFFF, w[2 * i + 1] >> 24, w[2 * i + 1] & 0xFFFFFF)
              for i in range(n_work, n_work + n_merge)]
    ws = _lib.lib.mi_varlen_workspace_size(out, H)
    assert ws == n_partials * H * rows * (D + 2) * 4
    return (n_work, n_merge, n_partials), pieces, merges


def _duo_schedule(out, words, lengths, cu, H, H_kv, D):
    """Parse and check the persistent duo kernel's schedule: {n_wg, n_merge, n_partials,
    layout}, n_wg 8-word entries {first item word, count, the first item's 4 words, 0, 0},
    the merges, then 4-word items {seq0, L, tile << 16 | split << 8 | n_split - 1,
    head << 24 | slot}. Returns the pieces of head 0 in the common (seq, tile, split,
    n_split, slot) form, after checking every head has the same pieces."""
    n_wg, n_merge, n_partials, layout = out[0], out[1], out[2], out[3]
    assert layout == (3 << 20) | (D << 8) | 64 and 1 <= n_wg <= 512
    u = [out[i] & 0xFFFFFFFF for i in range(words)]
    mb = 4 + 8 * n_wg
    merges = [(u[mb + 2 * i] >> 16, u[mb + 2 * i] & 0xFFFF, u[mb + 1 + 2 * i] >> 24, u[mb + 1 + 2 * i] & 0xFFFFFF)
              for i in range(n_merge)]
    item_base = mb + 2 * n_merge
    seq_of = {c: i for i, c in enumerate(cu[:-1])}
    per_head = {h: [] for h in range(H)}
    seen_words = 0
    for wg in range(n_wg):
        entry = out[4 + 8 * wg: 12 + 8 * wg]
        first, count = entry[0], entry[1]
        assert first == item_base + seen_words and count >= 1
        assert list(entry[2:6]) == list(out[first:first + 4]) and list(entry[6:]) == [0, 0]  # item 0 inline
        costs = []
        for i in range(count):
            seq0, L, w2, w3 = (u[first + 4 * i + j] for j in range(4))
            seq = seq_of[seq0]
            assert lengths[seq] == L
            tile, split, ns, h, slot = w2 >> 16, (w2 >> 8) & 0xFF, (w2 & 0xFF) + 1, w3 >> 24, w3 & 0xFFFFFF
            per_head[h].append((seq, tile, split, ns, slot))
            if n_wg == 256 * (1 if D == 256 else 2) and H_kv % 8 == 0:  # a KV head's items stay on one XCD
                assert (h // (H // H_kv)) % 8 == wg % 8
            elif n_wg == 256 * (1 if D == 256 else 2) and 8 % H_kv == 0:  # ... on its block of 8 / H_kv XCDs
                assert h // (H // H_kv) == (wg % 8) // (8 // H_kv)
            costs.append(_piece_work(lengths, (seq, tile, split, ns, slot), 3))
        assert costs == sorted(costs, reverse=True)  # longest first within a workgroup
        seen_words += 4 * count
    assert item_base + seen_words == words
    pieces = sorted(per_head[0])
    assert all(sorted(per_head[h]) == pieces for h in range(H))
    ws = _lib.lib.mi_varlen_workspace_size(out, H)
    assert ws == n_partials * H * 64 * (D + 2) * 4
    # in the common form the caller's checks expect: longest first
    pieces.sort(key=lambda p: -_piece_work(lengths, p, 3))
    return (len(pieces), n_merge, n_partials), pieces, merges


def _tile_work(lengths, s, t, kind, causal=True):
    end = min(lengths[s], (t + 1) * ROWS[kind])
    return -(-(end if causal else lengths[s]) // KEYS[kind])


def _piece_work(lengths, p, kind):
    s, t, sp, ns, _ = p
    n = _tile_work(lengths, s, t, kind)
    return (sp + 1) * n // ns - sp * n // ns


@pytest.mark.parametrize("lengths,H,kernel", [
    ([100, 1, 700, 64, 65, 1742, 450], 16, None),     # duo kernel (< 8192 tokens), fills the chip
    ([100, 1, 700, 64, 65, 1742, 450], 16, "staged"),
    ([100, 1, 2100, 64, 65], 4, "ring"),              # underfilled: split pieces
    ([100, 8200], 2, None),                           # ring kernel (>= 8192 tokens), underfilled
    ([100, 1, 2100, 64, 65], 4, None),                # duo kernel, underfilled: split pieces
    ([100, 1, 2100, 64, 65], 2, "ring"),
    ([100, 1, 2100, 64, 65], 4, "duo"),
])
def test_schedule_covers_every_tile_once_heaviest_first(lengths, H, kernel):
    (n_work, n_merge, n_partials), pieces, merges = _schedule(lengths, H=H, H_kv=min(H, 8), kernel=kernel)
    kind = _kind(kernel, 128, lengths)
    rows = ROWS[kind]
    # every (tile, split) exactly once; splits of a tile share its n_split and slot
    seen = {}
    for s, t, sp, ns, slot in pieces:
        assert 0 <= sp < ns <= 4 and (s, t, sp) not in seen
        seen[(s, t, sp)] = (ns, slot)
    tiles = {(s, t) for s, n in enumerate(lengths) for t in range(-(-n // rows))}
    assert {(s, t) for s, t, _ in seen} == tiles
    for s, t in tiles:
        ns = seen[(s, t, 0)][0]
        assert all(seen[(s, t, sp)] == seen[(s, t, 0)] for sp in range(ns))
    # a merge entry for exactly the split tiles, each owning consecutive partial slots
    split_tiles = {(s, t): seen[(s, t, 0)] for s, t in tiles if seen[(s, t, 0)][0] > 1}
    assert {(s, t): (ns, slot) for s, t, ns, slot in merges} == split_tiles
    slots = sorted(slot for _, slot in split_tiles.values())
    assert slots == [sum(ns for ns, sl in split_tiles.values() if sl < x) for x in slots]
    assert n_partials == sum(ns for ns, _ in split_tiles.values()) and n_merge == len(merges)
    assert bool(merges) == (kind != 0 and len(tiles) * H < 256 * PER_CU[kind])
    # pieces partition their tile's key tiles and come heaviest first
    work = [_piece_work(lengths, p, kind) for p in pieces]
    assert all(x > 0 for x in work) and work == sorted(work, reverse=True)
    assert n_work == len(pieces)


@pytest.mark.parametrize("kernel,H", [("ring", 8), ("ring", 4), ("duo", 8)])
def test_schedule_splits_only_launches_that_underfill_the_chip(kernel, H):
    kind = KERNELS[kernel]
    rows = ROWS[kind]
    # one 2100-token segment: 17 ring tiles x 8 or 4 heads, 33 duo tiles x 8 heads < the chip,
    # so long tiles are cut to the per-CU share of the work (at least 8 units, at most 4
    # pieces)
    lengths = [2100]
    _, pieces, merges = _schedule(lengths, H=H, H_kv=4, kernel=kernel)
    total = sum(_tile_work(lengths, 0, t, kind) for t in range(-(-lengths[0] // rows)))
    cap = max(-(-(total * H) // (256 * PER_CU[kind])), 8)
    assert merges
    for p in pieces:
        n = _tile_work(lengths, p[0], p[1], kind)
        assert _piece_work(lengths, p, kind) <= max(cap, -(-n // 4))
    # 4096 tokens at 16 heads and the config-3 batch fill the chip: no splits
    for lengths in ([4096], [1742, 110, 658, 364, 390, 450, 152, 445]):
        _, pieces, merges = _schedule(lengths, H=16, kernel=kernel)
        assert not merges and all(p[3] == 1 for p in pieces)


def test_schedule_head_dim_256_runs_the_duo_kernel_one_workgroup_per_cu():
    """head_dim 256 defaults to the duo kernel with one persistent workgroup per CU (256 at
    most); a launch that fills them is not split."""
    lengths = [100, 1700]
    (_, n_merge, n_partials), pieces, _ = _schedule(lengths, D=256)
    assert n_merge == 0 and n_partials == 0
    host_cu = (ctypes.c_int32 * 3)(0, 100, 1800)
    words = _lib.lib.mi_varlen_schedule_for(host_cu, 2, 16, 8, 256, 1, -1, None, 0)
    out = (ctypes.c_int32 * words)()
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 2, 16, 8, 256, 1, -1, out, words) == words
    assert out[0] == 256 and out[3] == (3 << 20) | (256 << 8) | 64  # workgroups, duo layout
    assert sorted((s, t) for s, t, *_ in pieces) == sorted(
        {(s, t) for s, n in enumerate(lengths) for t in range(-(-n // 64))})


@pytest.mark.parametrize("H,H_kv,D", [(8, 2, 256), (16, 4, 128), (16, 1, 128)])
def test_schedule_gives_each_kv_head_its_block_of_xcds(H, H_kv, D):
    """A chip-filling duo launch whose KV heads divide the 8 XCDs deals each KV head's items
    to the workgroups of its block of 8 / H_kv XCDs (workgroup w on XCD w % 8; checked per
    item by the parser) and still covers every tile once per head; with one KV head every
    workgroup takes part."""
    lengths = [1742, 110, 658, 364, 390, 450, 152, 445]  # config 3
    (n_work, _, _), pieces, _ = _schedule(lengths, H=H, H_kv=H_kv, D=D)
    assert sorted((s, t) for s, t, *_ in pieces) == sorted(
        {(s, t) for s, n in enumerate(lengths) for t in range(-(-n // 64))})


def test_schedule_default_leaves_the_duo_kernel_past_255_heads():
    """The duo item word holds a head id in 8 bits: by default a batch of 256 or more heads
    runs the ring kernel at head_dim 64/128 and the register-staged kernel at 256, and naming
    the duo kernel for it is refused."""
    host_cu = (ctypes.c_int32 * 3)(0, 100, 400)

    def kind(H, H_kv, D, kernel=-1):
        words = _lib.lib.mi_varlen_schedule_for(host_cu, 2, H, H_kv, D, 1, kernel, None, 0)
        assert words > 0
        out = (ctypes.c_int32 * words)()
        assert _lib.lib.mi_varlen_schedule_for(host_cu, 2, H, H_kv, D, 1, kernel, out, words) == words
        return out[3] >> 20

    assert kind(255, 5, 128) == 3 and kind(256, 8, 128) == 1 and kind(256, 8, 64) == 1
    assert kind(255, 5, 256) == 3 and kind(256, 8, 256) == 0
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 2, 256, 8, 128, 1, 3, None, 0) == _lib.MI_ERR_UNSUPPORTED


def test_schedule_rejects_unknown_kernels_and_head_dims():
    host_cu = (ctypes.c_int32 * 2)(0, 5)
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 1, 16, 8, 128, 1, 7, None, 0) == _lib.MI_ERR_INVALID
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 1, 16, 8, 128, 1, -2, None, 0) == _lib.MI_ERR_INVALID
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 1, 16, 8, 128, 1, 2, None, 0) == _lib.MI_ERR_INVALID  # removed
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 1, 16, 8, 256, 1, 1, None, 0) == _lib.MI_ERR_UNSUPPORTED
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 1, 16, 8, 256, 1, 0, None, 0) > 0
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 1, 16, 8, 256, 1, 3, None, 0) > 0
    assert _lib.lib.mi_varlen_schedule_for(host_cu, 1, 16, 8, 512, 1, 3, None, 0) == _lib.MI_ERR_UNSUPPORTED


def test_schedule_rejects_empty_segments():
    host_cu = (ctypes.c_int32 * 3)(0, 5, 5)
    assert _lib.lib.mi_varlen_schedule(host_cu, 2, 16, 8, 128, 1, None, 0) == _lib.MI_ERR_INVALID


def test_rows_gemm_split_choice_and_argument_checks():
    split = _lib.lib.mi_rows_gemm_split
    # one launch of >= 192 workgroups with at most two 64-k steps per wave at the Qwen3-0.6B
    # decode projections; the lm_head (4748 column tiles) needs no split
    assert [split(32, n, k) for n, k in [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072)]] == [2, 8, 2, 6]
    assert split(32, 151936, 1024) == 1
    assert split(32, 64, 1000) == 0
    gemm = _lib.lib.mi_rows_gemm
    assert gemm(None, 1024, None, 1024, None, 64, None, 33, 64, 1024, 1, 2, None) == _lib.MI_ERR_INVALID
    assert "M=33" in _lib.last_error()
    assert gemm(None, 1024, None, 1024, None, 64, None, 4, 64, 1000, 1, 2, None) == _lib.MI_ERR_UNSUPPORTED
    assert gemm(None, 2048, None, 2048, None, 64, None, 4, 64, 2048, 1, 2, None) == _lib.MI_ERR_UNSUPPORTED
    assert "more than 1024" in _lib.last_error()
    assert gemm(None, 1024, None, 1024, None, 64, None, 4, 64, 1024, 2, 2, None) == _lib.MI_ERR_INVALID
    assert "NULL" in _lib.last_error()

