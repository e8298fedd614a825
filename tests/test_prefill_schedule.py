"""The host side of the packed-prefill launch: the schedules mi_varlen_schedule_for writes
(CPU only, no GPU calls).

The tall kernel's schedule carries the whole contract of its in-launch merge, so it is
decoded here word by word: every (segment, 128-row tile, head) must be covered by key
ranges that tile its causal range exactly once; a split tile has producers then one owner
(the piece with the diagonal), one counter and one partial slot per producer; and no
workgroup runs an owner before a producer, which is what makes every owner's wait end.
The default kernel choice follows the measured rule documented at kTallMinLen.
"""

from __future__ import annotations

import ctypes
import math

import pytest

from miattn import _lib

pytestmark = pytest.mark.skipif(not _lib.HIP_AVAILABLE, reason=f"libmiattn.so did not load: {_lib.LOAD_ERROR}")

PREFILL = {0: "staged", 1: "ring", 3: "duo", 4: "tall"}
ROLE_WHOLE, ROLE_PRODUCER, ROLE_OWNER = 0, 1, 2
TILE_ROWS, STEP_KEYS, ENTRY_WORDS, ITEM_WORDS = 128, 64, 8, 6


def _cu(lengths):
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return cu


def _schedule(lengths, H, H_kv, D=128, causal=True, kernel=-1):
    cu = _cu(lengths)
    host_cu = (ctypes.c_int32 * len(cu))(*cu)
    n = _lib.lib.mi_varlen_schedule_for(host_cu, len(lengths), H, H_kv, D, int(causal), kernel, None, 0)
    assert n > 0, _lib.lib.mi_last_error()
    words = (ctypes.c_int32 * n)()
    assert _lib.lib.mi_varlen_schedule_for(host_cu, len(lengths), H, H_kv, D, int(causal), kernel, words, n) == n
    return cu, list(words)


def _steps(L, tile, causal):
    end = min(L, (tile + 1) * TILE_ROWS)
    return math.ceil((end if causal else L) / STEP_KEYS)


def _decode_tall(cu, w, causal):
    n_wg, n_counters, n_partials, layout = w[:4]
    assert PREFILL[layout >> 20] == "tall" and layout & 0xFF == TILE_ROWS
    pieces, lists = {}, []
    for wg in range(n_wg):
        first, count = w[4 + ENTRY_WORDS * wg], w[5 + ENTRY_WORDS * wg]
        assert count >= 1
        items = []
        for i in range(count):
            it = w[first + ITEM_WORDS * i: first + ITEM_WORDS * (i + 1)]
            if i == 0:
                assert it == w[6 + ENTRY_WORDS * wg: 4 + ENTRY_WORDS * (wg + 1)], "the entry carries item 0 inline"
            seg = cu.index(it[0])
            assert cu[seg + 1] - it[0] == it[1]
            tile, head = it[2] >> 16, it[2] & 0xFFFF
            t0, t1 = it[3] >> 16, it[3] & 0xFFFF
            role, n_prod, counter = (it[4] >> 30) & 3, (it[4] >> 24) & 63, it[4] & 0xFFFFFF
            assert 0 <= t0 < t1 <= _steps(it[1], tile, causal)
            pieces.setdefault((seg, tile, head), []).append((t0, t1, role, n_prod, counter, it[5]))
            items.append(role)
        lists.append(items)
    return n_wg, n_counters, n_partials, pieces, lists


CASES = [
    pytest.param([1742, 110, 658, 364, 390, 450, 152, 445], 16, 8, True, id="config3"),
    pytest.param([17, 1, 128, 333], 16, 8, True, id="short"),
    pytest.param([2100], 8, 4, True, id="one-long-gqa2"),
    pytest.param([2100], 2, 1, True, id="one-long-h2"),
    pytest.param([2050, 70], 8, 4, False, id="non-causal"),
    pytest.param([1, 1, 17, 128, 1517, 3, 64, 200], 8, 1, True, id="8seg-mqa"),
    pytest.param([4311], 16, 8, True, id="4311"),
    pytest.param([8192], 16, 8, True, id="8192-no-split"),
]


@pytest.mark.parametrize("lengths,H,H_kv,causal", CASES)
def test_tall_schedule_covers_every_tile_once_and_orders_producers_first(lengths, H, H_kv, causal):
    cu, w = _schedule(lengths, H, H_kv, causal=causal, kernel=4)
    n_wg, n_counters, n_partials, pieces, lists = _decode_tall(cu, w, causal)
    assert n_wg <= 512  # two workgroups per CU on the 256-CU MI355X: the whole grid is resident
    assert len(pieces) == sum(math.ceil(n / TILE_ROWS) for n in lengths) * H
    counters, slots = set(), set()
    for (seg, tile, head), ps in pieces.items():
        ps.sort()
        L = cu[seg + 1] - cu[seg]
        assert ps[0][0] == 0 and ps[-1][1] == _steps(L, tile, causal)
        assert all(a[1] == b[0] for a, b in zip(ps, ps[1:])), "key ranges must tile the causal range"
        if len(ps) == 1:
            assert ps[0][2] == ROLE_WHOLE
            continue
        assert [p[2] for p in ps] == [ROLE_PRODUCER] * (len(ps) - 1) + [ROLE_OWNER]
        owner = ps[-1]
        assert owner[3] == len(ps) - 1
        assert len({p[4] for p in ps}) == 1 and owner[4] not in counters and 0 <= owner[4] < n_counters
        counters.add(owner[4])
        assert sorted(p[5] for p in ps[:-1]) == list(range(owner[5], owner[5] + owner[3]))
        for p in ps[:-1]:
            assert p[5] not in slots and 0 <= p[5] < n_partials
            slots.add(p[5])
    assert len(counters) == n_counters and len(slots) == n_partials
    for roles in lists:
        seen_owner = False
        for role in roles:
            assert not (role == ROLE_PRODUCER and seen_owner), "an owner must never precede a producer"
            seen_owner |= role == ROLE_OWNER


def test_tall_workspace_holds_the_counters_then_the_partials():
    cu, w = _schedule([1742, 110, 658], 16, 8, kernel=4)
    n_counters, n_partials = w[1], w[2]
    assert n_counters > 0 and n_partials > 0
    header = (ctypes.c_int32 * len(w))(*w)
    counter_bytes = (n_counters * 4 + 255) // 256 * 256
    part_floats = TILE_ROWS * 128 + 2 * TILE_ROWS
    assert _lib.lib.mi_varlen_workspace_size(header, 16) == counter_bytes + n_partials * part_floats * 4


@pytest.mark.parametrize("lengths,H,H_kv,D,expected", [
    pytest.param([1742, 110, 658, 364, 390, 450, 152, 445], 16, 8, 128, "duo", id="config3-duo"),
    pytest.param([1536] * 8, 16, 8, 128, "tall", id="8x1536-tall"),
    pytest.param([2048] * 8, 16, 8, 128, "tall", id="8x2048-tall"),
    pytest.param([2048] * 2, 16, 8, 128, "duo", id="2x2048-would-split-duo"),
    pytest.param([1024] * 16, 16, 8, 128, "duo", id="16x1024-duo"),
    pytest.param([8192], 16, 8, 128, "tall", id="8192-tall"),
    pytest.param([8192], 2, 1, 128, "ring", id="8192-underfilled-ring"),
    pytest.param([2048] * 8, 16, 8, 64, "tall", id="d64-tall"),
    pytest.param([2048] * 8, 8, 2, 256, "duo", id="d256-duo"),
    pytest.param([70, 5, 130], 256, 8, 128, "ring", id="256-heads-ring"),
])
def test_default_kernel_choice(lengths, H, H_kv, D, expected):
    _, w = _schedule(lengths, H, H_kv, D=D)
    assert PREFILL[w[3] >> 20] == expected


def test_tall_takes_head_dim_64_and_128_only():
    cu = (ctypes.c_int32 * 2)(0, 16)
    rc = _lib.lib.mi_varlen_schedule_for(cu, 1, 8, 2, 256, 1, 4, None, 0)
    assert rc == _lib.MI_ERR_UNSUPPORTED and b"tall kernel" in _lib.lib.mi_last_error()
