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


def _schedule(lengths, H=16, H_kv=8, D=128, causal=1):
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    host_cu = (ctypes.c_int32 * len(cu))(*cu)
    n = _lib.lib.mi_varlen_schedule(host_cu, len(lengths), H, H_kv, D, causal, None, 0)
    out = (ctypes.c_int32 * max(n, 1))()
    assert _lib.lib.mi_varlen_schedule(host_cu, len(lengths), H, H_kv, D, causal, out, n) == n
    return [(out[i] >> 16, out[i] & 0xFFFF) for i in range(n)]


def test_schedule_covers_every_tile_once_heaviest_first():
    lengths = [100, 1, 700, 64, 65]
    rows = 64  # 64 query rows per workgroup (one head, 2 query blocks x 2 key halves)
    sched = _schedule(lengths)
    expected = {(s, t) for s, n in enumerate(lengths) for t in range(-(-n // rows))}
    assert sorted(sched) == sorted(expected)
    work = [min(lengths[s], (t + 1) * rows) for s, t in sched]
    kt = [-(-w // 64) for w in work]  # 64-key tiles
    assert kt == sorted(kt, reverse=True)


def test_schedule_rejects_empty_segments():
    host_cu = (ctypes.c_int32 * 3)(0, 5, 5)
    assert _lib.lib.mi_varlen_schedule(host_cu, 2, 16, 8, 128, 1, None, 0) == _lib.MI_ERR_INVALID
