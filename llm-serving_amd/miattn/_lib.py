"""ctypes binding of ``libmiattn.so`` (the C ABI in ``include/miattn.h``).

The library is loaded after ``torch`` so that its ``libamdhip64`` dependency resolves to
the HIP runtime torch already mapped (same soname): device pointers, streams and the
caching allocator then all belong to one runtime. Loading never touches a GPU; the first
launch does.

There is no fallback: when the library is missing, ``HIP_AVAILABLE`` is False and every
entry point raises ``RuntimeError`` naming the load error.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  -- must be imported before the library (see module docstring)

__all__ = [
    "HIP_AVAILABLE",
    "LOAD_ERROR",
    "LIB_PATH",
    "lib",
    "check",
    "dtype_code",
    "current_stream",
    "MI_OK",
    "MI_ERR_INVALID",
    "MI_ERR_UNSUPPORTED",
    "MI_ERR_WORKSPACE",
    "MI_ERR_LAUNCH",
]

MI_OK = 0
MI_ERR_INVALID = -1
MI_ERR_UNSUPPORTED = -2
MI_ERR_WORKSPACE = -3
MI_ERR_LAUNCH = -4

LIB_PATH = Path(os.environ.get("MIATTN_LIB", Path(__file__).resolve().parent / "libmiattn.so"))

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_int64 = ctypes.c_int64
_c_size_t = ctypes.c_size_t
_c_float = ctypes.c_float
_p_int64 = ctypes.POINTER(ctypes.c_int64)
_p_int32 = ctypes.POINTER(ctypes.c_int32)

# Exported symbol -> (restype, argtypes). Kept in step with include/miattn.h; the CPU test
# suite checks that every function the header declares is exported and bound here.
SIGNATURES: dict[str, tuple] = {
    "mi_last_error": (ctypes.c_char_p, []),
    "mi_abi_version": (_c_int, []),
    "mi_kv_slot_write": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_int64, _c_int,
         _c_int, _c_int64, _p_int64, _c_int, _c_void_p, _c_void_p],
    ),
    "mi_paged_decode_workspace_size": (_c_size_t, [_c_int] * 7),
    "mi_paged_decode": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_int, _p_int64, _c_float, _c_int, _c_void_p, _c_size_t,
         _c_void_p],
    ),
    "mi_paged_decode_fused": (
        _c_int,
        [_c_void_p, _c_int64, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int, _c_void_p,
         _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_int64, _p_int64, _c_float, _c_float, _c_int, _c_int, _c_void_p, _c_size_t,
         _c_void_p, _c_void_p],
    ),
    "mi_paged_decode_noalloc": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_int, _p_int64, _c_float, _c_int, _c_void_p],
    ),
    "mi_varlen_schedule": (
        _c_int, [_p_int32, _c_int, _c_int, _c_int, _c_int, _c_int, _p_int32, _c_int]
    ),
    "mi_varlen_schedule_for": (
        _c_int, [_p_int32, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p_int32, _c_int]
    ),
    "mi_varlen_workspace_size": (_c_size_t, [_p_int32, _c_int]),
    "mi_add_rms_norm": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_float, _c_int, _c_void_p],
    ),
    "mi_silu_mul": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_int, _c_int, _c_int, _c_void_p]),
    "mi_rows_gemm_split": (_c_int, [_c_int, _c_int, _c_int]),
    "mi_rows_gemm_glu": (
        _c_int,
        [_c_void_p, _c_int64, _c_void_p, _c_int64, _c_void_p, _c_int64, _c_int, _c_int, _c_int, _c_int, _c_void_p],
    ),
    "mi_argmax_rows": (_c_int, [_c_void_p, _c_int64, _c_int, _c_int, _c_void_p, _c_int, _c_void_p]),
    "mi_rows_gemm_argmax": (
        _c_int,
        [_c_void_p, _c_int64, _c_void_p, _c_int64, _c_void_p, _c_int64, _c_void_p, _c_int, _c_int, _c_int, _c_int,
         _c_void_p],
    ),
    "mi_greedy_advance_tiles": (
        _c_int,
        [_c_void_p, _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int64, _c_void_p, _c_int, _c_void_p],
    ),
    "mi_decode_step_begin": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int, _c_int, _c_void_p, _c_int64, _c_void_p, _c_int,
         _c_float, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p, _c_void_p],
    ),
    "mi_greedy_advance": (
        _c_int,
        [_c_void_p, _c_int64, _c_int, _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int64, _c_void_p,
         _c_int, _c_void_p],
    ),
    "mi_rows_gemm": (
        _c_int,
        [_c_void_p, _c_int64, _c_void_p, _c_int64, _c_void_p, _c_int64, _c_void_p, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_void_p],
    ),
    "mi_qk_norm_rope_write": (
        _c_int,
        [_c_void_p, _c_int64, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int, _c_void_p,
         _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_int, _c_int64, _c_float, _c_int, _c_int, _c_void_p, _c_void_p],
    ),
    "mi_varlen_prefill": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int,
         _c_int, _c_void_p, _c_size_t, _c_void_p, _c_void_p],
    ),
    "mi_prefill_wait_limit": (_c_int, [_c_int]),
}

ABI_VERSION = 13


def _load():
    try:
        handle = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        return None, f"{type(exc).__name__}: {exc}"
    for name, (restype, argtypes) in SIGNATURES.items():
        try:
            fn = getattr(handle, name)
        except AttributeError:
            return None, f"{LIB_PATH} does not export {name}; rebuild it"
        fn.restype = restype
        fn.argtypes = argtypes
    version = handle.mi_abi_version()
    if version != ABI_VERSION:
        return None, f"{LIB_PATH} has ABI version {version}, this shim expects {ABI_VERSION}"
    return handle, None


lib, LOAD_ERROR = _load()
HIP_AVAILABLE: bool = lib is not None

_DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"dtype must be fp16, bf16 or fp32, got {dtype}") from None


def current_stream(device: torch.device) -> int:
    """Raw ``hipStream_t`` of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def last_error() -> str:
    msg = lib.mi_last_error() if lib is not None else None
    return msg.decode(errors="replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Map a C status to the reference's exception split: contract -> ValueError,
    runtime -> RuntimeError."""
    if rc == MI_OK:
        return
    message = f"{what}: {last_error()}"
    if rc == MI_ERR_LAUNCH:
        raise RuntimeError(message)
    raise ValueError(message)


def require_library(what: str) -> None:
    if lib is None:
        raise RuntimeError(
            f"{what} requires libmiattn.so (the HIP kernels), but it could not be loaded "
            f"from {LIB_PATH}: {LOAD_ERROR}. Build it with __graft_entry__.build(); there is "
            "no fallback implementation."
        )


def int64_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (ctypes.c_int64 * len(values))(*values)
