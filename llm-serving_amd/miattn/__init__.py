"""miattn -- MI355X (gfx950) HIP kernels for the paged-KV serving attention hot path.

Drop-in modules, each mirroring one reference interface:

* :mod:`miattn.decode`  -- ``paged_decode``, ``paged_decode_plan``, ``PagedDecodePlan``,
  ``TRITON_AVAILABLE`` (reference ``model/triton_decode.py``);
* :mod:`miattn.varlen`  -- ``HipVarlen`` (also exported as ``FlashVarlen``), ``SdpaVarlen``,
  ``backend_for`` (reference ``model/attention/varlen.py``);
* :mod:`miattn.paged`   -- ``PagedPool``, ``PagedKV``, ``PagedWriteSink`` (reference
  ``model/paged.py`` and ``serve/engine.py``'s sink);
* :mod:`miattn.packed`  -- ``PackedPrefill`` (reference ``model/packed.py``).

Device work on a HIP device goes through ``libmiattn.so`` (C ABI in ``include/miattn.h``);
when the library is missing those entry points raise instead of computing anything another
way. Host (CPU) pools and the CPU prefill arm behave as the reference's own host arms.
"""

from ._lib import HIP_AVAILABLE, LIB_PATH, LOAD_ERROR
from .decode import TRITON_AVAILABLE, PagedDecodePlan, paged_decode, paged_decode_plan
from .packed import PackedPrefill, as_packed_prefill
from .paged import PagedKV, PagedPool, PagedWriteSink
from .varlen import FlashVarlen, HipVarlen, SdpaVarlen, backend_for

__all__ = [
    "HIP_AVAILABLE", "LIB_PATH", "LOAD_ERROR", "TRITON_AVAILABLE", "PagedDecodePlan", "paged_decode",
    "paged_decode_plan", "PackedPrefill", "as_packed_prefill", "PagedKV", "PagedPool", "PagedWriteSink",
    "FlashVarlen", "HipVarlen", "SdpaVarlen", "backend_for",
]
