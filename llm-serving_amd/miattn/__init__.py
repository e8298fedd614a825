"""miattn -- MI355X (gfx950) HIP kernels for the paged-KV serving attention hot path.

Drop-in modules, each mirroring one reference interface:

* :mod:`miattn.decode`  -- ``paged_decode``, ``paged_decode_plan``, ``PagedDecodePlan``,
  ``TRITON_AVAILABLE`` (reference ``model/triton_decode.py``);
* :mod:`miattn.varlen`  -- ``HipVarlen`` / ``backend_for`` (reference
  ``model/attention/varlen.py``, CUDA arm);
* :mod:`miattn.paged`   -- ``PagedPool``, ``PagedKV``, ``PagedWriteSink`` (reference
  ``model/paged.py`` and ``serve/engine.py`` sinks);
* :mod:`miattn.packed`  -- ``PackedPrefill`` (reference ``model/packed.py``);
* :mod:`miattn.block_manager` -- ``BlockManager`` (reference ``serve/block_manager.py``).

All device work goes through ``libmiattn.so`` (C ABI in ``include/miattn.h``); when the
library is missing the entry points raise instead of computing anything another way.
"""

from ._lib import HIP_AVAILABLE, LIB_PATH, LOAD_ERROR
from .block_manager import BlockManager
from .decode import TRITON_AVAILABLE, PagedDecodePlan, paged_decode, paged_decode_plan
from .packed import PackedPrefill, as_packed_prefill
from .paged import PagedKV, PagedPool, PagedWriteSink
from .varlen import HipVarlen, backend_for

__all__ = [
    "HIP_AVAILABLE", "LIB_PATH", "LOAD_ERROR", "TRITON_AVAILABLE", "BlockManager", "PagedDecodePlan",
    "paged_decode", "paged_decode_plan", "PackedPrefill", "as_packed_prefill", "PagedKV", "PagedPool",
    "PagedWriteSink", "HipVarlen", "backend_for",
]
