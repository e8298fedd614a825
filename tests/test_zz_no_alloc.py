"""mi_paged_decode_noalloc (split-K partials in the library's per-GPU scratch array) against
mi_paged_decode with a caller workspace, through the C ABI: bit-identical outputs on two
calls in a row, the second with a smaller batch (the scratch keeps the first call's
partials), and a clear refusal of a shape whose partials exceed the array."""

from __future__ import annotations

import pytest
import torch

from miattn import _lib, paged_decode
from miattn import workloads as W

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 8 << 20  # MI_DECODE_SCRATCH_BYTES


def _noalloc(q, k, v, table, seqlen, out, scale):
    B, H, D = q.shape
    _, bs, H_kv, _ = k.shape
    strides = _lib.int64_array((*q.stride(), *k.stride(), *v.stride(), *out.stride(), table.stride(0)))
    return _lib.lib.mi_paged_decode_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(), seqlen.data_ptr(), out.data_ptr(), B, H, H_kv,
        D, bs, table.shape[1], strides, scale, _lib.dtype_code(q.dtype), _lib.current_stream(q.device))


def test_noalloc_decode_equals_the_workspace_entry_point_on_two_calls(cuda):
    big = W.paged_decode_config(n_layer=1, device=cuda)                      # config 2: B=32, 8192 blocks
    small = W.paged_decode_config(B=5, lengths=[3000, 1, 0, 700, 129], n_blocks=512, n_layer=1, device=cuda, seed=9)
    for inp in (big, small):                                                 # second call: smaller input
        q, k, v = inp.q[0], inp.k_caches[0], inp.v_caches[0]
        assert _lib.lib.mi_paged_decode_workspace_size(q.shape[0], 16, 8, 128, 16, inp.block_table.shape[1], 2) \
            <= SCRATCH_BYTES
        expected = paged_decode(q, k, v, inp.block_table, inp.seqlen)
        out = torch.full_like(q, float("nan"))
        rc = _noalloc(q, k, v, inp.block_table, inp.seqlen, out, 128 ** -0.5)
        assert rc == _lib.MI_OK, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, expected)


def test_noalloc_refuses_a_shape_beyond_the_scratch(cuda):
    B, H, H_kv, D = 600, 16, 8, 128   # (512 + 600) splits x 16 heads x 130 fp32 > 8 MiB
    assert _lib.lib.mi_paged_decode_workspace_size(B, H, H_kv, D, 16, 4, 2) > SCRATCH_BYTES
    q = torch.zeros(B, H, D, dtype=torch.bfloat16, device=cuda)
    k = torch.zeros(4, 16, H_kv, D, dtype=torch.bfloat16, device=cuda)
    table = torch.zeros(B, 4, dtype=torch.int32, device=cuda)
    seqlen = torch.ones(B, dtype=torch.int32, device=cuda)
    out = torch.empty_like(q)
    rc = _noalloc(q, k, k, table, seqlen, out, 1.0)
    assert rc == _lib.MI_ERR_WORKSPACE
    assert "scratch" in _lib.last_error()
