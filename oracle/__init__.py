"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A plain restatement (numpy / torch-on-CPU) of the reference's algorithms for the three
hot-path pieces, each function citing the reference file:line it follows:

* ``oracle.slots``  -- slot-map closed form and the per-token / per-block write loops
  (reference ``model/paged.py:150-168,474-501``; ``tests/reference/paged.py:93-124``;
  ``tests/unit/test_paged_kv.py:63-80``);
* ``oracle.decode`` -- the dense paged-decode oracles: float64 per-token softmax
  (reference ``tests/unit/test_triton_decode.py:75-105``) and the fp32 gather + einsum
  oracle (reference ``tests/reference/paged.py:225-274``);
* ``oracle.seat``   -- the CPU seat path: ``KvSlab`` write + mask/bias and the
  ``hand_baddbmm`` decode math with softmax in the input dtype (reference
  ``model/slab.py:251-328``, ``model/attention/hand_baddbmm.py:80-149``);
* ``oracle.varlen`` -- packed prefill: the longhand fp32 per-segment oracle (reference
  ``tests/unit/test_attention_varlen.py:71-92``) and the SDPA-per-segment arm (reference
  ``model/attention/varlen.py:259-290``).

Who may use it: ``tests/`` (as the checker), ``__graft_entry__.smoke()`` (as the
checker) and ``bench.py``'s ``cpu_baseline`` leg (the reference's CPU seat path, timed as
a reported baseline). The product package ``miattn`` never imports it; its entry points
fail loudly when the HIP library is absent instead of computing through anything here.

How each function is pinned (beyond restating the reference) is recorded next to the
function and checked in ``tests/test_oracle_*.py``: the reference tests' known-answer
values (``tests/golden/``), independent library routines (torch SDPA in float64), closed
forms and brute force on tiny inputs.
"""
