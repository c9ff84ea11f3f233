"""CPU oracle for the MoE layer hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check results or as the timed
CPU baseline.  The product (``resihp-megatron_amd/``) never imports it.

Contents:

``route_c``   ctypes bridge to ``route_ref.c``: the bit-exact routing contract
              (fixed-order fp32/fp64 router logits, lowest-id top-k, gates,
              counts / offsets / permutation).
``moe_ref``   float64 torch restatement of ``resihp/runtime/moe.py`` (seeds,
              parameters, route, expert FFN, combine, autograd backward, Adam,
              bias update, training loop) plus the extensions the MI355X
              build adds (SwiGLU experts, sigmoid scoring, shared experts,
              FP8 delayed scaling).

Every oracle function is pinned by a check in ``tests/test_oracle_*.py``:
the reference's own recorded float64 outputs (``tests/golden``), a closed
form, brute force on tiny inputs, or a library routine.
"""
