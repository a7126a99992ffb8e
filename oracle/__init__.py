"""CPU oracle for the FP8 block-scale DeepSeek-V3 MoE operator.

TEST INFRASTRUCTURE ONLY. Nothing in the product path imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only to check results (or as the timed CPU baseline),
never as the computation that is shipped or measured on the GPU.

* ``cpu_ref``  -- a PyTorch-on-CPU restatement of ``reference moe/ref_moe.py:4-168``
  (same operations in the same order, fp32), plus its routing and dispatch
  stages exposed separately for bit-exact checks.
* ``np_ref``   -- independent checks: the OCP e4m3 decode table from the spec,
  a brute-force routing search over all 70 group subsets, and a float64 NumPy
  recomputation of selected output rows.
"""
