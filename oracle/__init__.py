"""Test oracle for the DSA path -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference algorithms, used as the checker by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``.
Nothing in the product package (``ascendc_kernel_amd``) imports it, and it is
never the thing measured as the product.

Modules
  sparse_attn  Task1 restatement in torch (runs on CPU or GPU) + an fp64 brute force
               (reference/task1_v0_ref.py:5-55)
  indexer      Task2 restatement in torch (CPU or GPU) incl. the constructor's RNG
               consumption (reference/task2_v0_ref.py:21-172)
  rules        numpy statements of the bit-level rules (bf16 rounding, RoPE rounding
               variants, head-sum order, top-k tie order, mask/fill)

Pinning (which check fixes which function) is listed in the header of each module.
Functions marked "parity unpinned" there have no independent check.
"""
