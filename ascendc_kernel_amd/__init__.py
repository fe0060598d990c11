"""MI355X-native DeepSeek-sparse-attention path (Task1 sparse attention, Task2 lightning indexer).

Drop-in modules with the reference's PyTorch signatures:
  ascendc_kernel_amd.task1_sparse_attn.Model   (reference/task1_v0_ref.py:27-36)
  ascendc_kernel_amd.task2_indexer.Model       (reference/task2_v0_ref.py:106-144)
Both call hand-written gfx950 HIP kernels through the C ABI in include/dsa_abi.h.
"""
from . import _native, task1_sparse_attn, task2_indexer  # noqa: F401

__all__ = ["task1_sparse_attn", "task2_indexer"]
