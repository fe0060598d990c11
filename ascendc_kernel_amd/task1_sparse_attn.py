"""Task1 drop-in: sparse attention with attention sink on MI355X.

Same surface as the reference module reference/task1_v0_ref.py:27-55 (and its
Ascend counterpart ``ModelNew`` in src/task1_sparse_attn.py:666-823):
``Model(n_heads, head_dim)`` with the ``attn_sink`` parameter, and
``forward(q, kv, topk_idxs)`` returning a fresh bf16 tensor shaped like q.
Module-level ``get_inputs()`` / ``get_init_inputs()`` build the reference's
benchmark inputs (task1_v0_ref.py:39-55).

The forward runs the gfx950 kernel behind ``dsa_sparse_attn_fwd``; inputs must
be on the HIP device. There is no fallback: unsupported shapes raise.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _native


class Model(nn.Module):
    """Drop-in for ``Model`` of reference/task1_v0_ref.py:27-36."""

    #: kernel choice passed to the C ABI (auto = multiplicity kernel when n_kv <= 32)
    variant: int = _native.DSA_SA_AUTO

    def __init__(self, n_heads: int, head_dim: int):
        super().__init__()
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.softmax_scale = head_dim ** -0.5
        self.attn_sink = nn.Parameter(torch.zeros(n_heads, dtype=torch.float32))

    def forward(self, q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor) -> torch.Tensor:
        if q.shape[2] != self.n_heads or q.shape[3] != self.head_dim:
            raise ValueError(f"q {tuple(q.shape)} does not match n_heads={self.n_heads}, "
                             f"head_dim={self.head_dim}")
        return _native.sparse_attn_fwd(q, kv, topk_idxs, self.attn_sink, self.softmax_scale,
                                       self.variant)


# The Ascend submission names its module ModelNew (src/task1_sparse_attn.py:666).
ModelNew = Model

batch_size = 8
seq_len = 2600
n_kv = 32
n_heads = 64
head_dim = 128
topk = 16


def get_inputs():
    """Benchmark inputs of reference/task1_v0_ref.py:47-51 (CPU tensors)."""
    q = torch.randn(batch_size, seq_len, n_heads, head_dim, dtype=torch.bfloat16)
    kv = torch.randn(batch_size, n_kv, head_dim, dtype=torch.bfloat16)
    topk_idxs = torch.randint(0, n_kv, (batch_size, seq_len, topk), dtype=torch.int32)
    return [q, kv, topk_idxs]


def get_init_inputs():
    return [n_heads, head_dim]
