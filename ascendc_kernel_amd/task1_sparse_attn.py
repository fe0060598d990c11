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

    def __init__(self, n_heads: int, head_dim: int, v_dim: int = None):
        """`v_dim` (not in the reference, default None = head_dim): value width for sparse
        MLA, where kv rows carry head_dim key channels of which the first v_dim are the value."""
        super().__init__()
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.v_dim = v_dim
        self.softmax_scale = head_dim ** -0.5
        self.attn_sink = nn.Parameter(torch.zeros(n_heads, dtype=torch.float32))
        # (key, _native.Prepared) of the last call. The prepared launch holds its inputs, so
        # their memory cannot be reused for other tensors (which could repeat a pointer)
        # while the key that names them is cached.
        self._plan = None

    def forward(self, q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor) -> torch.Tensor:
        # Steady state (the Ascend ModelNew's fast path binds its launch after the third call
        # with the same input pointers, src/task1_sparse_attn.py:751-755,789-801): the same
        # pointers, shapes, dtypes, sink and stream as the last call reuse its checked and
        # marshalled launch; only the fresh output is allocated. Anything else (including an
        # in-place update of attn_sink, which moves its version counter) prepares anew.
        dev = q.device
        if dev.type == _native.PLAN_DEVICE_TYPE and q.is_contiguous() and kv.is_contiguous() and topk_idxs.is_contiguous():
            sink = self.attn_sink
            key = (q.data_ptr(), kv.data_ptr(), topk_idxs.data_ptr(), q.shape, kv.shape, topk_idxs.shape,
                   q.dtype, kv.dtype, topk_idxs.dtype, sink.data_ptr(), sink._version,
                   _native.stream_handle(dev), self.variant, self.v_dim)
            plan = self._plan
            if plan is None or plan[0] != key:
                plan = self._plan = (key, self._prepare(q, kv, topk_idxs))
            return plan[1].run()
        return self._prepare(q, kv, topk_idxs).run()

    def _prepare(self, q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor) -> "_native.Prepared":
        if q.dim() != 4 or q.shape[2] != self.n_heads or q.shape[3] != self.head_dim:
            raise ValueError(f"q {tuple(q.shape)} does not match n_heads={self.n_heads}, "
                             f"head_dim={self.head_dim}")
        if self.v_dim is not None and self.v_dim != self.head_dim:
            return _native.prepare_sparse_mla(q, kv, topk_idxs, self.attn_sink, self.softmax_scale, self.v_dim)
        return _native.prepare_sparse_attn(q, kv, topk_idxs, self.attn_sink, self.softmax_scale, self.variant)


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


def get_gather_inputs(batch_size=4, seq_len=4096, n_kv=8192, topk=512, device="cuda", seed=42):
    """configs[3] (true-gather) inputs, built on `device`: q [b, m, 64, 128] and
    kv [b, n_kv, 128] bf16 ~N(0,1); token t selects min(t+1, topk) distinct rows of
    the causally visible range [0, t] in random order, the remaining slots are -1
    (the reference's masked marker, task1_v0_ref.py:8)."""
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(batch_size, seq_len, n_heads, head_dim, generator=g, device=device).to(torch.bfloat16)
    kv = torch.randn(batch_size, n_kv, head_dim, generator=g, device=device).to(torch.bfloat16)
    idx = torch.empty(batch_size, seq_len, topk, dtype=torch.int32, device=device)
    cols = torch.arange(n_kv, device=device)
    step = 256
    for t0 in range(0, seq_len, step):
        t = torch.arange(t0, min(seq_len, t0 + step), device=device)
        sc = torch.rand(batch_size, len(t), n_kv, generator=g, device=device)
        sc = sc.masked_fill(cols[None, None, :] > t[None, :, None], -1.0)
        val, ix = sc.topk(topk, dim=-1)
        idx[:, t0:t0 + len(t)] = torch.where(val >= 0, ix, torch.full_like(ix, -1)).to(torch.int32)
    return [q, kv, idx]


def get_mla_inputs(seq_len=8192, n_heads_mla=128, d_qk=576, topk=2048, device="cuda", seed=42):
    """configs[4] sparse-MLA inputs, built on `device`: q [1, m, 128, 576] and the latent
    kv [1, m, 576] bf16 ~N(0,1); token t selects min(t+1, topk) distinct rows of [0, t]
    (the causal top-k the indexer hands over), remaining slots -1."""
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(1, seq_len, n_heads_mla, d_qk, generator=g, device=device).to(torch.bfloat16)
    kv = torch.randn(1, seq_len, d_qk, generator=g, device=device).to(torch.bfloat16)
    idx = torch.empty(1, seq_len, topk, dtype=torch.int32, device=device)
    cols = torch.arange(seq_len, device=device)
    for t0 in range(0, seq_len, 256):
        t = torch.arange(t0, min(seq_len, t0 + 256), device=device)
        sc = torch.rand(1, len(t), seq_len, generator=g, device=device)
        sc = sc.masked_fill(cols[None, None, :] > t[None, :, None], -1.0)
        val, ix = sc.topk(topk, dim=-1)
        idx[:, t0:t0 + len(t)] = torch.where(val >= 0, ix, torch.full_like(ix, -1)).to(torch.int32)
    return [q, kv, idx]
