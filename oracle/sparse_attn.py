"""Task1 oracle: sparse attention with attention sink.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

sparse_attn_ref  follows reference/task1_v0_ref.py:5-24 op for op (fp32 einsums on
                 the gathered rows, sink in the denominator, bf16 output). Device
                 agnostic: on a GPU it is the "reference PyTorch path on the same GPU".
                 Pinned by: tests/golden/task1_*.npz written by importing the reference
                 (exact on CPU), and by the closed forms in tests/test_oracle_sparse_attn.py
                 (all slots masked -> 0; q = 0 -> uniform weights incl. the sink; all
                 slots equal -> closed form; slot-permutation invariance; fp64 brute force).
sparse_attn_fp64 independent per-row fp64 loop (small shapes only), used to pin the above.
v_dim            sparse-MLA extension of both (keys = kv[..., :d_qk], values = kv[..., :v_dim]);
                 pinned by the fp64 loop and by reducing to the reference when v_dim = d.
Model / get_inputs / get_init_inputs  restate task1_v0_ref.py:27-55.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn


def sparse_attn_ref(q, kv, attn_sink, topk_idxs, softmax_scale, v_dim=None):
    """reference/task1_v0_ref.py:5-24. v_dim (an extension for sparse MLA; None = the
    reference): the scores use kv[..., :d] with d = q's width, the output sums
    kv[..., :v_dim] (the reference is v_dim = d = kv's width)."""
    b, m, h, _ = q.shape
    k = topk_idxs.shape[-1]
    keep = topk_idxs >= 0                                                  # :8
    rows = kv[torch.arange(b, device=q.device)[:, None, None].expand(b, m, k),
              topk_idxs.clamp(min=0).long()]                               # :9-11
    rows = rows.masked_fill(~keep.unsqueeze(-1), 0.0)                      # :12
    d = q.shape[-1]
    krows = rows if rows.shape[-1] == d else rows[..., :d]
    vrows = rows if v_dim is None else rows[..., :v_dim]
    logits = torch.einsum("bmhd,bmtd->bmht", q.float(), krows.float()) * softmax_scale  # :13
    logits = logits.masked_fill(~keep.unsqueeze(2), float("-inf"))         # :14
    sink = attn_sink.float().view(1, 1, h, 1)                              # :15
    top = torch.maximum(torch.amax(logits, dim=-1, keepdim=True), sink)    # :16-17
    ex = torch.exp(logits - top).masked_fill(~keep.unsqueeze(2), 0.0)      # :18-19
    denom = ex.sum(dim=-1, keepdim=True) + torch.exp(sink - top)           # :20-21
    out = torch.einsum("bmht,bmtd->bmhd", ex / denom, vrows.float())       # :22-23
    return out.to(q.dtype)                                                 # :24


def sparse_attn_fp64(q, kv, attn_sink, topk_idxs, softmax_scale, v_dim=None) -> np.ndarray:
    """Independent fp64 statement of the same maths, one (b, m, h) row at a time."""
    qn = q.double().cpu().numpy()
    kvn = kv.double().cpu().numpy()
    kn = kvn[..., :qn.shape[-1]]
    vn = kvn if v_dim is None else kvn[..., :v_dim]
    idx = topk_idxs.cpu().numpy()
    sink = attn_sink.double().cpu().numpy()
    b, m, h, _ = qn.shape
    dv = vn.shape[-1]
    out = np.zeros((b, m, h, dv))
    for bi in range(b):
        for mi in range(m):
            sel = [int(j) for j in idx[bi, mi] if j >= 0]
            for hi in range(h):
                s = [float(np.dot(qn[bi, mi, hi], kn[bi, j])) * softmax_scale for j in sel]
                mx = max(s + [sink[hi]])
                e = [np.exp(v - mx) for v in s]
                z = sum(e) + np.exp(sink[hi] - mx)
                acc = np.zeros(dv)
                for w, j in zip(e, sel):
                    acc += (w / z) * vn[bi, j]
                out[bi, mi, hi] = acc
    return out


class Model(nn.Module):
    """reference/task1_v0_ref.py:27-36."""

    def __init__(self, n_heads: int, head_dim: int):
        super().__init__()
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.softmax_scale = head_dim ** -0.5
        self.attn_sink = nn.Parameter(torch.zeros(n_heads, dtype=torch.float32))

    def forward(self, q, kv, topk_idxs):
        return sparse_attn_ref(q, kv, self.attn_sink, topk_idxs, self.softmax_scale)


def get_inputs(batch_size=8, seq_len=2600, n_kv=32, n_heads=64, head_dim=128, topk=16):
    """reference/task1_v0_ref.py:47-51 (same RNG calls in the same order)."""
    q = torch.randn(batch_size, seq_len, n_heads, head_dim, dtype=torch.bfloat16)
    kv = torch.randn(batch_size, n_kv, head_dim, dtype=torch.bfloat16)
    idx = torch.randint(0, n_kv, (batch_size, seq_len, topk), dtype=torch.int32)
    return [q, kv, idx]


def get_init_inputs(n_heads=64, head_dim=128):
    return [n_heads, head_dim]


def gather_inputs(b, m, h, d, n_kv, topk, generator=None, device="cpu"):
    """configs[3]-style inputs: token t selects min(t+1, topk) distinct rows of [0, t]
    (random order), remaining slots -1 (the reference's masked marker)."""
    q = torch.randn(b, m, h, d, generator=generator).to(torch.bfloat16).to(device)
    kv = torch.randn(b, n_kv, d, generator=generator).to(torch.bfloat16).to(device)
    idx = torch.empty(b, m, topk, dtype=torch.int32)
    cols = torch.arange(n_kv)
    for t0 in range(0, m, 256):
        t = torch.arange(t0, min(m, t0 + 256))
        sc = torch.rand(b, len(t), n_kv, generator=generator)
        sc = sc.masked_fill(cols[None, None, :] > t[None, :, None], -1.0)
        val, ix = sc.topk(topk, dim=-1)
        idx[:, t0:t0 + len(t)] = torch.where(val >= 0, ix, torch.full_like(ix, -1)).to(torch.int32)
    return q, kv, idx.to(device)
