"""Task2 oracle: the lightning indexer.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

indexer_forward  follows Model.forward of reference/task2_v0_ref.py:123-144 op for op
                 (F.linear, in-place RoPE on the q view, scaled weights, bf16 einsum,
                 relu_ * w, head sum, additive -inf mask, topk, -1/offset fill). The only
                 change is that the two mask aranges are created on x.device instead
                 of with .cuda(), so the same code runs on the CPU and on the GPU.
                 On the GPU it is the reference path the kernel must equal bit for bit.
                 Pinned by: tests/golden/task2_*.npz, written by importing the reference
                 on CPU (exact equality of the int64 output and of the constructor's
                 weights), and stage-wise by oracle/rules.py (RoPE rounding, bf16
                 rounding of the weights, head-sum order, top-k tie order, mask/fill).
apply_rotary_emb task2_v0_ref.py:93-104 (forward direction, the only one the path uses).
IndexerRef       constructor with the reference's parameter creation order (:106-121),
                 so torch.manual_seed(s) gives the reference's weights.
make_args / get_inputs / get_init_inputs  task2_v0_ref.py:147-172 with a device argument.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn


@dataclass
class IndexerArgs:
    """The ModelArgs fields the indexer reads (task2_v0_ref.py:21-61)."""
    max_batch_size: int = 4
    max_seq_len: int = 4096
    dim: int = 4096
    q_lora_rank: int = 1024
    rope_head_dim: int = 64
    index_n_heads: int = 64
    index_head_dim: int = 128
    index_topk: int = 512


def make_args() -> IndexerArgs:
    """Contest configuration (task2_v0_ref.py:147-150)."""
    return IndexerArgs(max_batch_size=8, max_seq_len=2600, dim=1024, index_n_heads=16,
                       index_head_dim=64, index_topk=128, q_lora_rank=256, rope_head_dim=32)


def _bf16_param(out_f: int, in_f: int) -> nn.Parameter:
    """task2_v0_ref.py:65-71: empty bf16 weight, kaiming_uniform_(a=sqrt(5))."""
    w = nn.Parameter(torch.empty(out_f, in_f, dtype=torch.bfloat16))
    nn.init.kaiming_uniform_(w, a=math.sqrt(5))
    return w


class IndexerRef(nn.Module):
    """Reference parameter layout: wq_b.weight then weights_proj.weight (task2_v0_ref.py:116-117)."""

    def __init__(self, args, freqs_cis, kv_cache, compress_ratio: int = 4):
        super().__init__()
        self.n_heads = args.index_n_heads
        self.head_dim = args.index_head_dim
        self.rope_head_dim = args.rope_head_dim
        self.index_topk = args.index_topk
        self.wq_b = nn.Module()
        self.wq_b.weight = _bf16_param(self.n_heads * self.head_dim, args.q_lora_rank)
        self.weights_proj = nn.Module()
        self.weights_proj.weight = _bf16_param(self.n_heads, args.dim)
        self.compress_ratio = compress_ratio
        self.kv_cache = kv_cache
        self.freqs_cis = freqs_cis
        self.einsum_rows = None  # see index_scores

    def forward(self, x, qr, start_pos: int, offset: int):
        return indexer_forward(self.wq_b.weight, self.weights_proj.weight, self.kv_cache,
                               self.freqs_cis, x, qr, start_pos, offset, self.n_heads,
                               self.head_dim, self.rope_head_dim, self.index_topk,
                               self.compress_ratio, self.einsum_rows)


def apply_rotary_emb(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    """task2_v0_ref.py:93-104: rotate pairs of x in place (through its float copy)."""
    y = x
    xc = torch.view_as_complex(x.float().unflatten(-1, (-1, 2)))
    shape = (1, xc.size(1), xc.size(-1)) if xc.ndim == 3 else (1, xc.size(1), 1, xc.size(-1))
    y.copy_(torch.view_as_real(xc * freqs_cis.view(*shape)).flatten(-2))
    return y


def index_scores(wq, ww, kv_cache, freqs_cis, x, qr, start_pos, n_heads, head_dim, rope_head_dim,
                 ratio, einsum_rows=None) -> torch.Tensor:
    """task2_v0_ref.py:124-137: the bf16 [b, s, T] score after the mask.

    einsum_rows: when set, the einsum of :133 runs on at most that many tokens of one
    batch at a time. Every output is still one fp32 dot product over head_dim rounded
    once to bf16; what changes is the GEMM algorithm torch-ROCm picks for the call, and
    with it the fp32 summation order over head_dim, which differs between algorithms
    for a few products in a billion (measured on the MI355X)."""
    bsz, seqlen, _ = x.size()
    fc = freqs_cis[start_pos:start_pos + seqlen]                               # :125
    end_pos = start_pos + seqlen                                               # :128
    q = F.linear(qr, wq).unflatten(-1, (n_heads, head_dim))                    # :129-130
    apply_rotary_emb(q[..., -rope_head_dim:], fc)                              # :131
    w = F.linear(x, ww) * (head_dim ** -0.5 * n_heads ** -0.5)                 # :132
    kv = kv_cache[:bsz, :end_pos // ratio]
    if einsum_rows is None:
        score = torch.einsum("bshd,btd->bsht", q, kv)                          # :133
    else:
        score = torch.cat([torch.cat([torch.einsum("bshd,btd->bsht", q[i:i + 1, c:c + einsum_rows], kv[i:i + 1])
                                      for c in range(0, seqlen, einsum_rows)], dim=1)
                           for i in range(bsz)])
    score = (score.relu_() * w.unsqueeze(-1)).sum(dim=2)                       # :134
    if start_pos == 0:                                                         # :135-137
        dev = x.device
        cols = torch.arange(seqlen // ratio, device=dev).repeat(seqlen, 1)
        lim = torch.arange(1, seqlen + 1, device=dev).unsqueeze(1) // ratio
        score += torch.where(cols >= lim, float("-inf"), 0)
    return score


def select_topk(score: torch.Tensor, start_pos: int, offset: int, index_topk: int,
                ratio: int) -> torch.Tensor:
    """task2_v0_ref.py:138-143: top-k indices, then -1 for masked picks / + offset."""
    seqlen = score.size(1)
    end_pos = start_pos + seqlen
    idx = score.topk(min(index_topk, end_pos // ratio), dim=-1)[1]            # :138
    if start_pos == 0:                                                         # :139-141
        lim = torch.arange(1, seqlen + 1, device=score.device).unsqueeze(1) // ratio
        idx = torch.where(idx >= lim, -1, idx + offset)
    else:                                                                      # :142-143
        idx += offset
    return idx


def indexer_forward(wq, ww, kv_cache, freqs_cis, x, qr, start_pos, offset, n_heads, head_dim,
                    rope_head_dim, index_topk, ratio, einsum_rows=None) -> torch.Tensor:
    """task2_v0_ref.py:123-144 (einsum_rows: as in index_scores)."""
    score = index_scores(wq, ww, kv_cache, freqs_cis, x, qr, start_pos, n_heads, head_dim,
                         rope_head_dim, ratio, einsum_rows)
    return select_topk(score, start_pos, offset, index_topk, ratio)


def precompute_freqs_cis(rope_head_dim, max_seq_len, theta=10000.0, device="cpu"):
    """task2_v0_ref.py:166-170."""
    freqs = 1.0 / (theta ** (torch.arange(0, rope_head_dim, 2)[: rope_head_dim // 2].float() / rope_head_dim))
    t = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.outer(t, freqs).float().to(device)
    return torch.polar(torch.ones_like(freqs), freqs).view(max_seq_len, -1)


def get_inputs(args=None, batch_size=8, seq_len=2600, device="cpu"):
    """task2_v0_ref.py:152-160."""
    a = args or make_args()
    x = torch.randn(batch_size, seq_len, a.dim, dtype=torch.bfloat16).to(device)
    qr = torch.randn(batch_size, seq_len, a.q_lora_rank, dtype=torch.bfloat16).to(device)
    return [x, qr, 0, 0]


def get_init_inputs(args=None, compress_ratio=4, device="cpu"):
    """task2_v0_ref.py:162-172."""
    a = args or make_args()
    freqs_cis = precompute_freqs_cis(a.rope_head_dim, a.max_seq_len, 10000.0, device)
    kv_cache = torch.randn(a.max_batch_size, a.max_seq_len // compress_ratio, a.index_head_dim,
                           dtype=torch.bfloat16).to(device)
    return [a, freqs_cis, kv_cache, compress_ratio]
