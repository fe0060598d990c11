"""Task2 drop-in: the DeepSeek lightning indexer on MI355X.

Same surface as reference/task2_v0_ref.py: ``ModelArgs`` (:21-61), the
``Linear``/``ColumnParallelLinear`` projections (:63-91) and
``Model(args, freqs_cis, kv_cache, compress_ratio=4)`` with
``forward(x, qr, start_pos, offset) -> int64 [b, s, min(index_topk, end_pos//ratio)]``
(:106-144), plus ``get_inputs()``/``get_init_inputs()`` (:147-172). The
constructor creates ``wq_b`` then ``weights_proj`` with the same initialisers,
so a seeded construction yields the reference's weights.

forward = two torch projections (``F.linear``, the reference's own op) and one
gfx950 kernel that applies RoPE, the score, the relu-weighted head sum, the
causal mask and the top-k (``dsa_indexer_score_topk``). Inputs must be on the
HIP device; unsupported configurations raise.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Literal, Tuple

import torch
import torch.nn.functional as F
from torch import nn

from . import _native

world_size = 1
rank = 0
block_size = 128
fp4_block_size = 32


@dataclass
class ModelArgs:
    """Configuration record with the reference's fields and defaults (task2_v0_ref.py:21-61)."""
    max_batch_size: int = 4
    max_seq_len: int = 4096
    dtype: Literal["bf16", "fp8"] = "fp8"
    scale_fmt: Literal[None, "ue8m0"] = "ue8m0"
    expert_dtype: Literal[None, "fp4"] = None
    scale_dtype: Literal["fp32", "fp8"] = "fp8"
    vocab_size: int = 129280
    dim: int = 4096
    moe_inter_dim: int = 4096
    n_layers: int = 7
    n_hash_layers: int = 0
    n_mtp_layers: int = 1
    n_heads: int = 64
    n_routed_experts: int = 8
    n_shared_experts: int = 1
    n_activated_experts: int = 2
    score_func: Literal["softmax", "sigmoid", "sqrtsoftplus"] = "sqrtsoftplus"
    route_scale: float = 1.
    swiglu_limit: float = 0.
    q_lora_rank: int = 1024
    head_dim: int = 512
    rope_head_dim: int = 64
    norm_eps: float = 1e-6
    o_groups: int = 8
    o_lora_rank: int = 1024
    window_size: int = 128
    compress_ratios: Tuple[int] = (0, 0, 4, 128, 4, 128, 4, 0)
    compress_rope_theta: float = 40000.0
    original_seq_len: int = 0
    rope_theta: float = 10000.0
    rope_factor: float = 40
    beta_fast: int = 32
    beta_slow: int = 1
    index_n_heads: int = 64
    index_head_dim: int = 128
    index_topk: int = 512
    hc_mult: int = 4
    hc_sinkhorn_iters: int = 20
    hc_eps: float = 1e-6


class Linear(nn.Module):
    """Bias-free bf16 projection with the reference's initialisation (task2_v0_ref.py:63-83)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=dtype or torch.bfloat16))
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        self.register_parameter("scale", None)
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features))
            bound = 1 / math.sqrt(in_features)
            nn.init.uniform_(self.bias, -bound, bound)
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.bias is not None:
            raise NotImplementedError("the indexer projections carry no bias")
        return F.linear(x, self.weight)


class ColumnParallelLinear(Linear):
    """Single-rank column-parallel projection (task2_v0_ref.py:85-91)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype=None):
        assert out_features % world_size == 0
        self.part_out_features = out_features // world_size
        super().__init__(in_features, self.part_out_features, bias, dtype)


class Model(nn.Module):
    """Drop-in for ``Model`` of reference/task2_v0_ref.py:106-144."""

    #: which torch rounding of the RoPE complex product to reproduce
    rope_mode: int = _native.DSA_ROPE_TORCH_ROCM

    def __init__(self, args: ModelArgs, freqs_cis: torch.Tensor, kv_cache: torch.Tensor,
                 compress_ratio: int = 4):
        super().__init__()
        self.dim = args.dim
        self.n_heads = args.index_n_heads
        self.n_local_heads = args.index_n_heads // world_size
        self.head_dim = args.index_head_dim
        self.rope_head_dim = args.rope_head_dim
        self.index_topk = args.index_topk
        self.q_lora_rank = args.q_lora_rank
        self.wq_b = ColumnParallelLinear(self.q_lora_rank, self.n_heads * self.head_dim)
        self.weights_proj = ColumnParallelLinear(self.dim, self.n_heads, dtype=torch.bfloat16)
        self.softmax_scale = self.head_dim ** -0.5
        self.compress_ratio = compress_ratio
        self.kv_cache = kv_cache
        self.freqs_cis = freqs_cis

    def forward(self, x: torch.Tensor, qr: torch.Tensor, start_pos: int, offset: int) -> torch.Tensor:
        bsz, seqlen, _ = x.size()
        ratio = self.compress_ratio
        end_pos = start_pos + seqlen
        n_cand = end_pos // ratio
        k_out = min(self.index_topk, n_cand)
        if k_out <= 0:
            return torch.empty(bsz, seqlen, 0, dtype=torch.int64, device=x.device)
        freqs = self.freqs_cis[start_pos:end_pos]
        if self._q_proj_fused(qr):
            # q = RoPE(qr . wq_b^T) in one kernel, bit-equal to F.linear + apply_rotary_emb
            # (task2_v0_ref.py:129-131) for this shape class.
            q = _native.indexer_q_proj(qr, self.wq_b.weight, freqs, self.head_dim, self.rope_head_dim,
                                       self.rope_mode)
            freqs = None
        else:
            q = self.wq_b(qr).unflatten(-1, (self.n_local_heads, self.head_dim))
        wl = self.weights_proj(x)
        w_scale = self.softmax_scale * self.n_heads ** -0.5
        return _native.indexer_score_topk(
            q, self.kv_cache, wl, w_scale, freqs, self.rope_head_dim,
            n_cand, k_out, ratio, start_pos == 0, offset, self.rope_mode)

    #: smallest token count (b * s) for which the fused query projection is used
    Q_PROJ_MIN_TOKENS = 64

    def _q_proj_fused(self, qr: torch.Tensor) -> bool:
        """Whether q comes from dsa_indexer_q_proj instead of F.linear + RoPE in the score
        kernel: q_lora_rank 256, rope_head_dim 32, bf16, at least 64 tokens. There the
        kernel's natural-order k accumulation equals torch-ROCm's F.linear bit for bit
        (tests/test_gpu_indexer_proj.py sweeps the token count); below 64 tokens hipBLASLt
        switches to algorithms that reduce k in another order, so F.linear stays."""
        w = self.wq_b.weight
        return (qr.is_cuda and qr.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
                and qr.shape[-1] == 256 and self.rope_head_dim == 32
                and w.shape[0] % 256 == 0 and self.head_dim in (64, 128)
                and qr.shape[0] * qr.shape[1] >= self.Q_PROJ_MIN_TOKENS)


ModelNew = Model


def _make_args() -> ModelArgs:
    """Contest configuration (task2_v0_ref.py:147-150)."""
    return ModelArgs(max_batch_size=8, max_seq_len=2600, dim=1024, index_n_heads=16,
                     index_head_dim=64, index_topk=128, q_lora_rank=256, rope_head_dim=32)


def get_inputs(device: str = "cuda"):
    """Benchmark inputs of task2_v0_ref.py:152-160."""
    a = _make_args()
    batch_size = 8
    seq_len = 2600
    x = torch.randn(batch_size, seq_len, a.dim, dtype=torch.bfloat16).to(device)
    qr = torch.randn(batch_size, seq_len, a.q_lora_rank, dtype=torch.bfloat16).to(device)
    return [x, qr, 0, 0]


def precompute_freqs_cis(rope_head_dim: int, max_seq_len: int, theta: float = 10000.0,
                         device: str = "cuda") -> torch.Tensor:
    """RoPE table as built in task2_v0_ref.py:166-170 (angles on `device`, polar there)."""
    freqs = 1.0 / (theta ** (torch.arange(0, rope_head_dim, 2)[: rope_head_dim // 2].float() / rope_head_dim))
    t = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.outer(t, freqs).float().to(device)
    return torch.polar(torch.ones_like(freqs), freqs).view(max_seq_len, -1)


def get_init_inputs(device: str = "cuda"):
    """Constructor inputs of task2_v0_ref.py:162-172."""
    a = _make_args()
    compress_ratio = 4
    freqs_cis = precompute_freqs_cis(a.rope_head_dim, a.max_seq_len, 10000.0, device)
    kv_cache = torch.randn(a.max_batch_size, a.max_seq_len // compress_ratio, a.index_head_dim,
                           dtype=torch.bfloat16).to(device)
    return [a, freqs_cis, kv_cache, compress_ratio]


# ---------------------------------------------------------------- the DSA layer indexer
def c5_args() -> ModelArgs:
    """configs[4] indexer: 64 heads x 128 from qr[1,8192,1536] and x[1,8192,7168], top-2048.
    rope_head_dim is not given by the config; the ModelArgs default (64) is used."""
    return ModelArgs(max_batch_size=1, max_seq_len=8192, dim=7168, index_n_heads=64,
                     index_head_dim=128, index_topk=2048, q_lora_rank=1536, rope_head_dim=64)


def get_c5_init_inputs(device: str = "cuda", compress_ratio: int = 1):
    """Constructor inputs for configs[4]: kv_cache [1, 8192, 128] bf16 ~N(0,1), ratio 1."""
    a = c5_args()
    freqs_cis = precompute_freqs_cis(a.rope_head_dim, a.max_seq_len, 10000.0, device)
    kv_cache = torch.randn(a.max_batch_size, a.max_seq_len // compress_ratio, a.index_head_dim,
                           dtype=torch.bfloat16).to(device)
    return [a, freqs_cis, kv_cache, compress_ratio]


def get_c5_inputs(device: str = "cuda"):
    """Forward inputs for configs[4]: x [1, 8192, 7168], qr [1, 8192, 1536] bf16 ~N(0,1)."""
    a = c5_args()
    x = torch.randn(1, a.max_seq_len, a.dim, dtype=torch.bfloat16).to(device)
    qr = torch.randn(1, a.max_seq_len, a.q_lora_rank, dtype=torch.bfloat16).to(device)
    return [x, qr, 0, 0]
