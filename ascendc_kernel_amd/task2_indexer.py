"""Task2 drop-in: the DeepSeek lightning indexer on MI355X.

Same surface as reference/task2_v0_ref.py: ``ModelArgs`` (:21-61), the
``Linear``/``ColumnParallelLinear`` projections (:63-91) and
``Model(args, freqs_cis, kv_cache, compress_ratio=4)`` with
``forward(x, qr, start_pos, offset) -> int64 [b, s, min(index_topk, end_pos//ratio)]``
(:106-144), plus ``get_inputs()``/``get_init_inputs()`` (:147-172). The
constructor creates ``wq_b`` then ``weights_proj`` with the same initialisers,
so a seeded construction yields the reference's weights.

forward = the two projections, then one gfx950 kernel for the score, the
relu-weighted head sum, the causal mask and the top-k (``dsa_indexer_score_topk``).
The projections run as one kernel launch (``dsa_indexer_projections``: q with RoPE,
and the head weights), as the query-projection kernel beside ``F.linear``, as one
decode launch for 1..16 tokens (``dsa_indexer_decode_projections``, both products in
hipBLASLt's split-k order; the score kernel applies RoPE), or as two ``F.linear`` (the
reference's own op; the score kernel then applies RoPE), whichever ``projection_route``
picks: a kernel only where its rounding was measured equal to ``F.linear`` on this
torch-ROCm build. Inputs must be on the HIP device;
unsupported configurations raise.
"""
from __future__ import annotations

import bisect
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


#: The torch-ROCm build (torch.__version__, torch.version.hip) and CU count on which the
#: projection kernels' rounding was measured against F.linear (hipBLASLt chooses its
#: algorithm, and with it the order in which it sums k, by build, shape and CU count); on
#: anything else Model.forward keeps F.linear.
MEASURED_TORCH = ("2.10.0+rocm7.0", "7.0.51831")
MEASURED_CUS = 256
#: Token counts m = b * s (maximal intervals, inclusive) where F.linear equals the kernels'
#: natural-order k accumulation bit for bit on that build, measured for every m from 17 to
#: 131,072 on at least 2^18 outputs of each product by tests/golden/measure_projection_ranges.py
#: (tests/golden/projection_ranges.json): wq_b (k = 256, 1024 outputs) and weights_proj
#: (k = 1024, 16 outputs). Between the intervals hipBLASLt splits the k sum (over wave groups,
#: or stream-K tails); for weights_proj below 15,361 tokens that changes ~1.7e-4 of the outputs.
Q_EQUAL = (
    (17, 32768), (33153, 34304), (34433, 35456), (35585, 36608), (36737, 52096), (52225, 65664),
    (65793, 65920), (66433, 67584), (67713, 68736), (68865, 69888), (70017, 71040), (71169, 73344),
    (73473, 81920), (82049, 82176), (82433, 82560), (82817, 83328), (83457, 83712), (83841, 86144),
    (86273, 86528), (86657, 87552), (87681, 87936), (88065, 98304), (98433, 98560), (99329, 100608),
    (100737, 100992), (101121, 101888), (102017, 102272), (102401, 102656), (102785, 103936),
    (104065, 104320), (104449, 105216), (105345, 105984), (106113, 114688), (115073, 115200),
    (115585, 115712), (115841, 117504), (117633, 118016), (118145, 118528), (118657, 119040),
    (119169, 119424), (119553, 119936), (120065, 120448), (120577, 120960), (121089, 121344),
    (121473, 121856), (121985, 122368), (122497, 131072),
)
WL_EQUAL = (
    (15361, 15517), (15617, 15772), (15873, 16026), (16129, 16281), (16385, 65536),
    (65793, 66048), (66305, 66560), (66817, 67072), (67329, 67584), (67841, 68096), (68353, 68608),
    (68865, 69120), (69377, 69632), (69889, 70144), (70401, 70656), (70913, 71168), (71425, 71680),
    (71937, 72192), (72449, 72704), (72961, 73216), (73473, 73728), (73985, 74240), (74497, 74752),
    (75009, 75264), (75521, 75776), (76033, 76288), (76545, 76800), (77057, 77824), (78081, 78336),
    (78593, 131072),
)
#: smallest token count sent to the query-projection kernel (below it F.linear + the score
#: kernel's own RoPE is as fast)
Q_PROJ_MIN_TOKENS = 64
#: Decode (1..16 tokens) at the DeepSeek-V3.2 sizes (q_lora_rank, n_heads * head_dim, dim,
#: n_heads): there hipBLASLt runs both products with k split over 4 waves, the order
#: dsa_indexer_decode_projections reproduces (measured for every token count 1..16 on that
#: build, tests/test_gpu_decode_proj.py).
DECODE_MAX_TOKENS = 16
DECODE_SHAPE = (1536, 8192, 7168, 64)

_build_ok: dict = {}


def _measured_build(dev: torch.device) -> bool:
    ok = _build_ok.get(dev.index)
    if ok is None:
        ok = ((torch.__version__, torch.version.hip) == MEASURED_TORCH
              and torch.cuda.get_device_properties(dev).multi_processor_count == MEASURED_CUS)
        _build_ok[dev.index] = ok
    return ok


def _within(m: int, table) -> bool:
    i = bisect.bisect_right(table, (m, float("inf"))) - 1
    return i >= 0 and table[i][0] <= m <= table[i][1]


def projection_route(m: int, q_lora_rank: int, rope_head_dim: int, head_dim: int, n_q: int, dim: int,
                     n_w: int, bf16: bool, on_gpu: bool, build_ok: bool) -> str:
    """Which path computes the two projections of Model.forward for m = b * s tokens:
    'both'  one launch of dsa_indexer_projections (q with RoPE, and weights_proj);
    'q'     dsa_indexer_q_proj for q with RoPE, F.linear for weights_proj;
    'decode' one launch of dsa_indexer_decode_projections for both (no RoPE: the score
            kernel applies it);
    'torch' F.linear for both (the score kernel then applies RoPE).
    A kernel is used only where its rounding was measured equal to F.linear."""
    if not (bf16 and on_gpu and build_ok):
        return "torch"
    if 1 <= m <= DECODE_MAX_TOKENS and (q_lora_rank, n_q, dim, n_w) == DECODE_SHAPE:
        return "decode"
    if not (q_lora_rank == 256 and rope_head_dim == 32 and n_q % 256 == 0 and head_dim in (64, 128)
            and m >= Q_PROJ_MIN_TOKENS and _within(m, Q_EQUAL)):
        return "torch"
    if head_dim == 64 and dim == 1024 and n_w == 16 and _within(m, WL_EQUAL):
        return "both"
    return "q"


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
        # The last call's launch plan, and the fragment-packed projection weights with the
        # (pointer, version) pairs they were packed from. Plans hold their inputs, so their
        # memory cannot be reused for other tensors (which could repeat a pointer) while the
        # key that names them is cached.
        self._plan = None
        self._packed = None

    def route(self, x: torch.Tensor, qr: torch.Tensor) -> str:
        """projection_route for these inputs ('both', 'q', 'decode' or 'torch')."""
        wq, wp = self.wq_b.weight, self.weights_proj.weight
        return projection_route(
            qr.shape[0] * qr.shape[1], qr.shape[-1], self.rope_head_dim, self.head_dim, wq.shape[0], x.shape[-1],
            wp.shape[0], qr.dtype == x.dtype == wq.dtype == wp.dtype == torch.bfloat16,
            qr.is_cuda and x.is_cuda, qr.is_cuda and _measured_build(qr.device))

    def forward(self, x: torch.Tensor, qr: torch.Tensor, start_pos: int, offset: int) -> torch.Tensor:
        # Steady state (the Ascend ModelNew binds a no-argument launch of the whole forward
        # after the third call with the same pointers, src/task2_indexer.py:1069-1072,
        # 1340-1348): the same inputs, positions, weights (pointer and version), cache, table
        # and stream as the last call reuse its plan; only the fresh output is allocated.
        dev = x.device
        wq, wp, kv, fc = self.wq_b.weight, self.weights_proj.weight, self.kv_cache, self.freqs_cis
        # (A plan reads kv_cache and freqs_cis in place, so it sees their updates; it is kept
        # only where neither needs a contiguous copy, which would not.)
        if (dev.type == _native.PLAN_DEVICE_TYPE and x.is_contiguous() and qr.is_contiguous() and kv.dim() == 3
                and kv.stride(2) == 1 and kv.stride(1) == kv.shape[2] and fc.is_contiguous()):
            key = (x.data_ptr(), qr.data_ptr(), x.shape, qr.shape, x.dtype, qr.dtype, start_pos, offset,
                   wq.data_ptr(), wq._version, wp.data_ptr(), wp._version, kv.data_ptr(), kv.shape,
                   kv.stride(), fc.data_ptr(), fc.shape, _native.stream_handle(dev), self.rope_mode,
                   self.compress_ratio, self.index_topk)
            plan = self._plan
            if plan is None or plan.key != key:
                plan = self._plan = _IndexerPlan(self, x, qr, start_pos, offset, key)
            return plan.run()
        return _IndexerPlan(self, x, qr, start_pos, offset, None).run()

    def packed_weights(self):
        """(wq_b, weights_proj) in dsa_indexer_projections' fragment order, packed once per
        weight version (an in-place update moves a parameter's version counter; writes
        through .data do not, so after those call refresh_packed_weights())."""
        wq, wp = self.wq_b.weight, self.weights_proj.weight
        tag = (wq.data_ptr(), wq._version, wp.data_ptr(), wp._version)
        if self._packed is None or self._packed[0] != tag:
            self._packed = (tag, _native.pack_projection_weights(wq, wp))
        return self._packed[1]

    def refresh_packed_weights(self) -> None:
        """Drops the packed weights and the cached plan (after writes through .data)."""
        self._packed = None
        self._plan = None

    def _q_proj_fused(self, qr: torch.Tensor) -> bool:
        """Whether q comes from a projection kernel (dsa_indexer_q_proj or
        dsa_indexer_projections) rather than F.linear + RoPE in the score kernel."""
        wq, wp = self.wq_b.weight, self.weights_proj.weight
        return projection_route(
            qr.shape[0] * qr.shape[1], qr.shape[-1], self.rope_head_dim, self.head_dim, wq.shape[0], self.dim,
            wp.shape[0], qr.dtype == wq.dtype == torch.bfloat16, qr.is_cuda,
            qr.is_cuda and _measured_build(qr.device)) in ("both", "q")


class _IndexerPlan:
    """Everything Model.forward launches for one set of inputs, prepared once. Intermediate q
    and wl buffers of the kernel paths are kept and reused by later calls of the plan: the
    plan is keyed on the stream, and on one stream a call's projections start only after
    the previous call's score kernel has read them."""

    def __init__(self, model: Model, x: torch.Tensor, qr: torch.Tensor, start_pos: int, offset: int, key):
        self.key = key
        bsz, seqlen, _ = x.size()
        ratio = model.compress_ratio
        end_pos = start_pos + seqlen
        n_cand = end_pos // ratio
        k_out = min(model.index_topk, n_cand)
        self.empty = (bsz, seqlen) if k_out <= 0 else None
        self.device = x.device
        if self.empty is not None:
            return
        self.x, self.qr = x, qr
        self.wq, self.wp = model.wq_b.weight, model.weights_proj.weight
        freqs = model.freqs_cis[start_pos:end_pos]
        w_scale = model.softmax_scale * model.n_heads ** -0.5
        hd, rd, mode = model.head_dim, model.rope_head_dim, model.rope_mode
        self.route = model.route(x, qr)
        kv = model.kv_cache
        score_kw = dict(rope_head_dim=rd, n_cand=n_cand, k_out=k_out, ratio=ratio, causal=start_pos == 0,
                        offset=offset, rope_mode=mode)
        self.proj = None
        if self.route == "both":
            # q = RoPE(qr . wq_b^T) and wl = x . weights_proj^T in one launch
            # (task2_v0_ref.py:129-132), bit-equal to F.linear + apply_rotary_emb here.
            wq_p, wp_p = model.packed_weights()
            self.proj, q_shape, wl_shape, self.proj_keep = _native.prepare_indexer_projections(
                qr, wq_p, freqs, x, wp_p, hd, rd, mode)
            self.q = torch.empty(q_shape, dtype=torch.bfloat16, device=x.device)
            self.wl = torch.empty(wl_shape, dtype=torch.bfloat16, device=x.device)
            self.proj.set(_native.PROJ_SLOT_Q, self.q.data_ptr())
            self.proj.set(_native.PROJ_SLOT_WL, self.wl.data_ptr())
            self.score = _native.prepare_indexer_score_topk(self.q, kv, self.wl, w_scale, None, **score_kw)
        elif self.route == "decode":
            # q = qr . wq_b^T and wl = x . weights_proj^T in one launch, in hipBLASLt's
            # rounding at decode sizes (task2_v0_ref.py:129,132); RoPE in the score kernel.
            self.proj, _q_shape, wl_shape, self.proj_keep = _native.prepare_indexer_decode_projections(
                qr, self.wq, x, self.wp)
            self.q = torch.empty(bsz, seqlen, model.n_local_heads, hd, dtype=torch.bfloat16, device=x.device)
            self.wl = torch.empty(wl_shape, dtype=torch.bfloat16, device=x.device)
            self.proj.set(_native.DECODE_SLOT_Q, self.q.data_ptr())
            self.proj.set(_native.DECODE_SLOT_WL, self.wl.data_ptr())
            self.score = _native.prepare_indexer_score_topk(self.q, kv, self.wl, w_scale, freqs, **score_kw)
        elif self.route == "q":
            # q = RoPE(qr . wq_b^T) by dsa_indexer_q_proj; weights_proj stays F.linear.
            prep = _native.prepare_indexer_q_proj(qr, self.wq, freqs, hd, rd, mode)
            self.q = torch.empty(prep.out_shape, dtype=torch.bfloat16, device=x.device)
            prep.launch.set(prep.out_slot, self.q.data_ptr())
            self.proj, self.proj_keep = prep.launch, prep.keep
            wl0 = torch.empty(bsz, seqlen, model.n_heads, dtype=torch.bfloat16, device=x.device)
            self.score = _native.prepare_indexer_score_topk(self.q, kv, wl0, w_scale, None, **score_kw)
        else:
            # F.linear for both (task2_v0_ref.py:129-132); the score kernel applies RoPE.
            self.heads = (model.n_local_heads, hd)
            q0 = torch.empty(bsz, seqlen, model.n_local_heads, hd, dtype=torch.bfloat16, device=x.device)
            wl0 = torch.empty(bsz, seqlen, model.n_heads, dtype=torch.bfloat16, device=x.device)
            self.score = _native.prepare_indexer_score_topk(q0, kv, wl0, w_scale, freqs, **score_kw)

    def run(self) -> torch.Tensor:
        if self.empty is not None:
            return torch.empty(*self.empty, 0, dtype=torch.int64, device=self.device)
        launch = self.score.launch
        if self.route == "both" or self.route == "decode":
            self.proj()
        elif self.route == "q":
            self.proj()
            wl = F.linear(self.x, self.wp)
            launch.set(_native.SCORE_SLOT_WL, wl.data_ptr())
        else:
            q = F.linear(self.qr, self.wq).unflatten(-1, self.heads)
            wl = F.linear(self.x, self.wp)
            launch.set(_native.SCORE_SLOT_Q, q.data_ptr())
            launch.set(_native.SCORE_SLOT_WL, wl.data_ptr())
        # (The fresh q / wl tensors of the torch paths are released when this returns; the
        # caching allocator hands their memory only to later work on this stream.)
        return self.score.run()


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
