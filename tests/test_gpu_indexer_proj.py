"""The query projection with RoPE (dsa_indexer_q_proj) against torch on the MI355X.

F.linear (task2_v0_ref.py:129-130, via Linear.forward :81-83) of bf16 inputs on
torch-ROCm, then apply_rotary_emb (:131) on the bf16 q in torch-ROCm's rounding: the
kernel, which accumulates over k in ascending order with matrix-core products, gives
the same bits at the indexer's shapes (configs[2]: k = 256, n = 16 x 64; configs[4]:
k = 1536, n = 64 x 128) for the token counts below. For a few small token counts
hipBLASLt picks an algorithm that reduces k in another order; there the two differ by
one bf16 rounding of two fp32 sums taken in different orders, which the second test
bounds.
"""
import numpy as np
import pytest
import torch

from conftest import bits_of
from ascendc_kernel_amd import _native
from oracle import indexer as oix
from oracle import rules

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _case(k, n, d, rd, b, m, seed, dev):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    qr = torch.randn(b, m, k, generator=g).to(torch.bfloat16).to(dev)
    fr = oix.precompute_freqs_cis(rd, m, device=dev)
    ref = torch.nn.functional.linear(qr, w)
    ref_rope = ref.clone().unflatten(-1, (n // d, d))
    oix.apply_rotary_emb(ref_rope[..., -rd:], fr)
    return w, qr, fr, ref.unflatten(-1, (n // d, d)), ref_rope


SHAPES = {"c3": (256, 1024, 64, 32), "c5": (1536, 8192, 128, 64)}
# The configs[2] class (k = 256) is what Model.forward routes through the kernel from 64
# tokens up (task2_indexer.Model._q_proj_fused), so its token counts are swept densely.
EQUAL = [("c3", 8, 2600), ("c3", 1, 8), ("c3", 1, 64), ("c3", 1, 65), ("c3", 1, 96), ("c3", 3, 100),
         ("c3", 1, 129), ("c3", 1, 255), ("c3", 1, 640), ("c3", 2, 1000), ("c3", 1, 2048), ("c3", 4, 2600),
         ("c3", 1, 5000), ("c3", 3, 7777), ("c3", 1, 8192), ("c3", 8, 4096), ("c3", 16, 2600),
         ("c5", 1, 8192), ("c5", 1, 64), ("c5", 1, 1000), ("c5", 1, 4096), ("c5", 2, 200)]


@pytest.mark.parametrize("shape,b,m", EQUAL)
def test_q_proj_equals_f_linear_and_rope(gpu, shape, b, m):
    k, n, d, rd = SHAPES[shape]
    w, qr, fr, ref, ref_rope = _case(k, n, d, rd, b, m, 7 + m, gpu)
    _say("q_proj", shape, b, m)
    got = _native.indexer_q_proj(qr, w, None, d, rd)
    got_rope = _native.indexer_q_proj(qr, w, fr, d, rd)
    for name, x, y in (("F.linear", got, ref), ("F.linear + RoPE", got_rope, ref_rope)):
        ne = int((x.view(torch.int16) != y.view(torch.int16)).sum())
        assert ne == 0, f"{name}: {ne} of {y.numel()} outputs differ"


@pytest.mark.parametrize("shape", ["c3", "c5"])
def test_q_proj_small_token_counts(gpu, shape):
    """Token counts 1..16: where hipBLASLt reduces k in another order, an output may differ
    from F.linear by one bf16 rounding step plus what fp32 summation in any order can move
    the sum: |a - r| <= ulp_bf16(max(|a|, |r|)) + 2 k 2^-24 sum_i |q_i w_i| (the count of
    differing outputs is printed per m)."""
    k, n, d, rd = SHAPES[shape]
    counts = []
    for m in range(1, 17):
        w, qr, fr, ref, _ = _case(k, n, d, rd, 1, m, 100 + m, gpu)
        got = _native.indexer_q_proj(qr, w, None, d, rd)
        counts.append(int((got.view(torch.int16) != ref.view(torch.int16)).sum()))
        a, r = got.float().cpu().flatten(), ref.float().cpu().flatten()
        mag = (qr.float().abs().cpu() @ w.float().abs().cpu().T).flatten()
        big = torch.maximum(a.abs(), r.abs()).clamp_min(2.0 ** -126)
        ulp = torch.exp2(torch.floor(torch.log2(big)) - 7)
        bad = (a - r).abs() > ulp + 2 * k * 2.0 ** -24 * mag
        assert not bool(bad.any()), (m, int(bad.sum()))
    _say(f"[q_proj {shape}] outputs differing from F.linear for m = 1..16:", counts)


@pytest.mark.parametrize("b,m", [(1, 64), (2, 1000), (8, 2600)])
def test_q_proj_cpu_rope_rounding(gpu, b, m):
    """rope_mode DSA_ROPE_CPU (the CPU reference's non-FMA complex product): F.linear's q
    rotated by the oracle's CPU rule (oracle/rules.py rope 'cpu', pinned by the reference
    fixture) equals the kernel's output."""
    k, n, d, rd = SHAPES["c3"]
    w, qr, fr, ref, _ = _case(k, n, d, rd, b, m, 300 + m, gpu)
    got = _native.indexer_q_proj(qr, w, fr, d, rd, _native.DSA_ROPE_CPU)
    f = torch.view_as_real(fr).reshape(m, rd // 2, 2).cpu().numpy()
    want = rules.rope_bf16(bits_of(ref), f, rd, "cpu")
    ne = int((bits_of(got) != want).sum())
    assert ne == 0, f"{ne} of {want.size} outputs differ"
