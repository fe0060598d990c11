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


# ---------------------------------------------------------------- both projections, one launch
def _proj2_inputs(b, m, seed, dev, dim=1024):
    g = torch.Generator().manual_seed(seed)
    wq = (torch.randn(1024, 256, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    wp = (torch.randn(16, dim, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    qr = torch.randn(b, m, 256, generator=g).to(torch.bfloat16).to(dev)
    x = torch.randn(b, m, dim, generator=g).to(torch.bfloat16).to(dev)
    return wq, wp, qr, x


def _ne(a, b):
    return int((a.view(torch.int16) != b.view(torch.int16)).sum())


def test_pack_projection_weights_layout(gpu):
    """The packed fragments are the documented permutation of the weights (include/dsa_abi.h)."""
    wq, wp, _, _ = _proj2_inputs(1, 1, 1, gpu)
    pq, pw = _native.pack_projection_weights(wq, wp)
    # wq fragment f = ((r * 2 + i) * 16 + ks) * 64 + lane: rows 64 r + 32 i + lane % 32,
    # k 16 ks + 8 (lane / 32) .. + 7
    want_q = wq.view(16, 2, 32, 16, 2, 8).permute(0, 1, 3, 4, 2, 5).reshape(1024, 256)
    # wproj fragment e = (hg * 32 + ks) * 64 + lane: row 16 hg + lane % 16, k 32 ks + 8 (lane / 16)
    want_w = wp.view(1, 16, 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(16, 1024)
    assert torch.equal(pq.view(torch.int16), want_q.contiguous().view(torch.int16))
    assert torch.equal(pw.view(torch.int16), want_w.contiguous().view(torch.int16))


@pytest.mark.parametrize("seed", [0, 1])
def test_projections_full_shape_c3(gpu, seed):
    """configs[2] (8 x 2600 tokens): q equals F.linear + apply_rotary_emb and wl equals
    F.linear (task2_v0_ref.py:129-132) bit for bit, in torch-ROCm's and the CPU's RoPE rounding."""
    b, m = 8, 2600
    wq, wp, qr, x = _proj2_inputs(b, m, 50 + seed, gpu)
    fr = oix.precompute_freqs_cis(32, m, device=gpu)
    pq, pw = _native.pack_projection_weights(wq, wp)
    _say("projections c3 seed", seed)
    q, wl = _native.indexer_projections(qr, pq, fr, x, pw, 64, 32)
    ref = torch.nn.functional.linear(qr, wq).unflatten(-1, (16, 64))
    ref_rope = ref.clone()
    oix.apply_rotary_emb(ref_rope[..., -32:], fr)
    assert _ne(q, ref_rope) == 0
    assert _ne(wl, torch.nn.functional.linear(x, wp)) == 0
    qc, _ = _native.indexer_projections(qr, pq, fr, x, pw, 64, 32, _native.DSA_ROPE_CPU)
    f = torch.view_as_real(fr).reshape(m, 16, 2).cpu().numpy()
    assert int((bits_of(qc) != rules.rope_bf16(bits_of(ref), f, 32, "cpu")).sum()) == 0
    q0, _ = _native.indexer_projections(qr, pq, None, x, pw, 64, 32)
    assert _ne(q0, ref) == 0


def test_projections_token_count_sweep(gpu):
    """The token counts at which Model.forward uses a projection kernel (task2_indexer.Q_EQUAL,
    WL_EQUAL, measured for every count on the build MEASURED_TORCH names): at every interval
    end, at every count of the one-launch range around configs[2] (16,385 .. 24,576) and at
    every 31st count of the other intervals, the one-launch kernel (where both tables hold the
    count) or the query-projection kernel (q's table only) equals F.linear (+ RoPE) bit for bit."""
    from ascendc_kernel_amd import task2_indexer as t2
    _say("torch", torch.__version__, "hip", torch.version.hip, "measured on", t2.MEASURED_TORCH)
    hi = max(t2.Q_EQUAL[-1][1], t2.WL_EQUAL[-1][1])
    ms = set(range(16385, 24577))
    for a, b in t2.Q_EQUAL:
        ms.update((a, b))
        ms.update(range(a, b + 1, 31))
    ms = sorted(m for m in ms if m >= t2.Q_PROJ_MIN_TOKENS and t2._within(m, t2.Q_EQUAL))
    wq, wp, qr, x = _proj2_inputs(1, hi, 77, gpu)
    fr = oix.precompute_freqs_cis(32, hi, device=gpu)
    pq, pw = _native.pack_projection_weights(wq, wp)
    bad, n_both = [], 0
    for m in ms:
        xs, qs = x[:, :m], qr[:, :m]
        ref = torch.nn.functional.linear(qs, wq).unflatten(-1, (16, 64))
        oix.apply_rotary_emb(ref[..., -32:], fr[:m])
        if t2._within(m, t2.WL_EQUAL):
            n_both += 1
            q, wl = _native.indexer_projections(qs, pq, fr, xs, pw, 64, 32)
            if _ne(wl, torch.nn.functional.linear(xs, wp)) or _ne(q, ref):
                bad.append(m)
        elif _ne(_native.indexer_q_proj(qs, wq, fr, 64, 32), ref):
            bad.append(m)
    _say(f"[projections sweep] {len(ms)} token counts ({n_both} one-launch); differing at {bad[:20]}")
    assert not bad


@pytest.mark.parametrize("b,m", [(1, 16385), (3, 5601), (2, 10007), (5, 4099), (1, 65498), (1, 17), (3, 13)])
def test_projections_ragged_token_counts(gpu, b, m):
    """Token counts that are not multiples of the 16-token chains or 32-token tiles, several
    batches (the RoPE position is the token's index within its sequence)."""
    wq, wp, qr, x = _proj2_inputs(b, m, 90 + m, gpu)
    fr = oix.precompute_freqs_cis(32, m, device=gpu)
    pq, pw = _native.pack_projection_weights(wq, wp)
    q, wl = _native.indexer_projections(qr, pq, fr, x, pw, 64, 32)
    ref = torch.nn.functional.linear(qr, wq).unflatten(-1, (16, 64))
    oix.apply_rotary_emb(ref[..., -32:], fr)
    assert _ne(q, ref) == 0
    assert _ne(wl, torch.nn.functional.linear(x, wp)) == 0 or b * m < 16385


@pytest.mark.parametrize("b,m", [(1, 100000), (1, 131072), (4, 20000), (2, 33333), (1, 512), (7, 777)])
def test_q_proj_more_token_counts(gpu, b, m):
    """dsa_indexer_q_proj at counts of task2_indexer.Q_EQUAL up to its top, 131,072 tokens."""
    k, n, d, rd = SHAPES["c3"]
    w, qr, fr, ref, ref_rope = _case(k, n, d, rd, b, m, 11 + m, gpu)
    got = _native.indexer_q_proj(qr, w, fr, d, rd)
    assert _ne(got, ref_rope) == 0
