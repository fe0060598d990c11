"""Task2 parity on the MI355X.

1. torch-ROCm itself against the numpy rules (pins the oracle's behaviour on this GPU).
2. The RoPE kernel against torch's apply_rotary_emb on the same GPU (bit-exact).
3. The fused score/top-k kernel (through the drop-in Model and the C ABI) against
   the oracle run on the same GPU: int64 indices torch.equal, tie order included.
"""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, bf16_from_bits, bits_of
from ascendc_kernel_amd import _native
from ascendc_kernel_amd import task2_indexer as t2
from oracle import indexer as oix
from oracle import rules

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


# ---------------------------------------------------------------- torch-ROCm rules
def test_torch_rope_rule(gpu):
    g = torch.Generator().manual_seed(0)
    q = torch.randn(8, 2600, 16, 64, generator=g).to(torch.bfloat16)
    fr = oix.precompute_freqs_cis(32, 2600, device=gpu)
    _say("rule rope torch-rocm")
    qg = q.to(gpu)
    oix.apply_rotary_emb(qg[..., -32:], fr)
    want = rules.rope_bf16(bits_of(q), torch.view_as_real(fr).cpu().numpy(), 32, "torch_rocm")
    got = bits_of(qg)
    assert np.array_equal(got, want), int((got != want).sum())


def test_torch_head_sum_rule(gpu):
    g = torch.Generator().manual_seed(1)
    shape = (8, 2600, 16, 650)
    sgn = torch.randint(0, 2, shape, generator=g, dtype=torch.int32)
    ex = torch.randint(115, 139, shape, generator=g, dtype=torch.int32)
    mn = torch.randint(0, 128, shape, generator=g, dtype=torch.int32)
    x = ((sgn << 15) | (ex << 7) | mn).to(torch.int16).view(torch.bfloat16)
    _say("rule head-sum")
    got = bits_of(x.to(gpu).sum(dim=2))
    xs = bits_of(x[:1, :200])
    want = rules.bf16_round(rules.head_sum(np.moveaxis(rules.bf16_to_f32(xs), 2, -1), "rocm"))
    assert np.array_equal(got[:1, :200], want)


@pytest.mark.parametrize("k", [1, 2, 9, 16, 31, 32, 33, 64, 128, 200])
def test_torch_topk_rule(gpu, k):
    """torch-ROCm topk(sorted=True) order = rules.topk_torch (gather order, then the 32-slot
    bitonic network for k <= 32, a stable value sort above), -inf tails included."""
    g = torch.Generator().manual_seed(2 + k)
    rows = 1500 if k <= 32 else 3000
    x = torch.randint(-8, 8, (rows, 650), generator=g).to(torch.bfloat16)
    n_r = torch.randint(0, 651, (rows,), generator=g)
    x = x.masked_fill(torch.arange(650)[None, :] >= n_r[:, None], float("-inf"))
    _say("rule topk", k)
    got = x.to(gpu).topk(k, dim=-1)[1].cpu().numpy()
    want = rules.topk_torch(bits_of(x), k)
    bad = np.nonzero((got != want).any(axis=1))[0]
    if len(bad):
        r = int(bad[0])
        _say("row", r, "n_r", int(n_r[r]), "got", got[r][:40].tolist(), "want", want[r][:40].tolist())
    assert len(bad) == 0, len(bad)


def test_torch_weights_rule(gpu):
    g = torch.Generator().manual_seed(3)
    wl = torch.randn(1 << 16, generator=g).to(torch.bfloat16)
    for scale in (64 ** -0.5 * 16 ** -0.5, 128 ** -0.5 * 64 ** -0.5):
        assert np.array_equal(bits_of(wl.to(gpu) * scale), rules.weights_bits(bits_of(wl), scale))


# ---------------------------------------------------------------- RoPE kernel
@pytest.mark.parametrize("shape,rd", [((8, 2600, 16, 64), 32), ((2, 37, 16, 64), 32),
                                      ((1, 100, 4, 128), 64), ((3, 5, 16, 64), 64)])
def test_rope_kernel_matches_torch(gpu, shape, rd):
    g = torch.Generator().manual_seed(4)
    q = torch.randn(*shape, generator=g).to(torch.bfloat16).to(gpu)
    fr = oix.precompute_freqs_cis(rd, shape[1] + 7, device=gpu)[7:]
    _say("rope kernel", shape, rd)
    ref = q.clone()
    oix.apply_rotary_emb(ref[..., -rd:], fr)
    got = q.clone()
    _native.indexer_rope_(got, fr, rd, _native.DSA_ROPE_TORCH_ROCM)
    assert torch.equal(got, ref), int((got != ref).sum())


def test_rope_kernel_cpu_mode_matches_reference_fixture(gpu):
    f = np.load(os.path.join(GOLDEN, "task2_small.npz"))
    q = bf16_from_bits(f["rope_in"]).to(gpu)
    fr = torch.view_as_complex(torch.from_numpy(f["freqs"]).contiguous()).to(gpu)[:64]
    _say("rope kernel cpu mode")
    _native.indexer_rope_(q, fr, 32, _native.DSA_ROPE_CPU)
    assert np.array_equal(bits_of(q), f["rope_out"])


# ---------------------------------------------------------------- fused kernel
def _pair(args, seed, batch, kv_rows, device):
    torch.manual_seed(seed)
    fr = oix.precompute_freqs_cis(args.rope_head_dim, args.max_seq_len, device=device)
    kv = torch.randn(batch, kv_rows, args.index_head_dim, dtype=torch.bfloat16).to(device)
    torch.manual_seed(seed + 1)
    m = t2.Model(args, fr, kv, 4).to(device)
    r = oix.IndexerRef(args, fr, kv, 4).to(device)
    r.wq_b.weight.data.copy_(m.wq_b.weight.data)
    r.weights_proj.weight.data.copy_(m.weights_proj.weight.data)
    return m, r


def _check_equal(got, want, name):
    eq = torch.equal(got, want)
    if not eq:
        rows = (got != want).any(dim=-1)
        _say(f"[{name}] mismatching rows {int(rows.sum())} of {rows.numel()}")
    assert eq, name


def test_torch_score_einsum_sums_head_dim_in_order(gpu):
    """The premise of the bit-exact configs[2] parity: torch-ROCm's score einsum
    (task2_v0_ref.py:133) at [8, 2600, 16, 64] x [8, 650, 64] gives the same bits as the
    same einsum taken 128 tokens of one batch at a time (small GEMMs, which sum head_dim
    in ascending order, as the score kernel's chained MFMAs do). A torch or ROCm build
    whose GEMM algorithm for this shape sums in another order fails here first."""
    g = torch.Generator(device=gpu).manual_seed(7)
    q = torch.randn(8, 2600, 16, 64, device=gpu, generator=g).to(torch.bfloat16)
    kv = torch.randn(8, 650, 64, device=gpu, generator=g).to(torch.bfloat16)
    whole = torch.einsum("bshd,btd->bsht", q, kv)
    parts = torch.cat([torch.cat([torch.einsum("bshd,btd->bsht", q[i:i + 1, c:c + 128], kv[i:i + 1])
                                  for c in range(0, 2600, 128)], dim=1) for i in range(8)])
    n = int((whole.view(torch.int16) != parts.view(torch.int16)).sum())
    _say("score einsum products in another order:", n, "of", whole.numel(), torch.__version__, torch.version.hip)
    assert n == 0


@pytest.mark.parametrize("seeds", [(42, 5, 43), (1, 11, 12), (2, 21, 22)])
def test_full_shape_c3(gpu, seeds):
    """x[8,2600,1024], qr[8,2600,256], kv_cache[8,650,64], W ~ N(0, 0.02);
    seeds = (kv_cache / constructor, weights, inputs)."""
    ctor_seed, w_seed, in_seed = seeds
    args = t2._make_args()
    m, r = _pair(args, ctor_seed, 8, 650, gpu)
    g = torch.Generator().manual_seed(w_seed)
    with torch.no_grad():
        for p in (m.wq_b.weight, m.weights_proj.weight):
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16))
    r.wq_b.weight.data.copy_(m.wq_b.weight.data)
    r.weights_proj.weight.data.copy_(m.weights_proj.weight.data)
    torch.manual_seed(in_seed)
    x, qr, sp, off = t2.get_inputs(device=gpu)
    _say("case c3 full shape", seeds)
    got = m(x, qr, sp, off)
    want = r(x, qr, sp, off)
    torch.cuda.synchronize()
    _check_equal(got, want, "c3")
    assert torch.equal(got, m(x, qr, sp, off))


def test_reference_init_weights_c3(gpu):
    """Weights from the constructor (kaiming uniform), as get_init_inputs + Model give them."""
    args = t2._make_args()
    m, r = _pair(args, 7, 8, 650, gpu)
    torch.manual_seed(8)
    x, qr, _, _ = t2.get_inputs(device=gpu)
    _say("case c3 ctor weights")
    _check_equal(m(x, qr, 0, 0), r(x, qr, 0, 0), "c3-ctor")


SMALL = [
    # batch, seqlen, start_pos, offset, index_topk, kv_rows
    (2, 256, 0, 0, 32, 64),
    (1, 37, 0, 3, 128, 650),
    (3, 400, 0, 0, 128, 650),
    (2, 600, 0, -5, 64, 650),
    (2, 64, 64, 7, 32, 650),
    (1, 129, 300, 11, 128, 650),
    (4, 1000, 0, 0, 256, 650),
    (1, 2600, 0, 0, 128, 700),
    # decode at the configs[2] size: one new token per batch at the end of the
    # 2600-token context (no mask, +offset), and a 40-token chunk before it
    (8, 1, 2599, 5, 128, 650),
    (8, 40, 2560, 0, 128, 650),
    # either side of the fused query projection's 64-token gate, and 65 tokens of
    # 13-token sequences (the projection's 32-token tiles span several batches)
    (1, 63, 1500, 2, 128, 650),
    (1, 64, 1500, 2, 128, 650),
    (5, 13, 100, 0, 32, 650),
    # either side of the one-launch projections' lower end (16,385 tokens), inside the
    # range with other batch splits, a mid-sequence chunk, and near its upper end (65,498)
    # (the 16-head score kernel takes up to 2048 candidates: end_pos // 4 <= 2048)
    (2, 8192, 0, 0, 128, 2048),
    (5, 3277, 0, 1, 128, 820),
    (5, 3333, 0, 0, 64, 834),
    (4, 5000, 2000, 4, 128, 1750),
    (8, 8187, 0, 0, 32, 2047),
    # offsets beyond int32 (the output is int64: index + offset, -1 where masked)
    (2, 300, 0, (1 << 33) + 5, 64, 650),
    (1, 20, 500, -(1 << 40), 32, 650),
]


@pytest.mark.parametrize("keys", ["spread30", "equal", "equal_but_8"])
@pytest.mark.parametrize("start_pos,seqlen", [(2536, 64), (0, 600)])
def test_select_key_spreads(gpu, keys, start_pos, seqlen):
    """The 16-head kernel's selection with key rows scaled by 2^e per candidate (scores
    over many binades of both signs), with every key row equal (all valid candidates tie:
    the picks are decided by the index alone) and with all rows equal but 8 (ties at the
    k-th key). Without the mask (start_pos > 0, 650 candidates) and causal (start_pos 0,
    masked candidates filled with -1)."""
    batch, topk, kv_rows = 2, 128, 650
    args = oix.IndexerArgs(max_batch_size=batch, max_seq_len=2600, dim=1024, q_lora_rank=256,
                           rope_head_dim=32, index_n_heads=16, index_head_dim=64, index_topk=topk)
    m, r = _pair(args, 300 + seqlen, batch, kv_rows, gpu)
    g = torch.Generator().manual_seed(301)
    with torch.no_grad():
        if keys == "spread30":
            e = torch.randint(-30, 31, (kv_rows,), generator=g).float()
            m.kv_cache.mul_(torch.exp2(e).to(gpu)[None, :, None].to(torch.bfloat16))
        else:
            keep = m.kv_cache[:, :8].clone()
            m.kv_cache.copy_(m.kv_cache[:, 8:9].clone().expand_as(m.kv_cache))
            if keys == "equal_but_8":
                sel = torch.randperm(kv_rows, generator=g)[:8].to(gpu)
                m.kv_cache[:, sel] = keep
    assert m.kv_cache is r.kv_cache
    x = torch.randn(batch, seqlen, 1024, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(batch, seqlen, 256, generator=g).to(torch.bfloat16).to(gpu)
    _say("select key spread", keys, start_pos, seqlen)
    _check_equal(m(x, qr, start_pos, 2), r(x, qr, start_pos, 2), f"spread-{keys}-{start_pos}")


def test_noncontiguous_inputs(gpu):
    """x and qr as transposed views and a kv_cache with a padded row stride (the reference
    accepts any strides): the drop-in Model takes the unplanned path and gives the same
    indices as the reference and as its contiguous inputs."""
    batch, seqlen, topk = 2, 300, 64
    args = oix.IndexerArgs(max_batch_size=batch, max_seq_len=2600, dim=1024, q_lora_rank=256,
                           rope_head_dim=32, index_n_heads=16, index_head_dim=64, index_topk=topk)
    m, r = _pair(args, 401, batch, 650, gpu)
    g = torch.Generator().manual_seed(402)
    x = torch.randn(batch, 1024, seqlen, generator=g).to(torch.bfloat16).to(gpu).transpose(1, 2)
    qr = torch.randn(batch, 256, seqlen, generator=g).to(torch.bfloat16).to(gpu).transpose(1, 2)
    assert not x.is_contiguous() and not qr.is_contiguous()
    _say("case non-contiguous x, qr")
    want = r(x, qr, 0, 1)
    _check_equal(m(x, qr, 0, 1), want, "noncontig")
    _check_equal(m(x.contiguous(), qr.contiguous(), 0, 1), want, "noncontig-copy")
    # kv_cache rows with a stride of 96 elements (64 used)
    kvp = torch.zeros(batch, 650, 96, dtype=torch.bfloat16, device=gpu)
    kvp[..., :64] = m.kv_cache
    m.kv_cache = kvp[..., :64]
    r.kv_cache = kvp[..., :64]
    _check_equal(m(x, qr, 0, 1), r(x, qr, 0, 1), "noncontig-kv")


@pytest.mark.parametrize("case", SMALL)
def test_shapes_and_modes(gpu, case):
    batch, seqlen, start_pos, offset, topk, kv_rows = case
    args = oix.IndexerArgs(max_batch_size=batch, max_seq_len=max(2600, start_pos + seqlen), dim=1024,
                           q_lora_rank=256, rope_head_dim=32, index_n_heads=16,
                           index_head_dim=64, index_topk=topk)
    m, r = _pair(args, 100 + seqlen, batch, kv_rows, gpu)
    g = torch.Generator().manual_seed(seqlen)
    x = torch.randn(batch, seqlen, 1024, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(batch, seqlen, 256, generator=g).to(torch.bfloat16).to(gpu)
    _say("case", case)
    _check_equal(m(x, qr, start_pos, offset), r(x, qr, start_pos, offset), f"case{case}")


def test_separate_rope_equals_fused(gpu):
    args = t2._make_args()
    m, _ = _pair(args, 9, 2, 650, gpu)
    g = torch.Generator().manual_seed(10)
    x = torch.randn(2, 300, 1024, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(2, 300, 256, generator=g).to(torch.bfloat16).to(gpu)
    _say("case separate rope")
    q = torch.nn.functional.linear(qr, m.wq_b.weight).unflatten(-1, (16, 64)).contiguous()
    wl = torch.nn.functional.linear(x, m.weights_proj.weight)
    fused = _native.indexer_score_topk(q, m.kv_cache, wl, 64 ** -0.5 * 16 ** -0.5, m.freqs_cis[:300],
                                       32, 75, 75, 4, True, 0)
    _native.indexer_rope_(q, m.freqs_cis[:300], 32)
    sep = _native.indexer_score_topk(q, m.kv_cache, wl, 64 ** -0.5 * 16 ** -0.5, None, 32, 75, 75, 4,
                                     True, 0)
    assert torch.equal(fused, sep)


def test_reference_fixture_cpu_rounding(gpu):
    """Reference fixture (computed by the reference on the CPU): the kernel gets the CPU
    projections and the CPU RoPE rounding. Its rows may still differ from the fixture for
    two reasons only, and every differing row must be one of them:
      ties   the picks differ only among candidates whose reference score equals the row's
             k-th score (the CPU's topk order of equal values is not stable), or
      device the reference's CPU score and the kernel's score (torch-ROCm's GEMM and
             head-sum order) differ on a candidate the two picks disagree on.
    The kernel's indices are also exactly torch-ROCm's top-k of its own scores."""
    f = np.load(os.path.join(GOLDEN, "task2_small.npz"))
    wq, ww = bf16_from_bits(f["wq"]), bf16_from_bits(f["ww"])
    x, qr = bf16_from_bits(f["x"]), bf16_from_bits(f["qr"])
    q = torch.nn.functional.linear(qr, wq).unflatten(-1, (16, 64)).contiguous()
    wl = torch.nn.functional.linear(x, ww)
    fr = torch.view_as_complex(torch.from_numpy(f["freqs"]).contiguous())
    kv = bf16_from_bits(f["kv"])
    scale, k, n_cand = 64 ** -0.5 * 16 ** -0.5, 32, 64
    _say("case reference fixture")
    got = _native.indexer_score_topk(q.to(gpu), kv.to(gpu), wl.to(gpu), scale, fr.to(gpu)[:256], 32,
                                     n_cand, k, 4, True, 0, _native.DSA_ROPE_CPU).cpu().numpy().reshape(-1, k)
    s_dev = bits_of(_native.indexer_scores(q.to(gpu), kv.to(gpu), wl.to(gpu), scale, fr.to(gpu)[:256], 32,
                                           n_cand, 4, True, _native.DSA_ROPE_CPU)).reshape(-1, n_cand)
    # the reference's own scores: the oracle on the CPU (equal to the reference there)
    s_ref = bits_of(oix.index_scores(wq, ww, kv, fr, x, qr, 0, 16, 64, 32, 4)).reshape(-1, n_cand)
    want = f["out0"].reshape(-1, k)
    t = np.tile(np.arange(256), 2)
    n_r = np.minimum((t + 1) // 4, n_cand)
    assert np.array_equal(got, rules.fill(rules.topk_torch(s_dev, k), n_r, True, 0))
    key_ref = rules.order_key(s_ref).astype(np.int64)
    n_tie = n_dev = 0
    for r in np.nonzero((got != want).any(axis=1))[0]:
        g_ok, w_ok = got[r][got[r] >= 0], want[r][want[r] >= 0]
        assert len(g_ok) == len(w_ok), r
        kg, kw = np.sort(key_ref[r][g_ok])[::-1], np.sort(key_ref[r][w_ok])[::-1]
        if np.array_equal(kg, kw) and np.all(np.diff(key_ref[r][g_ok]) <= 0):
            n_tie += 1
            continue
        # candidates in contention: at or above the k-th score on either device
        key_dev = rules.order_key(s_dev[r]).astype(np.int64)
        kth_ref = np.sort(key_ref[r])[::-1][k - 1]
        kth_dev = np.sort(key_dev)[::-1][k - 1]
        top = (key_ref[r] >= kth_ref) | (key_dev >= kth_dev)
        assert ((s_dev[r] != s_ref[r]) & top).any(), f"row {r}: picks differ beyond ties with equal scores"
        n_dev += 1
    same_rows = float((got == want).all(axis=1).mean())
    _say(f"fixture: rows equal {same_rows:.4f}; differing rows: {n_tie} ties at the k-th score, "
         f"{n_dev} with CPU/GPU score differences ({int((s_dev != s_ref).sum())} of {s_ref.size} scores differ)")


@pytest.mark.parametrize("seqlen,start_pos", [(2600, 0), (301, 0), (64, 64), (120, 0)])
def test_score_stage_matches_torch(gpu, seqlen, start_pos):
    """The bf16 index_score the kernel ranks equals torch's on the same GPU, bit for bit."""
    args = t2._make_args()
    m, r = _pair(args, 21, 2, 650, gpu)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(2, seqlen, 1024, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(2, seqlen, 256, generator=g).to(torch.bfloat16).to(gpu)
    end = start_pos + seqlen
    n_cand = end // 4
    _say("score stage", seqlen, start_pos)
    want = oix.index_scores(r.wq_b.weight, r.weights_proj.weight, r.kv_cache, r.freqs_cis, x, qr,
                            start_pos, 16, 64, 32, 4)
    q = torch.nn.functional.linear(qr, m.wq_b.weight).unflatten(-1, (16, 64)).contiguous()
    wl = torch.nn.functional.linear(x, m.weights_proj.weight)
    got = _native.indexer_scores(q, m.kv_cache, wl, 64 ** -0.5 * 16 ** -0.5, m.freqs_cis[start_pos:end],
                                 32, n_cand, 4, start_pos == 0)
    gb, wb = bits_of(got), bits_of(want)
    ne = gb != wb
    if ne.any():
        i = np.argwhere(ne)[:8]
        _say("first mismatches (b,t,k, got, want):", [(tuple(int(v) for v in ii), hex(gb[tuple(ii)]), hex(wb[tuple(ii)])) for ii in i])
        # which candidates / heads: pattern summary
        _say("mismatch fraction", ne.mean(), "by k%32:", np.bincount(np.argwhere(ne)[:, 2] % 32, minlength=32).tolist())
    assert not ne.any(), int(ne.sum())
    # the kernel's top-k, given these (equal) scores, equals the rule
    k = min(128, n_cand)
    idx = _native.indexer_score_topk(q, m.kv_cache, wl, 64 ** -0.5 * 16 ** -0.5, m.freqs_cis[start_pos:end],
                                     32, n_cand, k, 4, start_pos == 0, 0).cpu().numpy()
    rows = gb.reshape(-1, n_cand)
    t = np.tile(np.arange(seqlen), 2)
    n_r = np.minimum((t + 1) // 4, n_cand) if start_pos == 0 else np.full(t.shape, n_cand)
    want_idx = rules.fill(rules.topk_torch(rows, k), n_r, start_pos == 0, 0)
    bad = (idx.reshape(-1, k) != want_idx).any(axis=1)
    if bad.any():
        r0 = int(np.argwhere(bad)[0][0])
        _say("first bad row", r0, "n_r", int(n_r[r0]), "got", idx.reshape(-1, k)[r0][:16].tolist(),
             "want", want_idx[r0][:16].tolist())
    assert not bad.any(), int(bad.sum())


@pytest.mark.parametrize("start_pos,seqlen,k", [(2536, 64, 128), (2536, 64, 32), (0, 2600, 128)])
def test_score_stage_nonfinite(gpu, start_pos, seqlen, k):
    """Scores that overflow to +-inf (about a quarter of the candidates carry an inf head):
    the kernel's bf16 score and its top-k equal torch's on the same GPU. With the causal
    mask (start_pos 0) only the unmasked scores are compared: the reference adds -inf to
    a masked +inf score, which gives NaN and ranks that masked candidate first (then
    filled with -1); the kernel counts masked candidates as -inf without scoring them, so
    its picks differ from the reference's on such rows. NaN scores are not covered: the
    kernel's packed relu maps a NaN with the sign bit set (the matrix cores' NaN) to 0
    where torch.relu keeps it."""
    args = t2._make_args()
    m, r = _pair(args, 31, 2, 650, gpu)
    g = torch.Generator().manual_seed(32)
    x = torch.randn(2, seqlen, 1024, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(2, seqlen, 256, generator=g).to(torch.bfloat16).to(gpu)
    wq = m.wq_b.weight.detach().clone()
    # channel 0 of heads 3 and 10 becomes -+3e38 on even tokens (rope leaves channel 0
    # alone), so q . k overflows to +-inf wherever |k_0| > ~1.13
    wq[3 * 64, 0] = 1e19
    wq[10 * 64, 0] = -1e19
    qr[:, 0::2, 0] = 3e19
    kv = m.kv_cache.detach().clone()
    end = start_pos + seqlen
    n_cand = end // 4
    causal = start_pos == 0
    _say("score stage non-finite", start_pos, seqlen, k)
    want = oix.index_scores(wq, m.weights_proj.weight, kv, m.freqs_cis, x, qr, start_pos, 16, 64, 32, 4)
    q = torch.nn.functional.linear(qr, wq).unflatten(-1, (16, 64)).contiguous()
    wl = torch.nn.functional.linear(x, m.weights_proj.weight)
    scale = 64 ** -0.5 * 16 ** -0.5
    fr = m.freqs_cis[start_pos:end]
    got = _native.indexer_scores(q, kv, wl, scale, fr, 32, n_cand, 4, causal)
    gb, wb = bits_of(got).reshape(-1, n_cand), bits_of(want).reshape(-1, n_cand)
    t = np.tile(np.arange(seqlen), 2)
    n_r = np.minimum((t + 1) // 4, n_cand) if causal else np.full(t.shape, n_cand)
    valid = np.arange(n_cand)[None, :] < n_r[:, None]
    g_nan = (gb & 0x7FFF) > 0x7F80
    w_nan = (wb & 0x7FFF) > 0x7F80
    n_inf = int((((wb & 0x7FFF) == 0x7F80) & valid).sum())
    _say(f"inf scores {n_inf}, NaN scores {int((w_nan & valid).sum())} of {int(valid.sum())}")
    assert n_inf > 1000 and not (w_nan & valid).any()
    same = (gb == wb) | (g_nan & w_nan)
    assert same[valid].all(), int((~same[valid]).sum())
    if causal:
        return
    idx = _native.indexer_score_topk(q, kv, wl, scale, fr, 32, n_cand, k, 4, False, 0).cpu().numpy()
    want_idx = oix.select_topk(want, start_pos, 0, k, 4).cpu().numpy()  # torch.topk on this GPU
    bad = (idx.reshape(-1, k) != want_idx.reshape(-1, k)).any(axis=1)
    assert not bad.any(), int(bad.sum())


def test_model_launch_plan_reuse(gpu):
    """Model.forward's cached plan (one launch of both projections at configs[2]): repeated
    calls agree and return fresh tensors; new inputs, new input contents under the same
    pointers, and in-place weight updates (new packed weights) each match the oracle."""
    args = t2._make_args()
    m, r = _pair(args, 31, 8, 650, gpu)
    torch.manual_seed(32)
    x, qr, sp, off = t2.get_inputs(device=gpu)
    assert m.route(x, qr) == "both"
    a, b = m(x, qr, sp, off), m(x, qr, sp, off)
    assert a.data_ptr() != b.data_ptr()
    _check_equal(a, b, "plan repeat")
    _check_equal(b, r(x, qr, sp, off), "plan vs oracle")
    x2, qr2, _, _ = t2.get_inputs(device=gpu)
    _check_equal(m(x2, qr2, sp, off), r(x2, qr2, sp, off), "plan new inputs")
    x2.copy_(x)
    _check_equal(m(x2, qr2, sp, off), r(x2, qr2, sp, off), "plan new contents")
    g = torch.Generator().manual_seed(33)
    with torch.no_grad():
        for p in (m.wq_b.weight, m.weights_proj.weight):
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16))
    r.wq_b.weight.data.copy_(m.wq_b.weight.data)
    r.weights_proj.weight.data.copy_(m.weights_proj.weight.data)
    _check_equal(m(x2, qr2, sp, off), r(x2, qr2, sp, off), "plan new weights")
    _check_equal(m(x2, qr2, 0, 3), r(x2, qr2, 0, 3), "plan new offset")
