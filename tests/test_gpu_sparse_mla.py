"""Sparse MLA (the attention of the configs[4] DSA layer) on the MI355X, through the C ABI,
against the oracle's sparse_attn_ref with a value width (keys kv[..., :576], values
kv[..., :512]) on the same GPU. Bar: bf16 within atol 1e-2 / rtol 1e-2; the fraction of
bit-identical outputs is printed."""
import pytest
import torch

from ascendc_kernel_amd import _native
from ascendc_kernel_amd import task1_sparse_attn as t1
from ascendc_kernel_amd import task2_indexer as t2
from oracle import indexer as oix
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu

DQK, DV = 576, 512
SCALE = DQK ** -0.5


def _say(*a):
    print(*a, flush=True)


def _compare(out, ref, name, atol=1e-2, rtol=1e-2):
    o, r = out.float(), ref.float()
    diff = (o - r).abs()
    bad = diff > atol + rtol * r.abs()
    exact = (out.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    _say(f"[{name}] bit-exact {exact:.6f} max|diff| {diff.max().item():.3e} over tol {int(bad.sum())}")
    assert not bad.any(), f"{name}: {int(bad.sum())} elements outside atol={atol} rtol={rtol}"
    assert torch.isfinite(o).all()
    return exact


def _compare_all_tokens(out, q, kv, sink, idx, scale, name, chunk=256):
    """_compare over every token of out[1, M, ...] with the oracle run on `chunk` tokens at
    a time (the oracle's gathered rows for all 8192 configs[4] tokens would be ~40 GB).
    Returns the fraction of bit-identical outputs."""
    m = out.shape[1]
    n_exact, n_all = 0.0, 0
    for i in range(0, m, chunk):
        sl = slice(i, min(m, i + chunk))
        ref = osa.sparse_attn_ref(q[:, sl], kv, sink, idx[:, sl], scale, v_dim=DV)
        e = _compare(out[:, sl], ref, f"{name} tokens {sl.start}..{sl.stop - 1}")
        n_exact += e * ref.numel()
        n_all += ref.numel()
        del ref
    exact = n_exact / n_all
    _say(f"[{name}] all {m} tokens: bit-exact {exact:.6f}")
    return exact


def _case(b, m, h, n_kv, topk, seed, masked=0.0, sink_scale=0.0, kv_dim=DQK, dev="cuda"):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, h, DQK, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, n_kv, kv_dim, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, n_kv, (b, m, topk), generator=g, dtype=torch.int32)
    if masked:
        idx[torch.rand(b, m, topk, generator=g) < masked] = -1
    sink = torch.randn(h, generator=g) * sink_scale
    return q.to(dev), kv.to(dev), idx.to(dev), sink.to(dev)


CASES = [
    # b, m, h, n_kv, topk, seed, masked, sink
    (1, 24, 128, 300, 64, 1, 0.2, 1.0),
    (2, 9, 64, 100, 33, 2, 0.0, 0.0),
    (1, 5, 80, 2048, 2048, 3, 0.5, 0.5),
    (1, 6, 128, 40, 1, 4, 0.0, 2.0),
    (1, 12, 112, 500, 200, 5, 0.9, -1.0),
    (1, 7, 96, 3000, 1500, 6, 0.3, 0.5),
]


@pytest.mark.parametrize("case", CASES)
def test_mla_shapes_and_masks(gpu, case):
    b, m, h, n_kv, topk, seed, masked, sink_scale = case
    _say("mla case", case)
    q, kv, idx, sink = _case(b, m, h, n_kv, topk, seed, masked, sink_scale)
    out = _native.sparse_mla_fwd(q, kv, idx, sink, SCALE, DV)
    ref = osa.sparse_attn_ref(q, kv, sink, idx, SCALE, v_dim=DV)
    _compare(out, ref, f"mla{case}")


@pytest.mark.parametrize("qs,ks", [(16.0, 4.0), (0.0625, 1.0)])
def test_mla_large_and_flat_score_ranges(gpu, qs, ks):
    """q and the latent rows scaled by powers of two (exact in bf16): nearly one-hot
    softmax rows with the running max raised across blocks, and nearly flat ones."""
    q, kv, idx, sink = _case(1, 12, 128, 3000, 1024, 22, 0.1, 1.0)
    q, kv = (q.float() * qs).to(torch.bfloat16), (kv.float() * ks).to(torch.bfloat16)
    _say("mla score range", qs, ks)
    out = _native.sparse_mla_fwd(q, kv, idx, sink, SCALE, DV)
    ref = osa.sparse_attn_ref(q, kv, sink, idx, SCALE, v_dim=DV)
    _compare(out, ref, f"mla-range-{qs}-{ks}", atol=1e-2 * ks, rtol=1e-2)


def test_mla_masked_tokens_oob_and_wide_rows(gpu):
    """Fully masked tokens give 0; indices >= n_kv count as masked; kv rows wider than 576."""
    q, kv, idx, sink = _case(1, 6, 64, 50, 40, 6, 0.0, 1.0, kv_dim=640)
    idx[0, 1] = -1
    idx[0, 2, ::3] = 60
    _say("mla masked/oob/wide")
    out = _native.sparse_mla_fwd(q, kv, idx, sink, SCALE, DV)
    ref = osa.sparse_attn_ref(q, kv, sink, torch.where(idx >= 50, -1, idx), SCALE, v_dim=DV)
    _compare(out, ref, "mla-masked")
    assert torch.count_nonzero(out[0, 1]) == 0


def test_mla_int64_indices_read_in_kernel(gpu):
    """int64 indices (dsa_sparse_mla_fwd_i64, the indexer's dtype) give the int32 path's
    output bit for bit; values outside [0, n_kv), also beyond int32, are masked slots."""
    q, kv, idx, sink = _case(1, 10, 128, 700, 300, 8, 0.2, 0.5)
    _say("mla int64 in-kernel")
    i64 = idx.long()
    big = torch.tensor([2 ** 32 + 3, 2 ** 31, -(2 ** 32) + 5, 700, 2 ** 40 + 1],
                       dtype=torch.int64, device=gpu)
    sel = torch.rand(idx.shape, generator=torch.Generator().manual_seed(17)) < 0.2
    fill = big[torch.randint(0, len(big), idx.shape, generator=torch.Generator().manual_seed(18))]
    i64 = torch.where(sel.to(gpu), fill, i64)
    i32 = torch.where((i64 >= 0) & (i64 < 700), i64, -1).to(torch.int32)
    out64 = _native.sparse_mla_fwd(q, kv, i64, sink, SCALE, DV)
    out32 = _native.sparse_mla_fwd(q, kv, i32, sink, SCALE, DV)
    assert torch.equal(out64.view(torch.int16), out32.view(torch.int16))
    ref = osa.sparse_attn_ref(q, kv, sink, i32, SCALE, v_dim=DV)
    _compare(out64, ref, "mla-int64")


SPLIT_CASES = [
    # b, m, h, n_kv, topk, seed, masked, sink: few tokens, so the slot lists are split
    # over workgroups (dsa_sparse_mla_fwd_ws) and merged by the combine kernel
    # (the plans are for 256 CUs: ranges x head groups per token)
    (1, 1, 128, 8192, 2048, 31, 0.0, 0.0),    # decode at the configs[4] size: 32 x 4, 2 waves
    (1, 4, 128, 8192, 2048, 32, 0.1, 1.0),    # 16 x 4: 256 workgroups
    (1, 9, 128, 4000, 1024, 35, 0.05, 0.5),   # 11 x 2: 4 waves
    (2, 16, 64, 3000, 300, 33, 0.3, -1.0),    # topk not a multiple of 32; 5 x 1, 4 waves
    (1, 3, 96, 700, 2000, 34, 0.0, 2.0),      # slots beyond n_kv (and beyond int32) masked; 3 waves
    (1, 2, 64, 5000, 1500, 36, 0.2, 0.0),     # 16 x 2: 64 heads as two 2-wave groups
    (1, 17, 128, 3000, 1024, 37, 0.1, 0.0),   # 11 x 1: 8 waves
    (1, 40, 128, 2000, 512, 38, 0.0, 0.5),    # 6 x 1
    (2, 50, 64, 4000, 2048, 39, 0.05, 0.0),   # 100 tokens: 2 x 1
]


@pytest.mark.parametrize("case", SPLIT_CASES)
def test_mla_split_decode(gpu, case):
    """Split slot lists (decode): within tolerance of the oracle and of the one-pass
    kernel; a split whose whole slot range is masked contributes nothing."""
    b, m, h, n_kv, topk, seed, masked, sink_scale = case
    q, kv, idx, sink = _case(b, m, h, n_kv, topk, seed, masked, sink_scale)
    idx64 = idx.long()
    if topk == 2000:
        idx[..., 600:] = -1              # the later splits see only masked slots
        idx[..., 100:200:7] = n_kv + 5   # at or beyond n_kv: masked in the kernel
        idx[..., 250:260] = n_kv
        idx64 = idx.long()
        idx64[..., 201:300:5] = 2 ** 33 + 1   # beyond int32 (int64 entry point only)
        idx64[..., 301:320:3] = -(2 ** 40)
        idx[..., 201:300:5] = -1
        idx[..., 301:320:3] = -1
    lib = _native.load()
    assert lib.dsa_sparse_mla_workspace_bytes(b, m, h, topk) > 0, "expected a split plan"
    _say("mla split case", case)
    out = _native.sparse_mla_fwd(q, kv, idx, sink, SCALE, DV)
    one = _native.sparse_mla_fwd(q, kv, idx, sink, SCALE, DV, split=False)
    i64 = _native.sparse_mla_fwd(q, kv, idx64, sink, SCALE, DV)
    assert torch.equal(out.view(torch.int16), i64.view(torch.int16))
    ref = osa.sparse_attn_ref(q, kv, sink, torch.where(idx >= n_kv, -1, idx), SCALE, v_dim=DV)
    _compare(out, ref, f"split{case}")
    _compare(one, ref, f"one-pass{case}")
    _compare(out, one, f"split-vs-one-pass{case}")


@pytest.mark.parametrize("split", [False, True])
def test_mla_neg_inf_sink_masked_leading_block(gpu, split):
    """A -inf sink (no sink mass) with the first slot blocks fully masked: the running
    max must not produce exp2(-inf + inf) = NaN before the first valid slot. Half the
    heads get -inf, the rest a finite sink; a token with every slot masked and a -inf
    sink is NaN in the reference too and is left out."""
    b, m, h, n_kv, topk = 1, 3, 128, 4000, 2048
    q, kv, idx, sink = _case(b, m, h, n_kv, topk, 41, 0.0, 1.0)
    sink[::2] = float("-inf")
    idx[..., :96] = -1                   # blocks 0..2 of every token fully masked
    idx[0, 1, :1500] = -1                # token 1: most of its splits see only masked slots
    _say("mla -inf sink", split)
    out = _native.sparse_mla_fwd(q, kv, idx, sink, SCALE, DV, split=split)
    ref = osa.sparse_attn_ref(q, kv, sink, idx, SCALE, v_dim=DV)
    assert torch.isfinite(ref.float()).all()
    _compare(out, ref, f"mla-neg-inf-sink-split{split}")


def test_mla_drop_in_module(gpu):
    """task1 Model with v_dim: the drop-in surface routes to the MLA kernel."""
    q, kv, idx, sink = _case(1, 16, 128, 256, 128, 7, 0.1, 0.0)
    m = t1.Model(128, DQK, v_dim=DV).to(gpu)
    _say("mla module")
    out = m(q, kv, idx.long())
    ref = osa.sparse_attn_ref(q, kv, m.attn_sink, idx, m.softmax_scale, v_dim=DV)
    _compare(out, ref, "mla-module")


def test_full_shape_c5_mla(gpu):
    """configs[4] attention: q[1,8192,128,576], kv[1,8192,576], top-2048 causal picks
    (t1.get_mla_inputs). The kernel runs on the whole shape; the oracle checks all 8192
    tokens, 256 at a time."""
    _say("case c5 mla inputs")
    q, kv, idx = t1.get_mla_inputs(device=gpu)
    sink = torch.zeros(128, device=gpu)
    _say("case c5 mla kernel")
    out = _native.sparse_mla_fwd(q, kv, idx, sink, SCALE, DV)
    torch.cuda.synchronize()
    _say("case c5 mla oracle")
    exact = _compare_all_tokens(out, q, kv, sink, idx, SCALE, "c5-mla")
    assert exact > 0.97


def test_dsa_layer_indexer_then_mla(gpu):
    """The two halves chained as in the DSA layer (smaller sequence): the indexer's int64
    top-k (with -1 for masked picks) feeds the MLA kernel directly."""
    seqlen, topk = 1024, 512
    args = oix.IndexerArgs(max_batch_size=1, max_seq_len=seqlen, dim=7168, q_lora_rank=1536,
                           rope_head_dim=64, index_n_heads=64, index_head_dim=128, index_topk=topk)
    torch.manual_seed(51)
    fr = oix.precompute_freqs_cis(64, seqlen, device=gpu)
    kvc = torch.randn(1, seqlen, 128, dtype=torch.bfloat16).to(gpu)
    ix = t2.Model(args, fr, kvc, 1).to(gpu)
    g = torch.Generator().manual_seed(52)
    with torch.no_grad():
        for p in (ix.wq_b.weight, ix.weights_proj.weight):
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16))
    x = torch.randn(1, seqlen, 7168, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(1, seqlen, 1536, generator=g).to(torch.bfloat16).to(gpu)
    _say("case dsa layer")
    with torch.no_grad():
        topk_idxs = ix(x, qr, 0, 0)
    assert topk_idxs.dtype == torch.int64 and tuple(topk_idxs.shape) == (1, seqlen, topk)
    qm = torch.randn(1, seqlen, 128, DQK, generator=g).to(torch.bfloat16).to(gpu)
    kvm = torch.randn(1, seqlen, DQK, generator=g).to(torch.bfloat16).to(gpu)
    attn = t1.Model(128, DQK, v_dim=DV).to(gpu)
    out = attn(qm, kvm, topk_idxs)
    ref = osa.sparse_attn_ref(qm, kvm, attn.attn_sink, topk_idxs, attn.softmax_scale, v_dim=DV)
    _compare(out, ref, "dsa-layer")


def test_dsa_layer_c5_full_size_chained(gpu):
    """configs[4] prefill chained as in the reference (task2_v0_ref.py:138-143 output is
    task1_v0_ref.py:8-12's topk_idxs): the indexer Model.forward at 8192 tokens with
    W ~ N(0, 0.02) gives int64 top-2048 picks equal to the oracle's on the same GPU; they
    go unchanged into Model(128, 576, v_dim=512), whose output is checked on all 8192
    tokens against the oracle's attention over the same picks (in chunks of 256 tokens)."""
    torch.manual_seed(42)
    init = t2.get_c5_init_inputs(device=gpu)
    ix = t2.Model(*init).to(gpu)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for p in (ix.wq_b.weight, ix.weights_proj.weight):
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16))
    r = oix.IndexerRef(*init).to(gpu)
    r.wq_b.weight.data.copy_(ix.wq_b.weight.data)
    r.weights_proj.weight.data.copy_(ix.weights_proj.weight.data)
    x, qr, sp, off = t2.get_c5_inputs(device=gpu)
    _say("case c5 chained: indexer")
    with torch.no_grad():
        picks = ix(x, qr, sp, off)
        torch.cuda.synchronize()
        _say("case c5 chained: indexer oracle")
        want = r(x, qr, sp, off)
        torch.cuda.synchronize()
    assert picks.dtype == torch.int64 and tuple(picks.shape) == (1, 8192, 2048)
    assert torch.equal(picks, want)
    del x, qr, want, r
    torch.cuda.empty_cache()
    qm, kvm, _ = t1.get_mla_inputs(device=gpu)
    attn = t1.Model(128, DQK, v_dim=DV).to(gpu)
    _say("case c5 chained: sparse MLA over the indexer's picks")
    out = attn(qm, kvm, picks)
    torch.cuda.synchronize()
    _say("case c5 chained: oracle attention over all 8192 tokens")
    exact = _compare_all_tokens(out, qm, kvm, attn.attn_sink, picks, attn.softmax_scale, "c5-chained")
    assert exact > 0.97
