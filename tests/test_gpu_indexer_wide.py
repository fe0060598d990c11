"""Task2 wide configuration (configs[4] indexer: 64 heads x 128, top-2048) on the MI355X.

1. torch-ROCm's 64-head sum against rules.head_sum('rocm_split2') (pins the order).
2. The bf16 index scores of the wide kernel against the oracle run on the same GPU.
3. int64 indices through the drop-in Model against the oracle (torch.equal, ties
   included), from small shapes to the full configs[4] size.
"""
import numpy as np
import pytest
import torch

from conftest import bits_of
from ascendc_kernel_amd import _native
from ascendc_kernel_amd import task2_indexer as t2
from oracle import indexer as oix
from oracle import rules

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _wide_bits(shape, g):
    sgn = torch.randint(0, 2, shape, generator=g, dtype=torch.int32)
    ex = torch.randint(115, 139, shape, generator=g, dtype=torch.int32)
    mn = torch.randint(0, 128, shape, generator=g, dtype=torch.int32)
    return ((sgn << 15) | (ex << 7) | mn).to(torch.int16).view(torch.bfloat16)


def _cancelling_bits(shape, g):
    """Small N(0,1) values plus eight exactly cancelling pairs of large values per output:
    every summation order of the heads rounds differently."""
    b, s_, h, t = shape
    x = torch.randn(shape, generator=g)
    perm = torch.argsort(torch.rand(b, s_, t, h, generator=g), dim=-1)
    big = torch.exp2(torch.randint(14, 21, (b, s_, t, 8), generator=g).float()) * (
        1 + torch.randint(0, 128, (b, s_, t, 8), generator=g).float() / 128)
    xt = x.permute(0, 1, 3, 2).contiguous()
    xt.scatter_(-1, perm[..., :8], big)
    xt.scatter_(-1, perm[..., 8:16], -big)
    return xt.permute(0, 1, 3, 2).contiguous().to(torch.bfloat16)


@pytest.mark.parametrize("b,s,t", [(1, 1, 128), (1, 1, 64), (2, 3, 130), (1, 7, 1001), (1, 40, 8190),
                                   (1, 1, 8189), (1, 2, 8192), (3, 5, 258), (1, 1, 66)])
def test_torch_head_sum_rule_64_all_splits(gpu, b, s, t):
    """torch-ROCm's x[b, s, 64, T].sum(dim=2) equals head_sum in the order rules.torch_head_split
    names (1, 2 or 4 threads) at shapes of each kind."""
    g = torch.Generator().manual_seed(b * 100000 + s * 10000 + t)
    x = _cancelling_bits((b, s, 64, t), g)
    order = rules.head_sum_order_64(b * s * t, t)
    _say("rule head-sum 64", (b, s, t), order)
    got = bits_of(x.to(gpu).sum(dim=2))
    want = rules.bf16_round(rules.head_sum(np.moveaxis(rules.bf16_to_f32(bits_of(x)), 2, -1), order))
    assert np.array_equal(got, want), int((got != want).sum())


def test_torch_head_sum_rule_64(gpu):
    """x[1, 512, 64, 1024].sum(dim=2): two threads (even / odd heads), four accumulators each."""
    g = torch.Generator().manual_seed(11)
    x = _wide_bits((1, 512, 64, 1024), g)
    _say("rule head-sum 64")
    got = bits_of(x.to(gpu).sum(dim=2))
    xs = rules.bf16_to_f32(bits_of(x[:, :64]))
    want = rules.bf16_round(rules.head_sum(np.moveaxis(xs, 2, -1), "rocm_split2"))
    assert np.array_equal(got[:, :64], want), int((got[:, :64] != want).sum())
    other = rules.bf16_round(rules.head_sum(np.moveaxis(xs, 2, -1), "rocm"))
    assert not np.array_equal(other, want)  # the planted data tells the two orders apart


def _args(seqlen, topk, rd=64, batch=1):
    return oix.IndexerArgs(max_batch_size=batch, max_seq_len=seqlen, dim=7168, q_lora_rank=1536,
                           rope_head_dim=rd, index_n_heads=64, index_head_dim=128, index_topk=topk)


def _pair(args, seed, kv_rows, ratio, device, wstd=None):
    torch.manual_seed(seed)
    fr = oix.precompute_freqs_cis(args.rope_head_dim, args.max_seq_len, device=device)
    kv = torch.randn(args.max_batch_size, kv_rows, args.index_head_dim, dtype=torch.bfloat16).to(device)
    torch.manual_seed(seed + 1)
    m = t2.Model(args, fr, kv, ratio).to(device)
    if wstd is not None:
        g = torch.Generator().manual_seed(seed + 2)
        with torch.no_grad():
            for p in (m.wq_b.weight, m.weights_proj.weight):
                p.copy_((torch.randn(p.shape, generator=g) * wstd).to(torch.bfloat16))
    r = oix.IndexerRef(args, fr, kv, ratio).to(device)
    r.wq_b.weight.data.copy_(m.wq_b.weight.data)
    r.weights_proj.weight.data.copy_(m.weights_proj.weight.data)
    return m, r


def _check_equal(got, want, name):
    eq = torch.equal(got, want)
    if not eq:
        rows = (got != want).any(dim=-1)
        r0 = int(torch.nonzero(rows.view(-1))[0])
        _say(f"[{name}] mismatching rows {int(rows.sum())} of {rows.numel()}; first {r0}:",
             got.view(-1, got.shape[-1])[r0, :12].tolist(), want.view(-1, want.shape[-1])[r0, :12].tolist())
    assert eq, name


@pytest.mark.parametrize("seqlen,start_pos", [(512, 0), (96, 0), (64, 128),
                                              # candidate counts of every head-split kind:
                                              # T = 1001 (1 thread), 130 (4), 128 with one
                                              # token (4), 64 with one token (1), 1002 (4)
                                              (1001, 0), (3, 127), (1, 127), (1, 63), (1002, 0)])
def test_wide_score_stage_matches_torch(gpu, seqlen, start_pos):
    args = _args(start_pos + seqlen, 2048)
    m, r = _pair(args, 31, start_pos + seqlen, 1, gpu, wstd=0.02)
    g = torch.Generator().manual_seed(32)
    x = torch.randn(1, seqlen, 7168, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(1, seqlen, 1536, generator=g).to(torch.bfloat16).to(gpu)
    end = start_pos + seqlen
    _say("wide score stage", seqlen, start_pos)
    want = oix.index_scores(r.wq_b.weight, r.weights_proj.weight, r.kv_cache, r.freqs_cis, x, qr,
                            start_pos, 64, 128, 64, 1)
    q = torch.nn.functional.linear(qr, m.wq_b.weight).unflatten(-1, (64, 128)).contiguous()
    wl = torch.nn.functional.linear(x, m.weights_proj.weight)
    got = _native.indexer_scores(q, m.kv_cache, wl, 128 ** -0.5 * 64 ** -0.5, m.freqs_cis[start_pos:end],
                                 64, end, 1, start_pos == 0)
    gb, wb = bits_of(got), bits_of(want)
    ne = gb != wb
    if ne.any():
        i = np.argwhere(ne)[:6]
        _say("first mismatches:", [(tuple(int(v) for v in ii), hex(gb[tuple(ii)]), hex(wb[tuple(ii)])) for ii in i],
             "fraction", float(ne.mean()))
    assert not ne.any(), int(ne.sum())


WIDE = [
    # seqlen, start_pos, offset, topk, ratio
    (512, 0, 0, 128, 1),
    (1024, 0, 5, 2048, 1),
    (700, 0, 0, 300, 1),
    (64, 128, 7, 64, 1),
    (256, 0, 0, 96, 2),
    (4, 8188, 9, 2048, 1),   # decode at the configs[4] size: 4 tokens at the end of 8192
    # decode shapes take the candidate split (few token groups: each workgroup scores
    # a run of candidate tiles): one token, 16 tokens (63 chunks of 2 tiles), ratio 2
    (1, 8191, 2, 2048, 1),
    (16, 4000, 0, 512, 1),
    (2, 3006, 1, 256, 2),
    # candidate counts that are not multiples of 4, and few outputs, where torch sums the
    # 64 heads over 1 or 4 threads instead of 2: decode one token at T = 8189 (odd),
    # 8190 (T % 4 == 2), 8191; two tokens at 8191; prefill of odd and 2-mod-4 lengths;
    # one token at T = 128 (4 threads) and T = 64 (1 thread); ratio 2 with T = 1502
    (1, 8188, 0, 2048, 1),
    (1, 8189, 3, 2048, 1),
    (1, 8190, 0, 2048, 1),
    (2, 8189, 0, 2048, 1),
    (1001, 0, 0, 2048, 1),
    (1002, 0, 4, 512, 1),
    (255, 0, 0, 100, 1),
    (1, 127, 0, 64, 1),
    (1, 63, 0, 32, 1),
    (1, 3004, 0, 1024, 2),
    (2, 1, 0, 3, 1),      # T = 3
    (1, 0, 0, 1, 1),      # T = 1: a single candidate (top-1 whatever its score)
    (300, 0, (1 << 35) + 1, 256, 1),   # an offset beyond int32 (int64 output)
    (2, 4000, -(1 << 36), 512, 1),
]


@pytest.mark.parametrize("case", WIDE)
def test_wide_shapes_and_modes(gpu, case):
    seqlen, start_pos, offset, topk, ratio = case
    end = start_pos + seqlen
    args = _args(end, topk)
    m, r = _pair(args, 200 + seqlen, end // ratio, ratio, gpu, wstd=0.02)
    g = torch.Generator().manual_seed(seqlen + 1)
    x = torch.randn(1, seqlen, 7168, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(1, seqlen, 1536, generator=g).to(torch.bfloat16).to(gpu)
    _say("wide case", case)
    _check_equal(m(x, qr, start_pos, offset), r(x, qr, start_pos, offset), f"wide{case}")


WIDE_BATCHES = [
    # batch, kv_cache batch rows (max_batch_size), seqlen, start_pos, offset, topk, ratio
    (3, 3, 300, 0, 0, 256, 1),        # prefill, one key row block per batch
    (2, 4, 700, 0, 5, 512, 2),        # fewer batches than the cache holds (kv_cache[:bsz])
    (2, 2, 2600, 0, 0, 2048, 1),      # prefill past K = 2048 in both batches (per-row select)
    (3, 3, 1, 4000, 1, 1024, 1),      # decode, one token per batch (candidate split)
    (2, 2, 4, 8188, 9, 2048, 1),      # decode at the configs[4] length, two batches
]


@pytest.mark.parametrize("case", WIDE_BATCHES)
def test_wide_batches(gpu, case):
    """Batches of the wide configuration (the configs[4] indexer has one): each batch's
    tokens score that batch's kv_cache rows, through prefill and decode launches.

    The reference's einsum (task2_v0_ref.py:133) over a whole batch of 2 x 2600 tokens
    runs as one GEMM whose algorithm sums head_dim in another fp32 order for a few
    products (333 of 865 M differ from the same einsum taken 128 tokens at a time, and
    659 from one einsum per batch); the kernel's scores equal those of the 128-token
    einsum bit for bit (all 13.5 M), and 4 of the 5,200 rows' picks differ from the
    whole-batch GEMM's. So the indices are checked with torch.equal against the
    reference with its einsum taken 128 tokens at a time, and the agreement with the
    single-GEMM reference is printed and held to 99.5 % of the rows."""
    bsz, max_b, seqlen, start_pos, offset, topk, ratio = case
    end = start_pos + seqlen
    args = _args(end, topk, batch=max_b)
    m, r = _pair(args, 500 + seqlen, end // ratio, ratio, gpu, wstd=0.02)
    g = torch.Generator().manual_seed(seqlen + 11)
    x = torch.randn(bsz, seqlen, 7168, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(bsz, seqlen, 1536, generator=g).to(torch.bfloat16).to(gpu)
    _say("wide batches", case)
    with torch.no_grad():
        got = m(x, qr, start_pos, offset)
        whole = r(x, qr, start_pos, offset)
        r.einsum_rows = 128
        want = r(x, qr, start_pos, offset)
    assert got.shape == (bsz, seqlen, min(topk, end // ratio))
    agree = float((got == whole).all(dim=-1).float().mean())
    _say("rows equal to the single-GEMM reference:", agree)
    assert agree >= 0.995
    _check_equal(got, want, f"wide-batches{case}")


@pytest.mark.parametrize("seqlen", [256, 4])
@pytest.mark.parametrize("keys", ["spread24", "spread60", "equal", "equal_but_100"])
def test_wide_select_key_spreads(gpu, seqlen, keys):
    """Top-2048 of 4096 candidates (start_pos 4096 - seqlen, no mask) with the key rows
    scaled by 2^e per candidate, so that the picks' scores span many binades of both
    signs (the selector's second radix pass then tells 15-96 high-byte bins apart), or
    with every key row equal (one score per token: one bin, the second pass skipped,
    the order decided by the index alone), or all equal but 100 (about 2,000 of the
    2,048 picks tie at the k-th key). 256 tokens take the 256-thread selector,
    4 tokens the 1024-thread one."""
    end, topk = 4096, 2048
    start_pos = end - seqlen
    args = _args(end, topk)
    m, r = _pair(args, 77, end, 1, gpu, wstd=0.02)
    g = torch.Generator().manual_seed(78)
    with torch.no_grad():
        if keys.startswith("equal"):
            keep = m.kv_cache.clone()
            m.kv_cache.copy_(m.kv_cache[:, :1].clone().expand_as(m.kv_cache))
            if keys == "equal_but_100":  # ~2,000 picks tie at the k-th key: index order decides
                sel = torch.randperm(end, generator=g)[:100].to(gpu)
                m.kv_cache[:, sel] = keep[:, sel]
        else:
            span = int(keys[len("spread"):])
            e = torch.randint(-span, span + 1, (end,), generator=g).float()
            m.kv_cache.mul_(torch.exp2(e).to(gpu)[None, :, None].to(torch.bfloat16))
    assert m.kv_cache is r.kv_cache
    x = torch.randn(1, seqlen, 7168, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(1, seqlen, 1536, generator=g).to(torch.bfloat16).to(gpu)
    _say("select key spread", seqlen, keys)
    with torch.no_grad():
        got = m(x, qr, start_pos, 3)
        want = r(x, qr, start_pos, 3)
    _check_equal(got, want, f"spread-{keys}-{seqlen}")


@pytest.mark.parametrize("input_seed", [43, None])
def test_full_shape_c5_indexer(gpu, input_seed):
    """configs[4] indexer: x[1,8192,7168], qr[1,8192,1536], kv_cache[1,8192,128], W ~ N(0, 0.02),
    causal, top-2048, ratio 1, rope_head_dim 64. input_seed None draws x and qr right after
    the model (the draw in which an accumulation through v_dot2c_f32_bf16 once changed the
    top-k of one row; the kernels now add with IEEE fp32 adds)."""
    torch.manual_seed(42)
    init = t2.get_c5_init_inputs(device=gpu)
    m = t2.Model(*init).to(gpu)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for p in (m.wq_b.weight, m.weights_proj.weight):
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16))
    if input_seed is not None:
        torch.manual_seed(input_seed)
    x, qr, sp, off = t2.get_c5_inputs(device=gpu)
    r = oix.IndexerRef(*init).to(gpu)
    r.wq_b.weight.data.copy_(m.wq_b.weight.data)
    r.weights_proj.weight.data.copy_(m.weights_proj.weight.data)
    _say("case c5 indexer full shape", input_seed)
    with torch.no_grad():
        got = m(x, qr, sp, off)
        torch.cuda.synchronize()
        _say("case c5 oracle")
        want = r(x, qr, sp, off)
        torch.cuda.synchronize()
    _check_equal(got, want, "c5-indexer")


@pytest.mark.parametrize("seqlen,topk,start_pos", [(1024, 2048, 0), (700, 300, 0), (96, 64, 160)])
def test_wide_single_kernel_and_workspace_paths(gpu, seqlen, topk, start_pos):
    """dsa_indexer_score_topk (keys of 4 tokens in LDS, fused top-k) and
    dsa_indexer_score_topk_ws (keys in the workspace, per-token select kernel) give the
    reference's indices."""
    end = start_pos + seqlen
    args = _args(end, topk)
    m, r = _pair(args, 300 + seqlen, end, 1, gpu, wstd=0.02)
    g = torch.Generator().manual_seed(seqlen + 7)
    x = torch.randn(1, seqlen, 7168, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(1, seqlen, 1536, generator=g).to(torch.bfloat16).to(gpu)
    _say("wide paths", seqlen, topk, start_pos)
    want = r(x, qr, start_pos, 3)
    q = torch.nn.functional.linear(qr, m.wq_b.weight).unflatten(-1, (64, 128)).contiguous()
    wl = torch.nn.functional.linear(x, m.weights_proj.weight)
    k = min(topk, end)
    for ws in (False, True):
        got = _native.indexer_score_topk(q, m.kv_cache, wl, 128 ** -0.5 * 64 ** -0.5, m.freqs_cis[start_pos:end],
                                         64, end, k, 1, start_pos == 0, 3, use_workspace=ws)
        _check_equal(got, want, f"wide-ws{ws}-{seqlen}-{topk}")
