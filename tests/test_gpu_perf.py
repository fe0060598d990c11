"""Same-GPU speed check: the HIP path against the reference PyTorch path.

north_star asks for both tasks to be faster than the reference's PyTorch path on
the same GPU. The reference path here is the oracle's op-for-op restatement of the
reference modules (oracle/sparse_attn.py, oracle/indexer.py) run by torch-ROCm.
Times are hipEvent medians over a few calls; the test prints them and requires the
HIP path to be faster at the benchmark configurations (configs[1], [2], [3], [4]).
The budget tests hold the kernels at the full configurations to times relative to a
calibration (a device copy, a bf16 matmul) measured in the same process.
"""
import statistics

import pytest
import torch

from ascendc_kernel_amd import task1_sparse_attn as t1
from ascendc_kernel_amd import task2_indexer as t2
from oracle import indexer as oix
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu


def _median_us(fn, reps=5, warm=2):
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        z.record()
        z.synchronize()
        ts.append(a.elapsed_time(z) * 1e3)
    return statistics.median(ts)


def _settled_us(fn, reps, min_seconds=0.3):
    """Mean hipEvent time of `reps` back-to-back calls after a warm-up that runs calls for at
    least `min_seconds` (the board raises its clock over the first tens of milliseconds of
    load; bench.py warms up the same way)."""
    import time
    t_end = time.perf_counter() + min_seconds
    fn()
    torch.cuda.synchronize()
    while time.perf_counter() < t_end:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    z.record()
    z.synchronize()
    return a.elapsed_time(z) * 1e3 / reps


# Budgets relative to a calibration timed in the same process, so that the clock and
# memory speed of the box cancel: the HBM-bound Task1 kernel against torch's device copy of
# the configs[1] q (340.8 MB read and written), every other kernel (matrix cores, VALU, the
# clock) against a bf16 [8192 x 8192] x [8192 x 8192] torch.matmul. A regression past
# ratio x calibration fails. Measured (copy 125.6 - 126.8 us, matmul 794 - 815 us; three
# runs on each box): c2 0.935 - 0.947 (two boxes), c3 kernel 0.0523 - 0.0527, c3
# projections 0.0276 - 0.0287, c3 Model.forward 0.0793 - 0.0835 (four boxes), c4 0.492 - 0.511 (two
# boxes), c5 MLA 6.50 - 6.87 (two boxes: the ratio that varies most between boxes), c5
# indexer kernels 0.845 - 0.847 (two boxes, the current selector). Each budget sits 5 %
# above the largest ratio measured on two boxes, 7 % above one measured on one box (the
# spread between boxes is up to ~6 %); configs[1]: 0.99, a 125 us equivalent at the
# copy's 126 us.
RATIO_BUDGET = {"c2": ("copy", 0.99), "c3_kernel": ("matmul", 0.0564), "c3_proj": ("matmul", 0.0301),
                "c3_model": ("matmul", 0.0877), "c4": ("matmul", 0.536), "c5_mla": ("matmul", 7.21),
                "c5_indexer": ("matmul", 0.89)}


@pytest.fixture(scope="module")
def calib(gpu):
    return calibrate(gpu)


def calibrate(gpu):
    """The calibration times (us) of this process: {'copy': ..., 'matmul': ...}."""
    torch.manual_seed(0)
    src = torch.randn(8, 2600, 64, 128, device=gpu).to(torch.bfloat16)
    dst = torch.empty_like(src)
    copy_us = _settled_us(lambda: dst.copy_(src), 50)
    del src, dst
    a = torch.randn(8192, 8192, device=gpu).to(torch.bfloat16)
    b = torch.randn(8192, 8192, device=gpu).to(torch.bfloat16)
    mm_us = _settled_us(lambda: torch.matmul(a, b), 20)
    del a, b
    torch.cuda.empty_cache()
    print(f"[calibration] copy {copy_us:.1f} us, matmul {mm_us:.1f} us", flush=True)
    return {"copy": copy_us, "matmul": mm_us}


def _check_budget(name, us, calib):
    base, ratio = RATIO_BUDGET[name]
    got = us / calib[base]
    print(f"[budget {name}] {us:.1f} us = {got:.4f} x {base} ({calib[base]:.1f} us); budget {ratio:.4f} "
          f"({ratio * calib[base]:.1f} us)", flush=True)
    assert got <= ratio, f"{name}: {us:.1f} us is {got:.4f} x {base}, budget {ratio:.4f}"


def test_budget_task1_c2(gpu, calib):
    torch.manual_seed(42)
    q, kv, idx = [x.to(gpu) for x in t1.get_inputs()]
    m = t1.Model(*t1.get_init_inputs()).to(gpu)
    us = _settled_us(lambda: m(q, kv, idx), 50)
    _check_budget("c2", us, calib)


def test_budget_task2_c3_kernel(gpu, calib):
    from ascendc_kernel_amd import _native
    torch.manual_seed(42)
    m = t2.Model(*t2.get_init_inputs(device=gpu)).to(gpu)
    x, qr, _, _ = t2.get_inputs(device=gpu)
    with torch.no_grad():
        q = torch.nn.functional.linear(qr, m.wq_b.weight).unflatten(-1, (16, 64)).contiguous()
        wl = torch.nn.functional.linear(x, m.weights_proj.weight)
        fn = lambda: _native.indexer_score_topk(q, m.kv_cache, wl, 64 ** -0.5 * 16 ** -0.5,
                                                None, 32, 650, 128, 4, True, 0)
        us = _settled_us(fn, 50)
    _check_budget("c3_kernel", us, calib)


def test_budget_task2_c3_projections_and_model(gpu, calib):
    """The one-launch projections (q with RoPE, and the head weights) and the whole
    Model.forward at configs[2]."""
    from ascendc_kernel_amd import _native
    torch.manual_seed(42)
    m = t2.Model(*t2.get_init_inputs(device=gpu)).to(gpu)
    x, qr, sp, off = t2.get_inputs(device=gpu)
    assert m.route(x, qr) == "both"
    pq, pw = m.packed_weights()
    with torch.no_grad():
        us_p = _settled_us(lambda: _native.indexer_projections(qr, pq, m.freqs_cis[:2600], x, pw, 64, 32), 50)
        us_m = _settled_us(lambda: m(x, qr, sp, off), 50)
    _check_budget("c3_proj", us_p, calib)
    _check_budget("c3_model", us_m, calib)


def test_budget_task1_c4(gpu, calib):
    q, kv, idx = t1.get_gather_inputs(device=gpu)
    m = t1.Model(64, 128).to(gpu)
    us = _settled_us(lambda: m(q, kv, idx), 10)
    _check_budget("c4", us, calib)


def test_budget_c5_mla(gpu, calib):
    q, kv, idx = t1.get_mla_inputs(device=gpu)
    m = t1.Model(128, 576, v_dim=512).to(gpu)
    us = _settled_us(lambda: m(q, kv, idx), 5, 0.2)
    _check_budget("c5_mla", us, calib)


def test_budget_c5_indexer_kernels(gpu, calib):
    """The configs[4] indexer kernels alone (wide score kernel + selector), as bench.py's
    indexer_kernel_us times them: q and the head weights from F.linear, causal top-2048."""
    from ascendc_kernel_amd import _native
    torch.manual_seed(42)
    m = t2.Model(*t2.get_c5_init_inputs(device=gpu)).to(gpu)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for prm in (m.wq_b.weight, m.weights_proj.weight):
            prm.copy_((torch.randn(prm.shape, generator=g) * 0.02).to(torch.bfloat16))
    x, qr, _, _ = t2.get_c5_inputs(device=gpu)
    with torch.no_grad():
        q = torch.nn.functional.linear(qr, m.wq_b.weight).unflatten(-1, (64, 128)).contiguous()
        wl = torch.nn.functional.linear(x, m.weights_proj.weight)
        fr = m.freqs_cis[:8192]
        fn = lambda: _native.indexer_score_topk(q, m.kv_cache, wl, 128 ** -0.5 * 64 ** -0.5, fr, 64, 8192, 2048,
                                                1, True, 0)
        us = _settled_us(fn, 10, 0.2)
    _check_budget("c5_indexer", us, calib)


def test_task1_c2_faster_than_torch_path(gpu):
    torch.manual_seed(42)
    q, kv, idx = [x.to(gpu) for x in t1.get_inputs()]
    m = t1.Model(*t1.get_init_inputs()).to(gpu)
    k_us = _median_us(lambda: m(q, kv, idx), reps=20)
    r_us = _median_us(lambda: osa.sparse_attn_ref(q, kv, m.attn_sink, idx, m.softmax_scale))
    print(f"[perf c2] kernel {k_us:.1f} us, torch path {r_us:.1f} us, x{r_us / k_us:.1f}", flush=True)
    assert k_us < r_us


def test_task2_c3_faster_than_torch_path(gpu):
    torch.manual_seed(42)
    m = t2.Model(*t2.get_init_inputs(device=gpu)).to(gpu)
    torch.manual_seed(42)
    r = oix.IndexerRef(*oix.get_init_inputs(device=gpu)).to(gpu)
    x, qr, sp, off = t2.get_inputs(device=gpu)
    with torch.no_grad():
        k_us = _median_us(lambda: m(x, qr, sp, off), reps=20)
        r_us = _median_us(lambda: r(x, qr, sp, off))
    print(f"[perf c3] Model.forward {k_us:.1f} us, torch path {r_us:.1f} us, x{r_us / k_us:.1f}", flush=True)
    assert k_us < r_us


def test_task1_c4_faster_than_torch_path(gpu):
    q, kv, idx = t1.get_gather_inputs(device=gpu)
    m = t1.Model(64, 128).to(gpu)
    k_us = _median_us(lambda: m(q, kv, idx), reps=10)

    def ref():  # chunks of 1024 tokens keep the torch path's temporaries near 2 GB
        for i in range(0, q.shape[1], 1024):
            osa.sparse_attn_ref(q[:, i:i + 1024], kv, m.attn_sink, idx[:, i:i + 1024], m.softmax_scale)
    r_us = _median_us(ref, reps=3, warm=1)
    print(f"[perf c4] kernel {k_us:.1f} us, torch path {r_us:.1f} us, x{r_us / k_us:.1f}", flush=True)
    assert k_us < r_us


def test_dsa_layer_c5_faster_than_torch_path(gpu):
    """the indexer Model.forward at full size; sparse MLA on 256 tokens of the
    full-size inputs (the torch path's gathered rows for all 8192 tokens would be ~40 GB)."""
    torch.manual_seed(42)
    init = t2.get_c5_init_inputs(device=gpu)
    m = t2.Model(*init).to(gpu)
    r = oix.IndexerRef(*init).to(gpu)
    r.wq_b.weight.data.copy_(m.wq_b.weight.data)
    r.weights_proj.weight.data.copy_(m.weights_proj.weight.data)
    x, qr, sp, off = t2.get_c5_inputs(device=gpu)
    with torch.no_grad():
        k_us = _median_us(lambda: m(x, qr, sp, off), reps=5)
        r_us = _median_us(lambda: r(x, qr, sp, off), reps=3, warm=1)
    print(f"[perf c5 indexer] Model.forward {k_us:.1f} us, torch path {r_us:.1f} us, x{r_us / k_us:.1f}", flush=True)
    assert k_us < r_us
    del x, qr
    q, kv, idx = t1.get_mla_inputs(device=gpu)
    attn = t1.Model(128, 576, v_dim=512).to(gpu)
    sl = slice(4096, 4096 + 256)
    qs, ids = q[:, sl].contiguous(), idx[:, sl].contiguous()
    k_us = _median_us(lambda: attn(qs, kv, ids), reps=10)
    r_us = _median_us(lambda: osa.sparse_attn_ref(qs, kv, attn.attn_sink, ids, attn.softmax_scale, v_dim=512),
                      reps=3, warm=1)
    print(f"[perf c5 mla, 256 tokens] kernel {k_us:.1f} us, torch path {r_us:.1f} us, x{r_us / k_us:.1f}", flush=True)
    assert k_us < r_us


@pytest.mark.parametrize("seqlen", [1, 4])
def test_dsa_decode_c5_faster_than_torch_path(gpu, seqlen):
    """Decode at the configs[4] size: `seqlen` new tokens at the end of the 8192-token
    context (start_pos 8192 - seqlen: no mask). The indexer Model.forward and sparse MLA
    over the indexer's int64 picks, each against its torch path, eager (host time
    included on both sides)."""
    torch.manual_seed(42)
    init = t2.get_c5_init_inputs(device=gpu)
    m = t2.Model(*init).to(gpu)
    r = oix.IndexerRef(*init).to(gpu)
    r.wq_b.weight.data.copy_(m.wq_b.weight.data)
    r.weights_proj.weight.data.copy_(m.weights_proj.weight.data)
    sp = 8192 - seqlen
    g = torch.Generator().manual_seed(40 + seqlen)
    x = torch.randn(1, seqlen, 7168, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(1, seqlen, 1536, generator=g).to(torch.bfloat16).to(gpu)
    q = torch.randn(1, seqlen, 128, 576, generator=g).to(torch.bfloat16).to(gpu)
    kv = torch.randn(1, 8192, 576, generator=g).to(torch.bfloat16).to(gpu)
    attn = t1.Model(128, 576, v_dim=512).to(gpu)
    with torch.no_grad():
        idx = m(x, qr, sp, 0)
        assert torch.equal(idx, r(x, qr, sp, 0))
        ki_us = _median_us(lambda: m(x, qr, sp, 0), reps=20)
        ri_us = _median_us(lambda: r(x, qr, sp, 0), reps=5)
        ka_us = _median_us(lambda: attn(q, kv, idx), reps=20)
        ra_us = _median_us(lambda: osa.sparse_attn_ref(q, kv, attn.attn_sink, idx, attn.softmax_scale,
                                                       v_dim=512), reps=5)
    print(f"[perf c5 decode s={seqlen}] indexer {ki_us:.1f} us vs torch {ri_us:.1f} us (x{ri_us / ki_us:.1f}); "
          f"sparse MLA {ka_us:.1f} us vs torch {ra_us:.1f} us (x{ra_us / ka_us:.1f})", flush=True)
    assert ki_us < ri_us and ka_us < ra_us
