#!/usr/bin/env python3
"""Benchmark of the MI355X DSA path; prints ONE JSON line.

Headline (BASELINE.json metric, configs[1]): Task1 sparse attention at the full
shape q[8,2600,64,128] bf16, kv[8,32,128], topk_idxs[8,2600,16] (drawn with
replacement), inputs resident in HBM. One step = one forward call of the drop-in
module (one kernel launch). value = algorithmic HBM bytes per call / time per call.

Also reported, each with hot-cache times and times with the 256 MB MALL flushed
(512 MB written and read back before every call; back-to-back flush + call pairs
minus the flushes alone, so that cold and hot calls are timed the same way; the
headline also gives one call timed alone after a flush):
  task1_c1      configs[0] on the GPU, beside the reference path on the host CPU;
  task1_c4      the true-gather kernel at configs[3] (MFMA-bound);
  task2         configs[2]: Model.forward (one launch for both projections, q with
                RoPE and the head weights, then the fused score / top-k kernel), the
                fused kernel and the projections kernel alone with their rooflines,
                and the reference path on the host CPU;
  dsa_layer_c5  configs[4]: the wide indexer, sparse MLA, and the whole prefill layer
                (indexer Model.forward whose int64 top-2048 feeds sparse MLA);
  dsa_decode_c5 one configs[4] decode step, HIP-graph replayed and eager.
cpu_baseline is the reference path (the oracle's restatement of task1_v0_ref.py) on
the host's CPU cores over the whole configs[1] workload.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16, published
TRAFFIC_SOURCE = "profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE per dispatch, copy-calibrated)"

T1_SHAPE = dict(b=8, m=2600, h=64, d=128, n_kv=32, topk=16)


def t1_bytes(b, m, h, d, n_kv, topk):
    """Algorithmic bytes of one Task1 call: q read + out write + kv + idx + sink."""
    return 2 * (b * m * h * d) * 2 + b * n_kv * d * 2 + b * m * topk * 4 + h * 4


def t2_bytes(b=8, s=2600, dim=1024, ql=256, t=650, d=64, h=16, rd=32, k=128):
    """Task2 configs[2]: compulsory bytes of Model.forward (x, qr, kv_cache, weights, freqs, out)."""
    return (b * s * dim * 2 + b * s * ql * 2 + b * t * d * 2 + h * d * ql * 2 + h * dim * 2
            + s * (rd // 2) * 8 + b * s * k * 8)


def t2_kernel_bytes(b=8, s=2600, t=650, d=64, h=16, k=128):
    """The fused kernel as Model.forward runs it: q read (already rotated by the projection
    kernel), wl read, kv_cache, int64 output."""
    return b * s * h * d * 2 + b * s * h * 2 + b * t * d * 2 + b * s * k * 8


def _say(msg):
    """Progress line on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _events_time(torch, fn, steps, stream):
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / steps  # ms per call


def _warm(torch, fn, steps, min_seconds=0.3):
    """`steps` untimed calls, then more until `min_seconds` of calls have run: the board
    raises its clock over the first tens of milliseconds of load (the first ~50 Task1 calls
    after start-up run ~15% slower), and the timed steps should see the settled clock."""
    t_end = time.perf_counter() + min_seconds
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def _flush(torch, flush):
    """Evicts the 256 MB MALL: 512 MB are written, then read back, so that the caches hold
    only clean lines of the flush buffer (with the write alone, its dirty lines would be
    written back to HBM during the next call and be counted against it)."""
    flush.fill_(1)
    flush.view(torch.int64).sum()


def _cold_time(torch, fn, reps, stream, flush):
    """Ms per call with the MALL flushed before every call, timed like the hot figure:
    `reps` back-to-back (flush, call) pairs minus `reps` flushes alone, median of 5 such
    differences. Each call then follows other work on the stream, as in the hot loop, so
    the two figures differ only by what the flush evicted."""
    d = []
    for _ in range(5):
        t = []
        for with_call in (True, False):
            a = torch.cuda.Event(enable_timing=True)
            z = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(reps):
                _flush(torch, flush)
                if with_call:
                    fn()
            z.record(stream)
            z.synchronize()
            t.append(a.elapsed_time(z))
        d.append((t[0] - t[1]) / reps)
    return statistics.median(d)


def _cold_single_time(torch, fn, reps, stream, flush):
    """Median ms of one call timed alone (its own event pair) right after a flush: this
    also counts the call's dispatch, which back-to-back calls overlap."""
    ts = []
    for _ in range(reps):
        _flush(torch, flush)
        a = torch.cuda.Event(enable_timing=True)
        z = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        z.record(stream)
        z.synchronize()
        ts.append(a.elapsed_time(z))
    return statistics.median(ts)


def _traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary, if present."""
    p = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f)["kernels"][kernel]["traffic_bytes"]
    except (OSError, ValueError, KeyError):
        return None


def _host():
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        cpu = platform.processor() or "unknown"
    return cpu, len(os.sched_getaffinity(0))


def _cpu_median_s(fn, warm, reps):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _roofline_hbm(nbytes, ms, traffic):
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic}


def _roofline_mfma(flop, ms):
    tf = flop / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the host-CPU reference legs")
    ap.add_argument("--no-task2", action="store_true")
    ap.add_argument("--no-c4", action="store_true", help="skip the configs[3] true-gather leg")
    ap.add_argument("--no-c5", action="store_true", help="skip the configs[4] DSA-layer (prefill) leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the configs[4] decode leg")
    ap.add_argument("--no-cold", action="store_true", help="skip the MALL-flushed timings")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run 5 plain device copies of 256 MiB (counter calibration for rocprofv3 --pmc)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every config fits one MI355X)", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from ascendc_kernel_amd import _native
    from ascendc_kernel_amd import task1_sparse_attn as t1
    from ascendc_kernel_amd import task2_indexer as t2

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    _native.load()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    cpu_model, ncores = _host()
    flush = None if a.no_cold else torch.empty(512 << 20, dtype=torch.uint8, device=dev)

    def cold(fn, reps):
        return None if flush is None else round(_cold_time(torch, fn, reps, stream, flush) * 1e3, 2)

    def cold_single(fn, reps):
        return None if flush is None else round(_cold_single_time(torch, fn, reps, stream, flush) * 1e3, 2)

    # ---------------- Task1 headline; the CPU copies of the inputs are kept
    # for the host-CPU reference leg.
    torch.manual_seed(42)
    q_cpu, kv_cpu, idx_cpu = t1.get_inputs()
    q, kv, idx = q_cpu.to(dev), kv_cpu.to(dev), idx_cpu.to(dev)
    model = t1.Model(*t1.get_init_inputs()).to(dev)
    with torch.no_grad():
        _warm(torch, lambda: model(q, kv, idx), a.warmup)
        ms = _events_time(torch, lambda: model(q, kv, idx), a.steps, stream)
        torch.cuda.synchronize()
        c2_cold = cold(lambda: model(q, kv, idx), 20)
        c2_cold_single = cold_single(lambda: model(q, kv, idx), 21)
        # The same bytes moved by torch's device copy (q read once, one output written).
        cpy = torch.empty_like(q)
        _warm(torch, lambda: cpy.copy_(q), 3, 0.1)
        ms_copy = _events_time(torch, lambda: cpy.copy_(q), a.steps, stream)
        del cpy
    nb = t1_bytes(**T1_SHAPE)
    gbps = nb / (ms * 1e-3) / 1e9
    if a.calib_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    result = {
        "metric": "µs/call + achieved HBM GB/s (% of peak), Task1 sparse-attn & Task2 indexer",
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_call": round(ms * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (torch.manual_seed(42), reference get_inputs distributions)",
        "config": {"workload": "task1_sparse_attn configs[1]: q[8,2600,64,128] bf16, kv[8,32,128], "
                               "topk_idxs[8,2600,16] int32 with replacement, attn_sink zeros",
                   "algorithmic_bytes": nb, "kernel": "sa_mult_kernel (multiplicity, MFMA)"},
        "roofline": _roofline_hbm(nb, ms, _traffic("sa_mult_kernel")),
        "traffic_source": TRAFFIC_SOURCE,
        "cold_mall_us_per_call": c2_cold,
        "cold_mall_single_call_us": c2_cold_single,
        "torch_copy_same_bytes": {"us": round(ms_copy * 1e3, 2),
                                  "GBps": round(2 * q.numel() * 2 / (ms_copy * 1e-3) / 1e9, 1)},
    }
    del q, kv, idx

    _say("configs[1] headline done")
    # ---------------- Task1 configs[0] (the reference's CPU config) on the GPU
    # (the reference's get_inputs draws with batch_size 1 and seq_len 160, seed 42)
    torch.manual_seed(42)
    q1c = torch.randn(1, 160, 64, 128, dtype=torch.bfloat16)
    kv1c = torch.randn(1, 32, 128, dtype=torch.bfloat16)
    idx1c = torch.randint(0, 32, (1, 160, 16), dtype=torch.int32)
    q1, kv1, idx1 = q1c.to(dev), kv1c.to(dev), idx1c.to(dev)
    with torch.no_grad():
        _warm(torch, lambda: model(q1, kv1, idx1), 10, 0.1)
        ms1 = _events_time(torch, lambda: model(q1, kv1, idx1), max(20, a.steps), stream)
        c1_cold = cold(lambda: model(q1, kv1, idx1), 40)
    result["task1_c1"] = {
        "workload": "task1 configs[0]: q[1,160,64,128] bf16, kv[1,32,128], topk_idxs[1,160,16] with replacement",
        "us_per_call": round(ms1 * 1e3, 2), "cold_mall_us_per_call": c1_cold,
        "algorithmic_bytes": t1_bytes(1, 160, 64, 128, 32, 16)}
    del q1, kv1, idx1

    _say("configs[0] done")
    # ---------------- Task1 true-gather
    if not a.no_c4:
        torch.cuda.empty_cache()
        q4, kv4, idx4 = t1.get_gather_inputs(device=dev)
        m4 = t1.Model(64, 128).to(dev)
        with torch.no_grad():
            _warm(torch, lambda: m4(q4, kv4, idx4), 3, 0.2)
            ms4 = _events_time(torch, lambda: m4(q4, kv4, idx4), max(5, a.steps // 5), stream)
            c4_cold = cold(lambda: m4(q4, kv4, idx4), 10)
        valid = int((idx4 >= 0).sum().item())
        flop4 = 4 * 64 * 128 * valid          # QK + PV over the valid slots
        b4 = t1_bytes(4, 4096, 64, 128, 8192, 512)
        result["task1_c4"] = {
            "workload": "task1 configs[3]: q[4,4096,64,128] bf16, kv[4,8192,128], topk 512 distinct "
                        "of [0,t], -1 padded",
            "kernel": "sa_gather_kernel",
            "us_per_call": round(ms4 * 1e3, 2),
            "cold_mall_us_per_call": c4_cold,
            "valid_slot_frac": round(valid / idx4.numel(), 4),
            "useful_TFLOPs": round(flop4 / (ms4 * 1e-3) / 1e12, 1),
            "mfma_frac": round(flop4 / (ms4 * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "issued_mfma_TFLOPs": round(1.5 * flop4 / (ms4 * 1e-3) / 1e12, 1),
            "algorithmic_bytes": b4,
            "GBps": round(b4 / (ms4 * 1e-3) / 1e9, 1),
            "traffic": _traffic("sa_gather_kernel"),
        }
        del q4, kv4, idx4

    _say("configs[3] done")
    # ---------------- Decode at the configs[4] size (before the prefill legs, so that the
    # prefill calls stay the last dispatches of their kernels): one DSA step for one new
    # token at position 8191 (indexer Model.forward, then sparse MLA over its int64
    # picks: split slot lists + combine), captured in a HIP graph and replayed; the
    # eager step (host time included) beside it.
    if not a.no_decode:
        torch.manual_seed(42)
        initd = t2.get_c5_init_inputs(device=dev)
        ixd = t2.Model(*initd).to(dev)
        gd = torch.Generator().manual_seed(5)
        with torch.no_grad():
            for pd in (ixd.wq_b.weight, ixd.weights_proj.weight):
                pd.copy_((torch.randn(pd.shape, generator=gd) * 0.02).to(torch.bfloat16))
        mlad = t1.Model(128, 576, v_dim=512).to(dev)
        gi = torch.Generator().manual_seed(7)
        xd = torch.randn(1, 1, 7168, generator=gi).to(torch.bfloat16).to(dev)
        qrd = torch.randn(1, 1, 1536, generator=gi).to(torch.bfloat16).to(dev)
        qd = torch.randn(1, 1, 128, 576, generator=gi).to(torch.bfloat16).to(dev)
        kvd = torch.randn(1, 8192, 576, generator=gi).to(torch.bfloat16).to(dev)
        stepd = lambda: mlad(qd, kvd, ixd(xd, qrd, 8191, 0))
        nd = max(20, a.steps)
        with torch.no_grad():
            side = torch.cuda.Stream(dev)
            side.wait_stream(stream)
            with torch.cuda.stream(side):
                for _ in range(3):
                    stepd()
            stream.wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                outd = stepd()
            _warm(torch, graph.replay, 5, 0.1)
            ms_dg = _events_time(torch, graph.replay, nd, stream)
            # Eight steps in one graph (as a serving loop captures every layer of a decode
            # forward in one graph): the per-replay launch gap is paid once per 8 steps.
            graph8 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph8):
                outs8 = [stepd() for _ in range(8)]
            _warm(torch, graph8.replay, 3, 0.1)
            ms_dg8 = _events_time(torch, graph8.replay, max(5, nd // 4), stream) / 8
            eq8 = all(bool(torch.equal(o.view(torch.int16), outd.view(torch.int16))) for o in outs8)
            _warm(torch, stepd, 2, 0.05)
            ms_de = _events_time(torch, stepd, nd, stream)
            eq = bool(torch.equal(outd.view(torch.int16), stepd().view(torch.int16)))
            # the indexer's projections alone (its cached launch: both products in one
            # kernel when the route is 'decode')
            pl = ixd._plan
            route_d = pl.route if pl is not None else None
            ms_dp = _events_time(torch, pl.proj, nd, stream) if route_d == "decode" else None
        dsa_decode = {
            "workload": "configs[4] decode: 1 new token at position 8191 of 8192; indexer 64x128 (qr[1,1,1536], "
                        "x[1,1,7168], kv_cache[1,8192,128], top-2048, no mask) then sparse MLA q[1,1,128,576] over "
                        "latent kv[1,8192,576] with the indexer's int64 picks",
            "graph_us_per_step": round(ms_dg * 1e3, 1),
            "eager_us_per_step": round(ms_de * 1e3, 1),
            "graph_replay_equals_eager": eq,
            "graph8_us_per_step": round(ms_dg8 * 1e3, 1),
            "graph8_replays_equal": eq8,
            "projection_route": route_d,
            "projections_us": round(ms_dp * 1e3, 2) if ms_dp is not None else None,
            "projections_bytes": 26117248,
        }
        del graph, graph8, outs8, outd, xd, qrd, qd, kvd, ixd, mlad
        torch.cuda.empty_cache()

    _say("configs[4] decode done")
    # ---------------- DSA layer: wide indexer + sparse MLA, and the layer
    # chained as in the reference (task2_v0_ref.py:138-143 output -> task1_v0_ref.py:8-12).
    if not a.no_c5:
        torch.cuda.empty_cache()
        torch.manual_seed(42)
        init5 = t2.get_c5_init_inputs(device=dev)
        ix5 = t2.Model(*init5).to(dev)
        g5 = torch.Generator().manual_seed(5)
        with torch.no_grad():
            for p5 in (ix5.wq_b.weight, ix5.weights_proj.weight):
                p5.copy_((torch.randn(p5.shape, generator=g5) * 0.02).to(torch.bfloat16))
        x5, qr5, sp5, off5 = t2.get_c5_inputs(device=dev)
        n5 = max(10, a.steps // 5)
        with torch.no_grad():
            _warm(torch, lambda: ix5(x5, qr5, sp5, off5), 2, 0.2)
            ms_ix = _events_time(torch, lambda: ix5(x5, qr5, sp5, off5), n5, stream)
            ix_cold = cold(lambda: ix5(x5, qr5, sp5, off5), 3)
            q5 = torch.nn.functional.linear(qr5, ix5.wq_b.weight).unflatten(-1, (64, 128)).contiguous()
            wl5 = torch.nn.functional.linear(x5, ix5.weights_proj.weight)
            fr5 = ix5.freqs_cis[:8192]
            kix = lambda: _native.indexer_score_topk(q5, ix5.kv_cache, wl5, 128 ** -0.5 * 64 ** -0.5, fr5,
                                                     64, 8192, 2048, 1, True, 0)
            _warm(torch, kix, 1, 0.1)
            ms_ixk = _events_time(torch, kix, n5, stream)
            picks = ix5(x5, qr5, sp5, off5)  # int64 [1, 8192, 2048], -1 for masked picks
            del q5, wl5
        torch.cuda.empty_cache()
        qm, kvm, idxm = t1.get_mla_inputs(device=dev)
        mla = t1.Model(128, 576, v_dim=512).to(dev)
        with torch.no_grad():
            _warm(torch, lambda: mla(qm, kvm, idxm), 2, 0.2)
            ms_mla = _events_time(torch, lambda: mla(qm, kvm, idxm), n5, stream)
            mla_cold = cold(lambda: mla(qm, kvm, idxm), 3)
            # The indexer's own picks (int64, read by the kernel as they are).
            ms_mla_real = _events_time(torch, lambda: mla(qm, kvm, picks), n5, stream)
            layer = lambda: mla(qm, kvm, ix5(x5, qr5, sp5, off5))
            _warm(torch, layer, 1, 0.1)
            ms_layer = _events_time(torch, layer, n5, stream)
            layer_cold = cold(layer, 3)
        valid_m = int((idxm >= 0).sum().item())
        valid_r = int((picks >= 0).sum().item())
        flop_m = valid_m * 128 * (576 + 512) * 2
        flop_r = valid_r * 128 * (576 + 512) * 2
        bytes_m = qm.numel() * 2 + 8192 * 128 * 512 * 2 + kvm.numel() * 2 + idxm.numel() * 4 + 128 * 4
        score_flop5 = 2 * 64 * 128 * (8192 * 8193 // 2)
        result["dsa_layer_c5"] = {
            "workload": "configs[4]: indexer 64x128 from qr[1,8192,1536] / x[1,8192,7168], kv_cache[1,8192,128], "
                        "causal top-2048 (ratio 1, rope_head_dim 64, W ~ N(0,0.02)); sparse MLA q[1,8192,128,576], "
                        "latent kv[1,8192,576], d_v 512; layer = indexer Model.forward whose int64 picks feed "
                        "sparse MLA (mla_us: synthetic causal picks of the same count)",
            "layer_us": round(ms_layer * 1e3, 1),
            "layer_cold_mall_us": layer_cold,
            "indexer_model_us": round(ms_ix * 1e3, 1),
            "indexer_model_cold_mall_us": ix_cold,
            "indexer_kernel_us": round(ms_ixk * 1e3, 1),
            "indexer_useful_score_TFLOPs": round(score_flop5 / (ms_ixk * 1e-3) / 1e12, 1),
            "mla_kernel": "sa_mla_kernel",
            "mla_us": round(ms_mla * 1e3, 1),
            "mla_cold_mall_us": mla_cold,
            "mla_useful_TFLOPs": round(flop_m / (ms_mla * 1e-3) / 1e12, 1),
            "mla_mfma_frac": round(flop_m / (ms_mla * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "mla_indexer_picks_us": round(ms_mla_real * 1e3, 1),
            "mla_indexer_picks_mfma_frac": round(flop_r / (ms_mla_real * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "mla_algorithmic_bytes": bytes_m,
            "mla_GBps": round(bytes_m / (ms_mla * 1e-3) / 1e9, 1),
            "traffic": {"sa_mla_kernel": _traffic("sa_mla_kernel"), "ix_wide_kernel": _traffic("ix_wide_kernel"),
                        "ix_select_kernel": _traffic("ix_select_kernel")},
        }
        del qm, kvm, idxm, picks, x5, qr5, ix5, mla
        torch.cuda.empty_cache()

    _say("configs[4] prefill done")
    # ---------------- Task2
    t2_cpu_inputs = None
    if not a.no_task2:
        torch.manual_seed(42)
        init = t2.get_init_inputs(device=dev)
        m2 = t2.Model(*init).to(dev)
        g = torch.Generator().manual_seed(5)
        with torch.no_grad():
            for p in (m2.wq_b.weight, m2.weights_proj.weight):
                p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16))
        x, qr, sp, off = t2.get_inputs(device=dev)
        with torch.no_grad():
            _warm(torch, lambda: m2(x, qr, sp, off), a.warmup, 0.2)
            ms2 = _events_time(torch, lambda: m2(x, qr, sp, off), a.steps, stream)
            m2_cold = cold(lambda: m2(x, qr, sp, off), 20)
            # The kernels as Model.forward runs them: both projections in one launch
            # (q rotated, and the head weights), then the fused score / top-k kernel.
            fr = m2.freqs_cis[:2600]
            assert m2.route(x, qr) == "both"
            pq, pw = m2.packed_weights()
            pfn = lambda: _native.indexer_projections(qr, pq, fr, x, pw, 64, 32)
            qp, wl = pfn()
            scale = 64 ** -0.5 * 16 ** -0.5
            kfn = lambda: _native.indexer_score_topk(qp, m2.kv_cache, wl, scale, None, 32, 650, 128, 4, True, 0)
            _warm(torch, kfn, 3, 0.1)
            msk = _events_time(torch, kfn, a.steps, stream)
            k_cold = cold(kfn, 20)
            _warm(torch, pfn, 3, 0.1)
            msp = _events_time(torch, pfn, a.steps, stream)
            # torch's two projections for comparison (F.linear; RoPE would then run inside the
            # score kernel), and the query-projection kernel alone (the 'q' route)
            lfn = lambda: (torch.nn.functional.linear(qr, m2.wq_b.weight),
                           torch.nn.functional.linear(x, m2.weights_proj.weight))
            _warm(torch, lfn, 3, 0.1)
            msl = _events_time(torch, lfn, a.steps, stream)
            qfn = lambda: _native.indexer_q_proj(qr, m2.wq_b.weight, fr, 64, 32)
            _warm(torch, qfn, 3, 0.1)
            msq = _events_time(torch, qfn, a.steps, stream)
        kb = t2_kernel_bytes()
        proj_flop = 2 * 8 * 2600 * (1024 * 256 + 16 * 1024)
        # qr and x read, both weights read, q and wl written, the RoPE table rows read
        proj_bytes = (8 * 2600 * 256 * 2 + 8 * 2600 * 1024 * 2 + 1024 * 256 * 2 + 16 * 1024 * 2
                      + 8 * 2600 * 1024 * 2 + 8 * 2600 * 16 * 2 + 2600 * 16 * 8)
        score_flop = 2 * 16 * 64 * sum(((t + 1) // 4) for t in range(2600)) * 8
        result["task2"] = {
            "workload": "task2_indexer configs[2]: x[8,2600,1024], qr[8,2600,256], kv_cache[8,650,64], "
                        "W ~ N(0,0.02), top-128, causal, ratio 4",
            "us_per_call": round(ms2 * 1e3, 2),
            "cold_mall_us_per_call": m2_cold,
            "model_bytes": t2_bytes(),
            "model_GBps": round(t2_bytes() / (ms2 * 1e-3) / 1e9, 1),
            "fused_kernel": "ix_score_topk_kernel",
            "fused_kernel_us": round(msk * 1e3, 2),
            "fused_kernel_cold_mall_us": k_cold,
            "fused_kernel_bytes": kb,
            "fused_kernel_useful_score_flop": score_flop,
            # The kernel is bound by neither roof (VALU: rounding chain + selection); both
            # fractions are reported, the HBM one as "roofline".
            "roofline": _roofline_hbm(kb, msk, _traffic("ix_score_topk_kernel")),
            "roofline_mfma": _roofline_mfma(score_flop, msk),
            "projections": {
                "kernel": "ix_proj2_kernel (one launch: q = RoPE(qr . wq_b^T) and wl = x . weights_proj^T, "
                          "bit-equal to F.linear + apply_rotary_emb and F.linear)",
                "us": round(msp * 1e3, 2),
                "flop": proj_flop,
                "TFLOPs": round(proj_flop / (msp * 1e-3) / 1e12, 1),
                "bytes": proj_bytes,
                "GBps": round(proj_bytes / (msp * 1e-3) / 1e9, 1),
                "roofline": _roofline_hbm(proj_bytes, msp, _traffic("ix_proj2_kernel")),
                "roofline_mfma": _roofline_mfma(proj_flop, msp),
                "torch_two_f_linear_us": round(msl * 1e3, 2),
                "q_proj_kernel_alone_us": round(msq * 1e3, 2),
            },
        }
        t2_cpu_inputs = (m2.wq_b.weight.detach().cpu(), m2.weights_proj.weight.detach().cpu(),
                         init[2].cpu(), x.cpu(), qr.cpu())
        del x, qr, qp, wl, m2

    if not a.no_decode:
        result["dsa_decode_c5"] = dsa_decode

    _say("configs[2] done")
    # ---------------- The reference path on the host CPU cores (the oracle's restatement
    # of the reference modules), on the same seeded inputs, after every GPU leg.
    if not a.no_cpu:
        from oracle import indexer as oix
        from oracle import sparse_attn as osa
        torch.set_num_threads(ncores)
        sink = torch.zeros(64)
        where = f"{ncores} threads of {cpu_model}"
        s1 = _cpu_median_s(lambda: osa.sparse_attn_ref(q1c, kv1c, sink, idx1c, 128 ** -0.5), 3, 20)
        result["task1_c1"].update({"cpu_us_per_call": round(s1 * 1e6, 1), "cpu_threads": ncores,
                                   "cpu_model": cpu_model, "cpu_runs": "3 warm-up + median of 20"})
        s2 = _cpu_median_s(lambda: osa.sparse_attn_ref(q_cpu, kv_cpu, sink, idx_cpu, 128 ** -0.5), 1, 5)
        result["cpu_baseline"] = {
            "value": round(nb / s2 / 1e9, 3), "unit": "GB/s", "cores": ncores, "kind": "port",
            "us_per_call": round(s2 * 1e6, 1),
            "sample": f"the whole configs[1] workload (q[8,2600,64,128], the headline's seeded inputs), "
                      f"1 warm-up + median of 5 calls of the oracle's sparse_attn_ref on {where}"}
        if t2_cpu_inputs is not None:
            wq, ww, kvc, xc, qrc = t2_cpu_inputs
            frc = oix.precompute_freqs_cis(32, 2600)
            f3 = lambda: oix.indexer_forward(wq, ww, kvc, frc, xc, qrc, 0, 0, 16, 64, 32, 128, 4)
            s3 = _cpu_median_s(f3, 1, 5)
            result["task2"]["cpu_baseline"] = {
                "value": round(t2_bytes() / s3 / 1e9, 3), "unit": "GB/s", "cores": ncores, "kind": "port",
                "us_per_call": round(s3 * 1e6, 1),
                "sample": f"the whole configs[2] Model.forward (x[8,2600,1024], the same weights and inputs), "
                          f"1 warm-up + median of 5 calls of the oracle's indexer_forward on {where}"}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
