"""Measure, for every token count m, whether torch-ROCm's F.linear of the indexer's two
projections (reference/task2_v0_ref.py:129-130 and :132, via Linear.forward :81-83) equals
the library's natural-order kernels bit for bit, and write tests/golden/projection_ranges.json.

Run on an MI355X box (it needs torch-ROCm on a GPU and the built library):
    python tests/golden/measure_projection_ranges.py [mmax] [out.json]
For m = 17 .. mmax (default 131072) it runs dsa_indexer_projections (q = qr . wq_b^T without
RoPE, k = 256, n = 1024; wl = x . weights_proj^T, k = 1024, n = 16) on windows of one set
of random inputs and compares each output tensor with F.linear. hipBLASLt chooses its
algorithm by m; where it splits the k sum (over wave groups, or stream-K tails) the two
differ, but only in a small fraction of the outputs (weights_proj's local split-k: about
1.7e-4 of them at m = 17 .. 8192), which one draw of a few thousand outputs misses. So
every m is compared on at least 2^18 outputs of each product: on as many consecutive
m-row windows of the inputs as that takes (one window for large m). The JSON holds the torch build, the CU count and the maximal intervals of m where
each product is equal; ascendc_kernel_amd/task2_indexer.py carries them as Q_EQUAL and
WL_EQUAL (tests/test_host.py checks the copy).
"""
from __future__ import annotations

import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from ascendc_kernel_amd import _native  # noqa: E402


def intervals(bad: torch.Tensor, lo: int, hi: int):
    out, start = [], None
    for m in range(lo, hi + 1):
        ok = not bool(bad[m])
        if ok and start is None:
            start = m
        if not ok and start is not None:
            out.append([start, m - 1])
            start = None
    if start is not None:
        out.append([start, hi])
    return out


def main():
    mmax = int(sys.argv[1]) if len(sys.argv) > 1 else 131072
    path = sys.argv[2] if len(sys.argv) > 2 else os.path.join(HERE, "projection_ranges.json")
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(123)
    wq = (torch.randn(1024, 256, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    wp = (torch.randn(16, 1024, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    qr = torch.randn(1, mmax, 256, generator=g).to(torch.bfloat16).to(dev)
    x = torch.randn(1, mmax, 1024, generator=g).to(torch.bfloat16).to(dev)
    pq, pw = _native.pack_projection_weights(wq, wp)
    bad = torch.zeros(mmax + 1, 2, dtype=torch.bool, device=dev)
    need = 1 << 18  # outputs compared per product and m
    for m in range(17, mmax + 1):
        windows = min(mmax // m, max(-(-need // (16 * m)), -(-need // (1024 * m))))
        for j in range(windows):
            qs, xs = qr[:, j * m:(j + 1) * m], x[:, j * m:(j + 1) * m]
            q, wl = _native.indexer_projections(qs, pq, None, xs, pw, 64, 32)
            if j * 1024 * m < need:
                bad[m, 0] |= (q.view(1, m, 1024).view(torch.int16) !=
                              torch.nn.functional.linear(qs, wq).view(torch.int16)).any()
            bad[m, 1] |= (wl.view(torch.int16) != torch.nn.functional.linear(xs, wp).view(torch.int16)).any()
        if m % 16384 == 0 or (m < 16384 and m % 2048 == 0):
            torch.cuda.synchronize()
            print("m", m, flush=True)
    bad = bad.cpu()
    res = {"torch": torch.__version__, "hip": torch.version.hip,
           "cus": torch.cuda.get_device_properties(dev).multi_processor_count, "mmax": mmax,
           "q_equal": intervals(bad[:, 0], 17, mmax), "wl_equal": intervals(bad[:, 1], 17, mmax)}
    with open(path, "w") as f:
        json.dump(res, f, indent=1)
    print(path, "q intervals", len(res["q_equal"]), "wl intervals", len(res["wl_equal"]))


if __name__ == "__main__":
    main()
