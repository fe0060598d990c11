"""Measure torch-ROCm's fp32 summation order for x.sum(dim=2), x bf16 [1, s, 64, T] (the head
sum of reference/task2_v0_ref.py:134 at 64 heads), and write tests/golden/torch_head_split.npz.

Run on an MI355X box (it needs torch-ROCm on a GPU):
    python tests/golden/measure_torch_head_split.py [out.npz]
For each (s, T) the planted input holds small N(0,1) values and eight exactly cancelling
pairs of large values per output, so that every summation order rounds differently. Each
candidate order "Y threads over heads y, y+Y, ..., four accumulators each, combined
((a0+a1)+a2)+a3, thread totals in a halving tree" (Y = 1, 2, 4, 8, 16) is evaluated in
numpy and compared bit for bit with torch's result; the fixture keeps N = s*T, T, the one
Y whose order matches every output, and the mismatch count of each candidate.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import rules  # noqa: E402

YS = (1, 2, 4, 8, 16)
TS = [2, 3, 4, 5, 6, 7, 8, 12, 15, 16, 17, 30, 31, 32, 33, 34, 62, 63, 64, 65, 66, 67, 68, 100, 126,
      127, 128, 129, 130, 131, 132, 190, 254, 255, 256, 257, 258, 259, 260, 510, 514, 515, 1026, 1027,
      4094, 4098, 4099, 8189, 8190, 8191, 8192]
SS = [1, 2, 3, 4, 8, 40, 129]


def planted(s, t, g):
    x = torch.randn(1, s, 64, t, generator=g)
    perm = torch.argsort(torch.rand(1, s, t, 64, generator=g), dim=-1)
    big = torch.exp2(torch.randint(14, 21, (1, s, t, 8), generator=g).float()) * (
        1 + torch.randint(0, 128, (1, s, t, 8), generator=g).float() / 128)
    xt = x.permute(0, 1, 3, 2).contiguous()
    xt.scatter_(-1, perm[..., :8], big)
    xt.scatter_(-1, perm[..., 8:16], -big)
    return xt.permute(0, 1, 3, 2).contiguous().to(torch.bfloat16)


def split_sum(v, y_threads):
    """v [..., 64] fp32: thread y sums heads y + Y*j with four accumulators (j % 4), combined
    ((a0+a1)+a2)+a3; the thread totals meet in a halving tree."""
    tot = []
    for y in range(y_threads):
        hs = list(range(y, 64, y_threads))
        acc = [np.zeros(v.shape[:-1], np.float32) for _ in range(4)]
        for j, h in enumerate(hs):
            acc[j % 4] = (acc[j % 4] + v[..., h]).astype(np.float32)
        tot.append((((acc[0] + acc[1]).astype(np.float32) + acc[2]).astype(np.float32) + acc[3]).astype(np.float32))
    off = y_threads // 2
    while off:
        for y in range(off):
            tot[y] = (tot[y] + tot[y + off]).astype(np.float32)
        off //= 2
    return tot[0]


def main(out_path):
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(11)
    rows = []
    for s in SS:
        for t in TS:
            if s * t > 300_000:
                continue
            x = planted(s, t, g)
            got = x.to(dev).sum(dim=2).cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
            xs = np.moveaxis(rules.bf16_to_f32(x.contiguous().view(torch.int16).numpy().view(np.uint16)), 2, -1)
            miss = [int((got != rules.bf16_round(split_sum(xs, y))).sum()) for y in YS]
            ok = [y for y, m in zip(YS, miss) if m == 0]
            print(f"s={s} T={t} N={s * t} mismatches {dict(zip(YS, miss))} -> {ok}", flush=True)
            rows.append((s * t, t, ok[0] if len(ok) == 1 else -1, *miss))
    a = np.array(rows, np.int64)
    np.savez_compressed(out_path, n_out=a[:, 0], t=a[:, 1], y=a[:, 2], mismatches=a[:, 3:],
                        candidates=np.array(YS, np.int64), torch_version=np.bytes_(torch.__version__))
    print("wrote", out_path, len(rows), "rows;", int((a[:, 2] < 0).sum()), "without a unique order")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else os.path.join(HERE, "torch_head_split.npz"))
