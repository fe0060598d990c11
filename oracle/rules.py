"""Bit-level rules of the Task2 rounding chain, stated in numpy.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Each rule is an independent statement (no torch arithmetic) of one step of
reference/task2_v0_ref.py:123-144 as torch executes it on a given device. Tests
check torch (CPU and, on the GPU box, torch-ROCm) against these rules, which
pins the torch restatement in oracle/indexer.py stage by stage, and check the
HIP kernel against the same rules.

  bf16_round      IEEE round-to-nearest-even fp32 -> bf16 (every .to(bf16)/copy_)
  rope            complex product of apply_rotary_emb (task2_v0_ref.py:93-104):
                  'cpu'        re = (a*c) - (b*d), im = (a*d) + (b*c), products rounded;
                  'torch_rocm' torch-ROCm's broadcast multiply: unroll slot (n//128)%4 < 3
                               re = fma(a, c, -(b*d)), im = fma(b, c, a*d); slot 3
                               re = fma(-b, d, a*c),  im = (a*d) + (b*c)
  head_sum        fp32 sum over the heads (task2_v0_ref.py:134): 'rocm' = four running
                  accumulators over heads j, j+4, j+8, j+12, combined ((a0+a1)+a2)+a3
                  (16 heads; 64 heads when torch does not split them); 'rocm_split2' =
                  that over the even and over the odd heads, then even + odd;
                  'rocm_split4' = that over heads y, y+4, ... for y = 0..3, then
                  (t0 + t2) + (t1 + t3); 'seq' = one accumulator in head order
  torch_head_split  how many threads torch-ROCm's reduction kernel splits 64 heads over
                  (1, 2 or 4) for a candidate count T and N = b*s*T outputs
  score_chain     bf16(head_sum(bf16(relu(bf16(S)) * w)))
  topk_order      indices of the k largest bf16 values, value descending then index
                  ascending (a stable order); -1/offset fill of task2_v0_ref.py:139-143
  topk_torch      torch-ROCm's topk(sorted=True) order: the k picks are gathered as
                  [values > k-th, index order] + [values == k-th, index order]; for k > 32
                  a stable sort by value follows (= topk_order); for 2 <= k <= 32 torch
                  sorts the gathered list with its 32-slot bitonic network, whose
                  compare-exchange also swaps equal values when the step's direction
                  flag is false, so tie order is that network's (stated in bitonic32)
FMA is emulated with x86 long double (64-bit significand): a*c is exact there and
the one rounding of the sum to long double precedes the rounding to fp32; a wrong
double rounding needs the sum to land within 2^-64 relative of an fp32 tie.
"""
from __future__ import annotations

import numpy as np

_LD = np.longdouble


def bf16_round(x) -> np.ndarray:
    """fp32 -> bf16 bits (uint16), round to nearest even; NaN -> quiet NaN."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    out = ((u + r) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _fma32(a, b, c) -> np.ndarray:
    return (_LD(1) * np.asarray(a, np.float32) * np.asarray(b, np.float32)
            + np.asarray(c, np.float32)).astype(np.float32)


def rope(a, b, c, d, mode: str, n=None):
    """(re, im) in fp32 of (a + ib)(c + id) with the given torch rounding."""
    a, b, c, d = (np.asarray(v, np.float32) for v in (a, b, c, d))
    ac, bd, ad, bc = a * c, b * d, a * d, b * c  # numpy fp32 products: one rounding each
    if mode == "cpu":
        return (ac - bd).astype(np.float32), (ad + bc).astype(np.float32)
    if mode != "torch_rocm":
        raise ValueError(mode)
    slot3 = ((np.asarray(n, np.int64) >> 7) & 3) == 3
    re = np.where(slot3, _fma32(-b, d, ac), _fma32(a, c, -bd))
    im = np.where(slot3, (ad + bc).astype(np.float32), _fma32(b, c, ad))
    return re.astype(np.float32), im.astype(np.float32)


def rope_bf16(q_bits, freqs, rd: int, mode: str, flat_offset: int = 0) -> np.ndarray:
    """RoPE of q (bf16 bits [b, s, h, d]) on its last rd channels; freqs [s, rd/2, 2] fp32."""
    q = np.array(q_bits, dtype=np.uint16, copy=True)
    b, s, h, dd = q.shape
    x = bf16_to_f32(q[..., dd - rd:]).reshape(b, s, h, rd // 2, 2)
    fr = np.asarray(freqs, np.float32).reshape(1, s, 1, rd // 2, 2)
    n = np.arange(b * s * h * (rd // 2), dtype=np.int64).reshape(b, s, h, rd // 2) + flat_offset
    re, im = rope(x[..., 0], x[..., 1], np.broadcast_to(fr[..., 0], x[..., 0].shape),
                  np.broadcast_to(fr[..., 1], x[..., 0].shape), mode, n)
    q[..., dd - rd:] = bf16_round(np.stack([re, im], -1).reshape(b, s, h, rd))
    return q


def head_sum(v, order: str = "rocm") -> np.ndarray:
    """fp32 sum over the last axis (the heads) in torch's accumulation order.

    'rocm'        one thread, four accumulators over heads j, j+4, j+8, ... combined
                  ((a0+a1)+a2)+a3 (torch-ROCm's reduction of a short middle dimension,
                  e.g. 16 heads);
    'rocm_split2' two threads over the even and the odd heads, each as 'rocm' over its
                  heads (accumulator i of thread y: heads y+2i+8m), then even + odd;
    'rocm_split4' four threads over heads y, y+4, ..., each as 'rocm' over its heads,
                  then (t0 + t2) + (t1 + t3) (torch-ROCm's halving tree);
                  for 64 heads torch_head_split says which of 'rocm' (1 thread),
                  'rocm_split2' and 'rocm_split4' torch uses;
    'seq'         one accumulator in head order."""
    v = np.asarray(v, np.float32)
    if order == "rocm_split2":
        if v.shape[-1] % 8:
            raise ValueError(order)
        even = head_sum(v[..., 0::2], "rocm")
        odd = head_sum(v[..., 1::2], "rocm")
        return (even + odd).astype(np.float32)
    if order == "rocm_split4":
        if v.shape[-1] % 16:
            raise ValueError(order)
        t = [head_sum(v[..., y::4], "rocm") for y in range(4)]
        return ((t[0] + t[2]).astype(np.float32) + (t[1] + t[3]).astype(np.float32)).astype(np.float32)
    if order == "seq":
        acc = np.zeros(v.shape[:-1], np.float32)
        for i in range(v.shape[-1]):
            acc = (acc + v[..., i]).astype(np.float32)
        return acc
    if order != "rocm" or v.shape[-1] % 4:
        raise ValueError(order)
    accs = []
    for j in range(4):
        acc = np.zeros(v.shape[:-1], np.float32)
        for i in range(j, v.shape[-1], 4):
            acc = (acc + v[..., i]).astype(np.float32)
        accs.append(acc)
    return (((accs[0] + accs[1]).astype(np.float32) + accs[2]).astype(np.float32) + accs[3]).astype(np.float32)


def torch_head_split(n_out: int, t: int) -> int:
    """Threads over which torch-ROCm's reduction kernel splits a 64-long middle dimension
    (x[b, s, 64, T].sum(dim=2), N = b*s*T outputs): the output is vectorised by 4, 2 or 1
    (the largest that divides T); a block is min(pow2(N / vec), 64) threads wide out of
    512 / vec, as tall as fits (at most 64), and the heads are split over its height only
    if each thread keeps at least 16 of them. T = 1 is reduced along another path."""
    vec = 4 if t % 4 == 0 else 2 if t % 2 == 0 else 1
    max_thr = 512 // vec
    dim0 = n_out // vec
    p2 = 1
    while p2 * 2 <= dim0 and p2 < max_thr:
        p2 *= 2
    height = min(64, max_thr // min(p2, 64))
    return height if 64 >= 16 * height else 1


def head_sum_order_64(n_out: int, t: int) -> str:
    """head_sum order name of torch-ROCm's 64-head sum for (N, T)."""
    return {1: "rocm", 2: "rocm_split2", 4: "rocm_split4"}[torch_head_split(n_out, t)]


def score_chain(s_bits, w_bits, order: str = "rocm") -> np.ndarray:
    """bf16 score bits [..., T] from S bits [..., H, T] and w bits [..., H] (head-sum order
    as in head_sum)."""
    s = bf16_to_f32(s_bits)
    s = np.maximum(s, np.float32(0))
    w = bf16_to_f32(w_bits)[..., None]
    prod = bf16_to_f32(bf16_round(s * w))            # bf16 x bf16 product, exact in fp32, one RNE
    tot = head_sum(np.moveaxis(prod, -2, -1), order)
    return bf16_round(tot)


def weights_bits(wl_bits, scale: float) -> np.ndarray:
    """bf16(fp32(wl) * fp32(scale)) (task2_v0_ref.py:132)."""
    return bf16_round(bf16_to_f32(wl_bits) * np.float32(scale))


def order_key(bits) -> np.ndarray:
    """Monotone uint16 key of bf16 values (NaN highest, -0 just below +0)."""
    u = np.asarray(bits, np.uint16).astype(np.uint32)
    k = np.where(u & 0x8000, u ^ 0xFFFF, u ^ 0x8000)
    k = np.where((u & 0x7FFF) > 0x7F80, 0xFFFF, k)
    return k.astype(np.uint32)


def topk_order(score_bits, k: int, n_valid=None) -> np.ndarray:
    """[rows, T] bf16 bits -> [rows, k] indices, value desc / index asc; entries at or beyond
    n_valid[row] count as -inf (ranked last, by index)."""
    sb = np.asarray(score_bits, np.uint16)
    rows, t = sb.shape
    key = order_key(sb).astype(np.int64)
    if n_valid is not None:
        col = np.arange(t)[None, :]
        key = np.where(col < np.asarray(n_valid)[:, None], key, -1)
    comp = key * 65536 + (65535 - np.arange(t)[None, :])
    order = np.argsort(-comp, axis=1, kind="stable")
    return order[:, :k]


def fill(idx, n_r, causal: bool, offset: int) -> np.ndarray:
    """task2_v0_ref.py:139-143 given the per-row causal limits n_r = (t+1)//ratio."""
    idx = np.asarray(idx, np.int64)
    if causal:
        return np.where(idx >= np.asarray(n_r)[:, None], -1, idx + offset)
    return idx + offset


def _float_key(bits) -> np.ndarray:
    """order_key with -0 and +0 merged: the ordering of float comparison (NaN highest)."""
    k = order_key(bits)
    return np.where(k == 0x7FFF, 0x8000, k)


def bitonic32(keys, vals, n: int):
    """torch's small bitonic key/value sort, descending: 32 slots, slots >= n invalid (sort
    last). Stages: size 2,4,8,16 with direction flag = bit (size/2) of the comparator's
    thread id (the slot pair's lower slot with the stride bit removed), then a final merge
    with flag false. A pair (A lower, B upper) exchanges when
    ((A > B and A valid) or B invalid) == flag."""
    ks = [int(x) for x in keys] + [0] * (32 - len(keys))
    vs = [int(x) for x in vals] + [0] * (32 - len(vals))
    ok = [i < n for i in range(32)]

    def step(size, stride, final):
        for tid in range(16):
            lo = 2 * tid - (tid & (stride - 1))
            hi = lo + stride
            flag = False if final else bool(tid & (size // 2))
            swap = (ks[lo] > ks[hi] and ok[lo]) or not ok[hi]
            if swap == flag:
                ks[lo], ks[hi] = ks[hi], ks[lo]
                vs[lo], vs[hi] = vs[hi], vs[lo]
                ok[lo], ok[hi] = ok[hi], ok[lo]

    size = 2
    while size < 32:
        stride = size // 2
        while stride > 0:
            step(size, stride, False)
            stride //= 2
        size *= 2
    stride = 16
    while stride > 0:
        step(32, stride, True)
        stride //= 2
    return vs[:n]


def topk_torch(score_bits, k: int) -> np.ndarray:
    """[rows, T] bf16 bits (masked entries already -inf) -> [rows, k] indices in the order
    torch-ROCm's topk(k, sorted=True) returns them."""
    sb = np.asarray(score_bits, np.uint16)
    rows, t = sb.shape
    key = order_key(sb).astype(np.int64)
    if k > 32:
        return topk_order(sb, k)
    fkey = _float_key(sb)
    out = np.empty((rows, k), np.int64)
    for r in range(rows):
        kth = np.sort(key[r])[::-1][k - 1]
        gt = np.nonzero(key[r] > kth)[0]
        eq = np.nonzero(key[r] == kth)[0][: k - len(gt)]
        arr = np.concatenate([gt, eq])
        if k <= 1:
            out[r] = arr[:k]
        else:
            out[r] = bitonic32(fkey[r][arr], arr, k)
    return out
