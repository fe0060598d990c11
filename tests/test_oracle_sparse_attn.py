"""Pins the Task1 oracle (oracle/sparse_attn.py) on the CPU.

Checks: the golden fixtures written by the reference itself (tests/golden/make_golden.py),
an independent fp64 brute force, and closed forms chosen so that a dropped sink
term, a missing scale, a wrong mask or a transposed operand each fail a test.
"""
import math
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, bf16_from_bits, bits_of
from oracle import sparse_attn as osa


def _fixture(name):
    return np.load(os.path.join(GOLDEN, name))


@pytest.mark.parametrize("name", ["task1_small.npz", "task1_masked.npz"])
def test_fixture_bit_exact(name):
    f = _fixture(name)
    q, kv = bf16_from_bits(f["q"]), bf16_from_bits(f["kv"])
    idx = torch.from_numpy(f["idx"])
    sink = torch.from_numpy(f["sink"])
    out = osa.sparse_attn_ref(q, kv, sink, idx, float(f["scale"]))
    assert np.array_equal(bits_of(out), f["out"])


def test_fixture_c1_reference_config():
    f = _fixture("task1_c1.npz")
    torch.manual_seed(int(f["seed"]))
    q, kv, idx = osa.get_inputs(batch_size=1, seq_len=160)
    import hashlib
    sha = lambda t: hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()
    if sha(q) != f["sha_q"].item().decode():
        pytest.skip("torch CPU RNG stream differs from the fixture's")
    assert sha(kv) == f["sha_kv"].item().decode() and sha(idx) == f["sha_idx"].item().decode()
    m = osa.Model(*osa.get_init_inputs())
    out = m(q, kv, idx)
    assert np.array_equal(bits_of(out), f["out"])


def _rand(b, m, h, d, n_kv, topk, seed, masked=0.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, m, h, d, generator=g).to(torch.bfloat16)
    kv = torch.randn(b, n_kv, d, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, n_kv, (b, m, topk), generator=g, dtype=torch.int32)
    if masked:
        idx[torch.rand(b, m, topk, generator=g) < masked] = -1
    sink = torch.randn(h, generator=g)
    return q, kv, idx, sink


def test_fp64_bruteforce():
    q, kv, idx, sink = _rand(2, 5, 4, 16, 9, 6, seed=1, masked=0.3)
    ref = osa.sparse_attn_fp64(q, kv, sink, idx, 16 ** -0.5)
    out = osa.sparse_attn_ref(q, kv, sink, idx, 16 ** -0.5).double().numpy()
    # bf16 output: within one bf16 rounding of the exact value
    assert np.all(np.abs(out - ref) <= np.abs(ref) * 2 ** -8 + 1e-6)


def test_all_masked_is_zero():
    q, kv, idx, sink = _rand(1, 3, 4, 16, 8, 5, seed=2)
    idx[:] = -1
    out = osa.sparse_attn_ref(q, kv, sink, idx, 0.25)
    assert torch.count_nonzero(out) == 0


def test_zero_query_uniform_weights_with_sink():
    # q = 0: every valid slot scores 0; with sink 0 the weights are 1/(n_valid + 1).
    q, kv, idx, _ = _rand(1, 4, 4, 16, 8, 5, seed=3, masked=0.4)
    q.zero_()
    sink = torch.zeros(4)
    out = osa.sparse_attn_ref(q, kv, sink, idx, 0.25).double()
    kvd = kv.double()
    for mi in range(4):
        sel = [int(j) for j in idx[0, mi] if j >= 0]
        exp = sum((kvd[0, j] for j in sel), torch.zeros(16, dtype=torch.float64)) / (len(sel) + 1)
        for hi in range(4):
            assert torch.allclose(out[0, mi, hi], exp, atol=1e-2, rtol=2 ** -8)


def test_single_index_closed_form():
    # all slots = j: out = kv_j * t e^s / (t e^s + e^sink)
    q, kv, idx, sink = _rand(1, 2, 3, 32, 6, 4, seed=4)
    idx[:] = 5
    scale = 32 ** -0.5
    out = osa.sparse_attn_ref(q, kv, sink, idx, scale).double()
    for mi in range(2):
        for hi in range(3):
            s = float(q[0, mi, hi].double() @ kv[0, 5].double()) * scale
            w = 4 * math.exp(s) / (4 * math.exp(s) + math.exp(float(sink[hi])))
            assert torch.allclose(out[0, mi, hi], w * kv[0, 5].double(), atol=1e-6, rtol=2 ** -7)


def test_slot_permutation_invariance():
    q, kv, idx, sink = _rand(2, 8, 4, 32, 10, 7, seed=5, masked=0.2)
    perm = torch.randperm(7, generator=torch.Generator().manual_seed(9))
    a = osa.sparse_attn_ref(q, kv, sink, idx, 0.2).float()
    b = osa.sparse_attn_ref(q, kv, sink, idx[..., perm], 0.2).float()
    assert torch.allclose(a, b, atol=1e-2, rtol=2 ** -7)


def test_value_width_extension():
    """v_dim (sparse MLA): v_dim = d is the reference path itself; v_dim < d matches the
    independent fp64 loop (keys = kv[..., :d_qk], values = kv[..., :v_dim])."""
    g = torch.Generator().manual_seed(17)
    q = torch.randn(1, 3, 4, 24, generator=g).to(torch.bfloat16)
    kv = torch.randn(1, 10, 24, generator=g).to(torch.bfloat16)
    idx = torch.randint(-1, 10, (1, 3, 6), generator=g, dtype=torch.int32)
    sink = torch.randn(4, generator=g)
    same = osa.sparse_attn_ref(q, kv, sink, idx, 0.2, v_dim=24)
    assert torch.equal(same, osa.sparse_attn_ref(q, kv, sink, idx, 0.2))
    got = osa.sparse_attn_ref(q, kv, sink, idx, 0.2, v_dim=16).float().numpy()
    want = osa.sparse_attn_fp64(q, kv, sink, idx, 0.2, v_dim=16)
    assert got.shape == (1, 3, 4, 16)
    assert np.allclose(got, want, atol=1e-2, rtol=1e-2)
    # keys wider than the query: only the first d_qk channels enter the scores
    kv2 = torch.cat([kv, torch.randn(1, 10, 8, generator=g).to(torch.bfloat16)], dim=-1)
    assert torch.equal(osa.sparse_attn_ref(q, kv2, sink, idx, 0.2, v_dim=16),
                       osa.sparse_attn_ref(q, kv, sink, idx, 0.2, v_dim=16))
