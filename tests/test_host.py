"""Host-side surface of the drop-in modules (CPU only, no kernel launches)."""
import pytest
import torch

from ascendc_kernel_amd import task1_sparse_attn as t1
from ascendc_kernel_amd import task2_indexer as t2
from oracle import indexer as oix
from oracle import sparse_attn as osa


def test_task1_surface():
    m = t1.Model(*t1.get_init_inputs())
    r = osa.Model(*osa.get_init_inputs())
    assert list(m.state_dict()) == list(r.state_dict()) == ["attn_sink"]
    assert m.softmax_scale == r.softmax_scale == 128 ** -0.5
    assert torch.equal(m.attn_sink, torch.zeros(64))
    assert t1.ModelNew is t1.Model
    # the module loads a reference state_dict unchanged
    r.attn_sink.data.normal_()
    m.load_state_dict(r.state_dict())
    assert torch.equal(m.attn_sink, r.attn_sink)


def test_task1_get_inputs():
    torch.manual_seed(0)
    q, kv, idx = t1.get_inputs()
    assert q.shape == (8, 2600, 64, 128) and q.dtype == torch.bfloat16
    assert kv.shape == (8, 32, 128) and idx.shape == (8, 2600, 16) and idx.dtype == torch.int32
    torch.manual_seed(0)
    q2, kv2, idx2 = osa.get_inputs()
    assert torch.equal(q, q2) and torch.equal(kv, kv2) and torch.equal(idx, idx2)


def test_task1_rejects_cpu_tensors():
    m = t1.Model(64, 128)
    q = torch.zeros(1, 2, 64, 128, dtype=torch.bfloat16)
    kv = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    idx = torch.zeros(1, 2, 16, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        m(q, kv, idx)
    with pytest.raises(ValueError):
        m(q[:, :, :32], kv, idx)


def test_task2_constructor_rng_and_state_dict():
    args = t2._make_args()
    kv = torch.zeros(8, 650, 64, dtype=torch.bfloat16)
    fr = torch.ones(2600, 16, dtype=torch.complex64)
    torch.manual_seed(123)
    m = t2.Model(args, fr, kv, 4)
    torch.manual_seed(123)
    r = oix.IndexerRef(oix.make_args(), fr, kv, 4)
    assert list(m.state_dict()) == ["wq_b.weight", "weights_proj.weight"]
    assert torch.equal(m.wq_b.weight, r.wq_b.weight)
    assert torch.equal(m.weights_proj.weight, r.weights_proj.weight)
    assert m.wq_b.weight.shape == (1024, 256) and m.weights_proj.weight.shape == (16, 1024)
    assert m.wq_b.scale is None and m.wq_b.bias is None
    assert t2.ModelNew is t2.Model


def test_task2_rejects_cpu_tensors():
    args = t2._make_args()
    kv = torch.zeros(8, 650, 64, dtype=torch.bfloat16)
    fr = torch.ones(2600, 16, dtype=torch.complex64)
    m = t2.Model(args, fr, kv, 4)
    x = torch.zeros(1, 8, 1024, dtype=torch.bfloat16)
    qr = torch.zeros(1, 8, 256, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device"):
        m(x, qr, 0, 0)
    # empty top-k (end_pos // ratio == 0) is an empty result, as in the reference
    out = m(x[:, :3], qr[:, :3], 0, 0)
    assert out.shape == (1, 3, 0) and out.dtype == torch.int64


def test_task2_args_match_reference_config():
    a = t2._make_args()
    assert (a.dim, a.index_n_heads, a.index_head_dim, a.index_topk, a.q_lora_rank, a.rope_head_dim,
            a.max_seq_len, a.max_batch_size) == (1024, 16, 64, 128, 256, 32, 2600, 8)


def test_task1_gather_inputs_properties():
    """configs[3] input builders: token t holds min(t+1, topk) distinct rows of [0, t], rest -1."""
    from oracle import sparse_attn as osa
    g = torch.Generator().manual_seed(3)
    built = [t1.get_gather_inputs(batch_size=2, seq_len=70, n_kv=96, topk=40, device="cpu", seed=5),
             list(osa.gather_inputs(2, 70, 64, 128, 96, 40, generator=g))]
    for q, kv, idx in built:
        assert idx.dtype == torch.int32 and tuple(idx.shape) == (2, 70, 40)
        assert q.dtype == torch.bfloat16 and kv.dtype == torch.bfloat16
        for b in range(2):
            for t in range(70):
                row = idx[b, t]
                n = min(t + 1, 40)
                valid = row[:n]
                assert bool((valid >= 0).all()) and bool((valid <= t).all())
                assert len(set(valid.tolist())) == n
                assert bool((row[n:] == -1).all())


# ---------------------------------------------------------------- projection routing
def test_projection_route_boundaries():
    """Model.forward uses a kernel for the projections only at token counts where its rounding
    was measured equal to F.linear (the interval tables), and only on the measured build."""
    c3 = dict(q_lora_rank=256, rope_head_dim=32, head_dim=64, n_q=1024, dim=1024, n_w=16, bf16=True,
              on_gpu=True, build_ok=True)
    r = lambda m, **kw: t2.projection_route(m, **{**c3, **kw})
    assert r(8 * 2600) == "both"                       # configs[2]
    for a, b in t2.WL_EQUAL:
        for m in (a, b):
            if m >= t2.Q_PROJ_MIN_TOKENS:
                assert r(m) == ("both" if t2._within(m, t2.Q_EQUAL) else "torch")
    for a, b in t2.Q_EQUAL:
        for m in (a - 1, a, b, b + 1):
            inq = t2._within(m, t2.Q_EQUAL) and m >= t2.Q_PROJ_MIN_TOKENS
            want = ("both" if t2._within(m, t2.WL_EQUAL) else "q") if inq else "torch"
            assert r(m) == want, m
    assert r(32768) == "both" and r(32769) == "torch"   # hipBLASLt splits wq_b's k sum above 32,768
    assert r(16384) == "q" and r(16385) == "both"
    assert r(63) == "torch" and r(64) == r(140) == r(15360) == "q" and r(15361) == "both"   # weights_proj
    assert r(8 * 2600, build_ok=False) == "torch"      # another torch / hipBLASLt build or CU count
    assert r(8 * 2600, on_gpu=False) == r(8 * 2600, bf16=False) == "torch"
    assert r(8 * 2600, dim=2048) == r(8 * 2600, n_w=32) == "q"
    assert r(8 * 2600, head_dim=128) == "q"            # the one-launch kernel is head_dim 64 only
    assert r(8 * 2600, q_lora_rank=1536) == r(8 * 2600, rope_head_dim=64) == "torch"   # configs[4]
    assert r(1) == "torch"                             # decode at the configs[2] sizes


def test_projection_route_decode():
    """1..16 tokens at the configs[4] sizes (q_lora_rank 1536, 64 x 128 query channels, dim
    7168, 64 head weights) take the decode launch, on the measured build only; any other
    size or count keeps F.linear."""
    c5 = dict(q_lora_rank=1536, rope_head_dim=64, head_dim=128, n_q=8192, dim=7168, n_w=64, bf16=True,
              on_gpu=True, build_ok=True)
    r = lambda m, **kw: t2.projection_route(m, **{**c5, **kw})
    assert [r(m) for m in range(1, 17)] == ["decode"] * 16
    assert r(0) == r(17) == r(8192) == "torch"
    assert r(1, build_ok=False) == r(1, on_gpu=False) == r(1, bf16=False) == "torch"
    assert r(1, n_q=4096) == r(1, dim=4096) == r(1, n_w=32) == r(1, q_lora_rank=1024) == "torch"


def test_projection_tables_match_measurement():
    """Q_EQUAL / WL_EQUAL are the intervals tests/golden/projection_ranges.json holds (written by
    tests/golden/measure_projection_ranges.py on the build MEASURED_TORCH names), sorted and
    disjoint."""
    import json
    import os
    from conftest import GOLDEN
    with open(os.path.join(GOLDEN, "projection_ranges.json")) as f:
        r = json.load(f)
    assert (r["torch"], r["hip"]) == t2.MEASURED_TORCH and r["cus"] == t2.MEASURED_CUS
    assert [tuple(v) for v in r["q_equal"]] == list(t2.Q_EQUAL)
    assert [tuple(v) for v in r["wl_equal"]] == list(t2.WL_EQUAL)
    for table in (t2.Q_EQUAL, t2.WL_EQUAL):
        assert all(a <= b for a, b in table)
        assert all(table[i][1] + 1 < table[i + 1][0] for i in range(len(table) - 1))
        for a, b in table:
            assert t2._within(a, table) and t2._within(b, table)
            assert not t2._within(a - 1, table) and not t2._within(b + 1, table)


# ---------------------------------------------------------------- steady-state launch plans
class _FakePrepared:
    """Stands in for _native.Prepared, which holds its inputs (`keep`) so that their memory
    cannot go to another tensor at the same address while the plan's key names it."""

    def __init__(self, log, shape, keep):
        self.log, self.shape, self.keep = log, shape, keep

    def run(self):
        self.log.append("run")
        return torch.zeros(self.shape)


def _fake_native(monkeypatch, log):
    from ascendc_kernel_amd import _native
    monkeypatch.setattr(_native, "stream_handle", lambda dev: 1234)
    monkeypatch.setattr(_native, "prepare_sparse_attn",
                        lambda q, kv, idx, sink, scale, variant:
                        log.append("prepare") or _FakePrepared(log, q.shape, (q, kv, idx)))
    monkeypatch.setattr(_native, "prepare_sparse_mla",
                        lambda q, kv, idx, sink, scale, v:
                        log.append("prepare") or _FakePrepared(log, q.shape, (q, kv, idx)))


def test_task1_plan_cache(monkeypatch):
    """The same inputs reuse the prepared launch; a changed pointer, shape, index dtype or an
    in-place update of attn_sink prepares anew (the cache is exercised on CPU tensors with the
    C ABI stubbed out)."""
    from ascendc_kernel_amd import _native
    log = []
    _fake_native(monkeypatch, log)
    m = t1.Model(64, 128)
    monkeypatch.setattr(_native, "PLAN_DEVICE_TYPE", "cpu")
    q = torch.zeros(1, 40, 64, 128, dtype=torch.bfloat16)
    kv = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    idx = torch.zeros(1, 40, 16, dtype=torch.int32)
    for _ in range(3):
        m(q, kv, idx)
    assert log.count("prepare") == 1 and log.count("run") == 3
    m(q.clone(), kv, idx)                              # another q pointer
    assert log.count("prepare") == 2
    m(q, kv, idx)                                      # back to the first: the cache holds one plan
    assert log.count("prepare") == 3
    m(q[:, :20].contiguous(), kv, idx[:, :20].contiguous())   # other shapes
    assert log.count("prepare") == 4
    m(q, kv, idx)
    with torch.no_grad():
        m.attn_sink.add_(1.0)                          # in-place parameter update
    m(q, kv, idx)
    assert log.count("prepare") == 6
    m(q, kv, idx.long())                               # int64 indices
    assert log.count("prepare") == 7
    m(q, kv, idx.long().contiguous())
    assert log.count("prepare") == 8                   # a new int64 tensor, new pointer


def test_task2_plan_cache(monkeypatch):
    """Model.forward of Task2 keeps one plan per (inputs, positions, weights, cache, stream):
    changing start_pos, offset, an input pointer or a weight's version builds a new one."""
    built = []

    class FakePlan:
        def __init__(self, model, x, qr, start_pos, offset, key):
            self.key = key
            built.append((start_pos, offset))

        def run(self):
            return torch.zeros(1)

    from ascendc_kernel_amd import _native
    monkeypatch.setattr(t2, "_IndexerPlan", FakePlan)
    monkeypatch.setattr(_native, "stream_handle", lambda dev: 99)
    monkeypatch.setattr(_native, "PLAN_DEVICE_TYPE", "cpu")
    a = t2._make_args()
    m = t2.Model(a, torch.ones(2600, 16, dtype=torch.complex64), torch.zeros(8, 650, 64, dtype=torch.bfloat16))
    x = torch.zeros(1, 64, 1024, dtype=torch.bfloat16)
    qr = torch.zeros(1, 64, 256, dtype=torch.bfloat16)
    for _ in range(3):
        m(x, qr, 0, 0)
    assert built == [(0, 0)]
    m(x, qr, 64, 0)
    m(x, qr, 64, 5)
    assert built == [(0, 0), (64, 0), (64, 5)]
    m(x.clone(), qr, 64, 5)
    assert len(built) == 4
    with torch.no_grad():
        m.weights_proj.weight.mul_(2)
    m(x.clone(), qr, 64, 5)
    assert len(built) == 5
