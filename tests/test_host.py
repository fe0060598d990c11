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
