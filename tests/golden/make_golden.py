"""Write the golden fixtures of tests/golden/ by running the reference PyTorch modules.

Run once, in the build container where /root/reference is mounted:
    python tests/golden/make_golden.py [/root/reference]
Only the resulting .npz files (inputs and outputs, bf16 stored as uint16 words) are
committed; the reference itself is not copied. Tests load the .npz files and never
read /root/reference.

Recorded change to the reference's behaviour: task2_v0_ref.py creates two arange
tensors with .cuda() inside forward (:136,140) and in get_init_inputs (:169-171).
There is no GPU here, so torch.Tensor.cuda is replaced by the identity while the
fixtures are written; all arithmetic runs on the CPU exactly as written.

Fixtures
  task1_small.npz   task1_v0_ref.Model, b=2 m=12 h=64 d=128 n_kv=32 topk=16 (get_inputs-style
                    draws with replacement), attn_sink = zeros (the reference initial value)
  task1_masked.npz  b=1 m=12 h=16 d=128 n_kv=48 topk=24 with -1 slots, random attn_sink
  task1_c1.npz      the reference's CPU config q[1,160,64,128] under torch.manual_seed(42):
                    output only (inputs are regenerated from the seed; their sha256 is stored)
  task2_small.npz   task2_v0_ref.Model built under torch.manual_seed(42) with a reduced
                    ModelArgs; weights, inputs and outputs for start_pos 0 and 64
  task2_freqs.npz   the RoPE table of task2_v0_ref.get_init_inputs (:162-172) under
                    torch.manual_seed(42): sha256 of freqs_cis and kv_cache, the first and
                    last rows of freqs_cis; the same for the configs[4] table (rope_head_dim
                    64, max_seq_len 8192, through the reference's own get_init_inputs with
                    its _make_args returning those arguments)

    python tests/golden/make_golden.py [/root/reference] [task1|task2|freqs ...]
writes the named fixtures (all of them by default).
"""
from __future__ import annotations

import hashlib
import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load(path: str, name: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def task1(ref_dir: str) -> None:
    t1 = _load(os.path.join(ref_dir, "reference", "task1_v0_ref.py"), "task1_v0_ref")
    # small, reference-style inputs
    torch.manual_seed(7)
    q = torch.randn(2, 12, 64, 128, dtype=torch.bfloat16)
    kv = torch.randn(2, 32, 128, dtype=torch.bfloat16)
    idx = torch.randint(0, 32, (2, 12, 16), dtype=torch.int32)
    m = t1.Model(64, 128)
    out = m(q, kv, idx)
    np.savez_compressed(os.path.join(HERE, "task1_small.npz"), q=_bits(q), kv=_bits(kv),
                        idx=idx.numpy(), sink=m.attn_sink.detach().numpy(), out=_bits(out),
                        scale=np.float64(m.softmax_scale))
    # masked slots, nonzero sink, n_kv > 32
    torch.manual_seed(8)
    q = torch.randn(1, 12, 16, 128, dtype=torch.bfloat16)
    kv = torch.randn(1, 48, 128, dtype=torch.bfloat16)
    idx = torch.randint(0, 48, (1, 12, 24), dtype=torch.int32)
    idx[0, :, 20:] = -1
    idx[0, 3, :] = -1
    idx[0, 5, :] = 7
    m = t1.Model(16, 128)
    with torch.no_grad():
        m.attn_sink.copy_(torch.randn(16) * 2)
    out = m(q, kv, idx)
    np.savez_compressed(os.path.join(HERE, "task1_masked.npz"), q=_bits(q), kv=_bits(kv),
                        idx=idx.numpy(), sink=m.attn_sink.detach().numpy(), out=_bits(out),
                        scale=np.float64(m.softmax_scale))
    # the reference CPU config, seed 42
    torch.manual_seed(42)
    t1.batch_size, t1.seq_len = 1, 160
    q, kv, idx = t1.get_inputs()
    m = t1.Model(*t1.get_init_inputs())
    out = m(q, kv, idx)
    np.savez_compressed(os.path.join(HERE, "task1_c1.npz"), out=_bits(out),
                        sha_q=np.bytes_(_sha(q)), sha_kv=np.bytes_(_sha(kv)),
                        sha_idx=np.bytes_(_sha(idx)), seed=np.int64(42))


def task2(ref_dir: str) -> None:
    saved = torch.Tensor.cuda
    torch.Tensor.cuda = lambda self, *a, **k: self
    try:
        t2 = _load(os.path.join(ref_dir, "reference", "task2_v0_ref.py"), "task2_v0_ref")
        args = t2.ModelArgs(max_batch_size=2, max_seq_len=256, dim=128, index_n_heads=16,
                            index_head_dim=64, index_topk=32, q_lora_rank=64, rope_head_dim=32)
        torch.manual_seed(42)
        rd = args.rope_head_dim
        freqs = 1.0 / (10000.0 ** (torch.arange(0, rd, 2)[: rd // 2].float() / rd))
        t = torch.arange(args.max_seq_len, dtype=torch.float32)
        freqs_cis = torch.polar(torch.ones(args.max_seq_len, rd // 2), torch.outer(t, freqs)).view(args.max_seq_len, -1)
        kv_cache = torch.randn(2, args.max_seq_len // 4, 64, dtype=torch.bfloat16)
        model = t2.Model(args, freqs_cis, kv_cache, 4)
        x = torch.randn(2, 256, args.dim, dtype=torch.bfloat16)
        qr = torch.randn(2, 256, args.q_lora_rank, dtype=torch.bfloat16)
        out0 = model(x, qr, 0, 0)
        x1 = torch.randn(2, 64, args.dim, dtype=torch.bfloat16)
        qr1 = torch.randn(2, 64, args.q_lora_rank, dtype=torch.bfloat16)
        out1 = model(x1, qr1, 64, 7)
        # RoPE on its own (apply_rotary_emb, task2_v0_ref.py:93-104)
        qrot = torch.randn(1, 64, 16, 64, dtype=torch.bfloat16)
        qrot_in = qrot.clone()
        t2.apply_rotary_emb(qrot[..., -rd:], freqs_cis[:64])
        np.savez_compressed(
            os.path.join(HERE, "task2_small.npz"),
            wq=_bits(model.wq_b.weight.detach()), ww=_bits(model.weights_proj.weight.detach()),
            freqs=torch.view_as_real(freqs_cis).numpy(), kv=_bits(kv_cache),
            x=_bits(x), qr=_bits(qr), out0=out0.numpy(),
            x1=_bits(x1), qr1=_bits(qr1), out1=out1.numpy(),
            rope_in=_bits(qrot_in), rope_out=_bits(qrot),
            cfg=np.array([2, 256, args.dim, args.q_lora_rank, 16, 64, rd, args.index_topk, 4], np.int64))
    finally:
        torch.Tensor.cuda = saved


def freqs(ref_dir: str) -> None:
    saved = torch.Tensor.cuda
    torch.Tensor.cuda = lambda self, *a, **k: self
    try:
        t2 = _load(os.path.join(ref_dir, "reference", "task2_v0_ref.py"), "task2_v0_ref")
        out = {}
        torch.manual_seed(42)
        _, fc, kv, ratio = t2.get_init_inputs()
        out.update(c3_sha=np.bytes_(_sha(torch.view_as_real(fc))), c3_kv_sha=np.bytes_(_sha(kv)),
                   c3_shape=np.array(fc.shape, np.int64), c3_ratio=np.int64(ratio),
                   c3_head=torch.view_as_real(fc[:4]).numpy(), c3_tail=torch.view_as_real(fc[-4:]).numpy())
        orig = t2._make_args
        t2._make_args = lambda: t2.ModelArgs(max_batch_size=1, max_seq_len=8192, dim=7168,
                                             index_n_heads=64, index_head_dim=128, index_topk=2048,
                                             q_lora_rank=1536, rope_head_dim=64)
        try:
            torch.manual_seed(42)
            _, fc, kv, _ = t2.get_init_inputs()
        finally:
            t2._make_args = orig
        out.update(c5_sha=np.bytes_(_sha(torch.view_as_real(fc))), c5_shape=np.array(fc.shape, np.int64),
                   c5_head=torch.view_as_real(fc[:4]).numpy(), c5_tail=torch.view_as_real(fc[-4:]).numpy())
        np.savez_compressed(os.path.join(HERE, "task2_freqs.npz"), **out)
    finally:
        torch.Tensor.cuda = saved


if __name__ == "__main__":
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    which = sys.argv[2:] or ["task1", "task2", "freqs"]
    torch.set_num_threads(1)
    for name in which:
        {"task1": task1, "task2": task2, "freqs": freqs}[name](ref)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
