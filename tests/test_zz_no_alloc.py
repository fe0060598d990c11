"""dsa_indexer_score_topk_noalloc, the allocation-free entry point, on the MI355X.

It runs the 64-head indexer with the library's static scratch array in place of a
caller workspace. Each call is checked against dsa_indexer_score_topk_ws (the same
kernels with a torch-allocated workspace) with torch.equal. The calls run in a row,
the later ones smaller than the first, so a stale key left in the shared array
would show up as a difference.
"""
import pytest
import torch

from ascendc_kernel_amd import _native
from oracle import indexer as oix

pytestmark = pytest.mark.gpu

W_SCALE = 128 ** -0.5 * 64 ** -0.5


def _say(*a):
    print(*a, flush=True)


def _inputs(s, n_cand, start_pos, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, s, 64, 128, generator=g).to(torch.bfloat16).to(dev)
    kv = torch.randn(1, n_cand, 128, generator=g).to(torch.bfloat16).to(dev)
    wl = (torch.randn(1, s, 64, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    fr = oix.precompute_freqs_cis(64, start_pos + s, device=dev)[start_pos:start_pos + s]
    return q, kv, wl, fr


def _noalloc(q, kv, wl, fr, n_cand, k_out, causal, offset):
    lib = _native.load()
    b, s, h, d = q.shape
    frv = torch.view_as_real(fr.contiguous())
    out = torch.empty(b, s, k_out, dtype=torch.int64, device=q.device)
    rc = lib.dsa_indexer_score_topk_noalloc(
        q.data_ptr(), kv.data_ptr(), kv.stride(0), wl.data_ptr(), W_SCALE, frv.data_ptr(),
        _native.DSA_ROPE_TORCH_ROCM, out.data_ptr(), b, s, h, d, 64, n_cand, k_out, 1,
        1 if causal else 0, offset, torch.cuda.current_stream(q.device).cuda_stream)
    assert rc == 0, lib.dsa_strerror(rc)
    return out


# (tokens, candidates, start_pos, top-k, causal, offset); scratch use b*s*n_cand*2 bytes:
# 8 MiB, 2 MiB, 16 KiB, then 2 MiB again with a different causal extent.
CALLS = [
    (512, 8192, 7680, 2048, False, 3),
    (1024, 1024, 0, 256, True, 0),
    (1, 8192, 8191, 2048, False, 0),
    (1024, 1024, 0, 512, True, 7),
]


def test_noalloc_matches_workspace_entry_point(gpu):
    for i, (s, t, sp, k, causal, off) in enumerate(CALLS):
        _say("noalloc call", i, (s, t, sp, k, causal, off))
        q, kv, wl, fr = _inputs(s, t, sp, 100 + i, gpu)
        got = _noalloc(q, kv, wl, fr, t, k, causal, off)
        want = _native.indexer_score_topk(q, kv, wl, W_SCALE, fr, 64, t, k, 1, causal, off,
                                          use_workspace=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}: {int((got != want).any(-1).sum())} rows differ"


def test_noalloc_first_call_inside_graph_capture(gpu):
    """The header's claim that the entry point works under HIP graph capture, with its first
    call of the process inside the capture: run in a fresh child process
    (tests/noalloc_capture_child.py), which replays the graph over new inputs and checks every
    replay against the workspace entry point and that the replays allocate nothing."""
    import os
    import subprocess
    import sys
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_child.py")
    _say("noalloc first call inside graph capture (child process)")
    r = subprocess.run([sys.executable, "-u", child], capture_output=True, text=True, timeout=240)
    _say(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and r.stdout.strip().endswith("OK")
