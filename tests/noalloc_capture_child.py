"""Child process of tests/test_zz_no_alloc.py::test_noalloc_first_call_inside_graph_capture.

The first dsa_indexer_score_topk_noalloc call of this process (hence its first use of the
static scratch array: the hipGetSymbolAddress lookup, the kernels' LDS limits and code
loading) is made while torch captures a HIP graph. The graph is replayed over two input
sets, twice each, with new inputs copied into the captured buffers; every replay must equal
dsa_indexer_score_topk_ws with a torch workspace (called only after the replays), and the
replays must not allocate (torch.cuda.memory_allocated before and after). Prints OK.
"""
import os
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from ascendc_kernel_amd import _native  # noqa: E402
from oracle import indexer as oix  # noqa: E402

W_SCALE = 128 ** -0.5 * 64 ** -0.5
S, T, K = 256, 2048, 512


def main():
    dev = torch.device("cuda:0")

    def inputs(seed):
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(1, S, 64, 128, generator=g).to(torch.bfloat16).to(dev)
        kv = torch.randn(1, T, 128, generator=g).to(torch.bfloat16).to(dev)
        wl = (torch.randn(1, S, 64, generator=g) * 0.5).to(torch.bfloat16).to(dev)
        return q, kv, wl

    fr = oix.precompute_freqs_cis(64, T, device=dev)[T - S:T]
    frv = torch.view_as_real(fr.contiguous())
    lib = _native.load()
    sets = [inputs(1), inputs(2)]
    q_s, kv_s, wl_s = [t.clone() for t in sets[0]]
    out_s = torch.empty(1, S, K, dtype=torch.int64, device=dev)
    got = [torch.empty_like(out_s) for _ in range(4)]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(graph):
        rcs.append(lib.dsa_indexer_score_topk_noalloc(
            q_s.data_ptr(), kv_s.data_ptr(), kv_s.stride(0), wl_s.data_ptr(), W_SCALE, frv.data_ptr(),
            _native.DSA_ROPE_TORCH_ROCM, out_s.data_ptr(), 1, S, 64, 128, 64, T, K, 1, 0, 0,
            torch.cuda.current_stream().cuda_stream))
    print("capture rc", rcs, flush=True)
    assert rcs == [0], lib.dsa_strerror(rcs[0])
    torch.cuda.synchronize()
    mem0 = torch.cuda.memory_allocated()
    for i, (q, kv, wl) in enumerate(sets * 2):
        q_s.copy_(q)
        kv_s.copy_(kv)
        wl_s.copy_(wl)
        graph.replay()
        torch.cuda.synchronize()
        got[i].copy_(out_s)
    torch.cuda.synchronize()
    mem1 = torch.cuda.memory_allocated()
    for i, (q, kv, wl) in enumerate(sets * 2):
        want = _native.indexer_score_topk(q, kv, wl, W_SCALE, fr, 64, T, K, 1, False, 0, use_workspace=True)
        torch.cuda.synchronize()
        print("replay", i, "equal", bool(torch.equal(got[i], want)), flush=True)
        assert torch.equal(got[i], want), i
    print("memory_allocated across the replays", mem0, mem1, flush=True)
    assert mem0 == mem1
    print("OK", flush=True)


if __name__ == "__main__":
    main()
