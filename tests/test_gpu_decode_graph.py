"""A DSA decode step (indexer Model.forward, then sparse MLA over its int64 picks) at
the configs[4] size, captured in a HIP graph through torch.cuda.graph: every replay,
with eager work and synchronisations between replays, equals the eager step bit for
bit. The wrappers allocate their workspaces from torch's caching allocator, which
serves graph capture from the graph's private pool."""
import pytest
import torch

from ascendc_kernel_amd import task1_sparse_attn as t1
from ascendc_kernel_amd import task2_indexer as t2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seqlen", [1, 4])
def test_decode_step_graph_replays_equal_eager(gpu, seqlen):
    torch.manual_seed(42)
    init = t2.get_c5_init_inputs(device=gpu)
    ix = t2.Model(*init).to(gpu)
    gw = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for p in (ix.wq_b.weight, ix.weights_proj.weight):
            p.copy_((torch.randn(p.shape, generator=gw) * 0.02).to(torch.bfloat16))
    attn = t1.Model(128, 576, v_dim=512).to(gpu)
    sp = 8192 - seqlen
    g = torch.Generator().manual_seed(50 + seqlen)
    x = torch.randn(1, seqlen, 7168, generator=g).to(torch.bfloat16).to(gpu)
    qr = torch.randn(1, seqlen, 1536, generator=g).to(torch.bfloat16).to(gpu)
    q = torch.randn(1, seqlen, 128, 576, generator=g).to(torch.bfloat16).to(gpu)
    kv = torch.randn(1, 8192, 576, generator=g).to(torch.bfloat16).to(gpu)
    print(f"case decode graph s={seqlen}", flush=True)
    with torch.no_grad():
        want_idx = ix(x, qr, sp, 0)
        want = attn(q, kv, want_idx)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                attn(q, kv, ix(x, qr, sp, 0))
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            g_idx = ix(x, qr, sp, 0)
            g_out = attn(q, kv, g_idx)
        for r in range(4):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(g_idx, want_idx), f"replay {r}: indices differ"
            assert torch.equal(g_out.view(torch.int16), want.view(torch.int16)), f"replay {r}: output differs"
            torch.randn(4096, device=gpu).sum().item()  # eager work between replays
