"""The decode projections (dsa_indexer_decode_projections) against torch on the MI355X.

For 1..16 tokens at the configs[4] sizes, Model.forward's two F.linear calls
(task2_v0_ref.py:129 and :132, via Linear.forward :81-83) run on torch-ROCm's
hipBLASLt with k split over 4 waves: in every depth block of 128 (q) or 512 (head
weights) chain c sums the c-th quarter in ascending k, the chains are added as
((c0 + c1) + c2) + c3 and rounded once to bf16. The kernel reproduces that order, so
its outputs equal F.linear's bit for bit:
  * planted inputs: rows of +-2^e values in cancelling pairs at random positions, so
    that a sum taken in another order changes several percent of the outputs after
    rounding (measured: pairing the chains as (c0 + c1) + (c2 + c3) changes 6 % of q and
    8 % of the head weights, interleaving the quarters inside a depth block more);
  * every token count 1..16 with the indexer's distributions (x, qr ~ N(0, 1),
    weights ~ N(0, 0.02)) and with values spread over 2^-12 .. 2^12.
Model.forward takes this launch for 1..16 tokens at these sizes (decode); the end-to-end
indices are compared with the reference module in tests/test_gpu_indexer_wide.py.
"""
import pytest
import torch

from ascendc_kernel_amd import _native
from ascendc_kernel_amd import task2_indexer as t2

pytestmark = pytest.mark.gpu

KQ, NQ, KW, NW = 1536, 8192, 7168, 64


def _say(*a):
    print(*a, flush=True)


def _require_measured_build(dev):
    if not t2._measured_build(dev):
        pytest.skip("hipBLASLt's summation order was measured on torch "
                    f"{t2.MEASURED_TORCH} with {t2.MEASURED_CUS} CUs only")


def _wide(shape, g, dev):
    m = torch.rand(shape, generator=g, device=dev) + 1.0
    e = torch.randint(-12, 13, shape, generator=g, device=dev).float()
    s = torch.where(torch.rand(shape, generator=g, device=dev) < 0.5, -1.0, 1.0)
    return (s * m * torch.exp2(e)).to(torch.bfloat16)


def _planted(n, k, g, dev, frac_pair=0.9, emax=14):
    """Rows of s * 2^e (e in 0..emax) where 90 % of the entries come in pairs (v, -v) at
    random positions, the rest ~ N(0, 1): with x = 1 the exact sum is small while partial
    sums are large, so the summation order shows in the rounded result."""
    e = torch.randint(0, emax + 1, (n, k), generator=g, device=dev).float()
    s = torch.where(torch.rand(n, k, generator=g, device=dev) < 0.5, -1.0, 1.0)
    w = s * torch.exp2(e)
    perm = torch.argsort(torch.rand(n, k, generator=g, device=dev), dim=1)
    npair = int(k * frac_pair) // 2
    a, b, rest = perm[:, :npair], perm[:, npair:2 * npair], perm[:, 2 * npair:]
    w.scatter_(1, b, -w.gather(1, a))
    w.scatter_(1, rest, torch.randn(n, rest.shape[1], generator=g, device=dev))
    return w.to(torch.bfloat16)


def _check(qr, wq, x, wp, tag):
    _say("case", tag)
    q, wl = _native.indexer_decode_projections(qr, wq, x, wp)
    rq = torch.nn.functional.linear(qr, wq)
    rw = torch.nn.functional.linear(x, wp)
    nq = int((q.view(torch.int16) != rq.view(torch.int16)).sum())
    nw = int((wl.view(torch.int16) != rw.view(torch.int16)).sum())
    assert nq == 0 and nw == 0, f"{tag}: q {nq} of {rq.numel()}, wl {nw} of {rw.numel()} outputs differ"


@pytest.mark.parametrize("m", [1, 4, 16])
def test_decode_projections_planted_order(gpu, m):
    _require_measured_build(gpu)
    g = torch.Generator(device=gpu).manual_seed(100 + m)
    wq, wp = _planted(NQ, KQ, g, gpu), _planted(NW, KW, g, gpu)
    qr = torch.ones(1, m, KQ, dtype=torch.bfloat16, device=gpu)
    x = torch.ones(1, m, KW, dtype=torch.bfloat16, device=gpu)
    _check(qr, wq, x, wp, f"planted m={m}")


@pytest.mark.parametrize("dist", ["natural", "wide"])
def test_decode_projections_every_token_count(gpu, dist):
    _require_measured_build(gpu)
    g = torch.Generator(device=gpu).manual_seed(7 if dist == "natural" else 8)
    for m in range(1, 17):
        for rep in range(2):
            if dist == "natural":
                wq = (torch.randn(NQ, KQ, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
                wp = (torch.randn(NW, KW, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
                qr = torch.randn(1, m, KQ, generator=g, device=gpu).to(torch.bfloat16)
                x = torch.randn(1, m, KW, generator=g, device=gpu).to(torch.bfloat16)
            else:
                wq, wp = _wide((NQ, KQ), g, gpu), _wide((NW, KW), g, gpu)
                qr, x = _wide((1, m, KQ), g, gpu), _wide((1, m, KW), g, gpu)
            _check(qr, wq, x, wp, f"{dist} m={m} rep={rep}")


@pytest.mark.parametrize("b,s", [(2, 8), (3, 5), (16, 1)])
def test_decode_projections_batched_rows(gpu, b, s):
    """Token rows from several sequences (b * s <= 16) are independent columns."""
    _require_measured_build(gpu)
    g = torch.Generator(device=gpu).manual_seed(b * 100 + s)
    wq = (torch.randn(NQ, KQ, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    wp = (torch.randn(NW, KW, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    qr = torch.randn(b, s, KQ, generator=g, device=gpu).to(torch.bfloat16)
    x = torch.randn(b, s, KW, generator=g, device=gpu).to(torch.bfloat16)
    _check(qr, wq, x, wp, f"batched {b}x{s}")


def test_model_decode_route(gpu):
    """Model.forward at the configs[4] sizes routes 1..16 tokens through the decode launch
    and more through F.linear."""
    _require_measured_build(gpu)
    init = t2.get_c5_init_inputs(device=gpu)
    m = t2.Model(*init).to(gpu)
    for s, want in ((1, "decode"), (16, "decode"), (17, "torch")):
        x = torch.zeros(1, s, KW, dtype=torch.bfloat16, device=gpu)
        qr = torch.zeros(1, s, KQ, dtype=torch.bfloat16, device=gpu)
        assert m.route(x, qr) == want, s
