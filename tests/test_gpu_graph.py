"""The C-ABI forward and backward captured into a HIP graph (torch.cuda.graph)
and replayed: the backward's second-stream fork and join (the intra-chunk VJP
and the query-side fold on the second stream, events before the key-side fold
and the reductions, the final join) are captured as event dependencies. Each
replay follows other eager work and a synchronization, and must reproduce the
eager results bitwise."""

import pytest
import torch

from oal_amd import _native
from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_captured_forward_backward_replays_match_eager(precision):
    dev = _dev()
    gen = torch.Generator().manual_seed(41)
    b, hq, hkv, n, g = 1, 14, 2, 640, 8
    dt = torch.bfloat16
    q = (torch.randn(b, hq, n, 64, generator=gen) * 0.5).to(dt).to(dev)
    k = (torch.randn(b, hkv, n, 64, generator=gen) * 0.5).to(dt).to(dev)
    v = torch.randn(b, hkv, n, 64, generator=gen).to(dt).to(dev)
    labels = torch.randint(0, g, (hq, 64), generator=gen, dtype=torch.int32)
    labels[:, :g] = torch.arange(g, dtype=torch.int32)
    factor = torch.randn(hq, (g + 1) * (g + 2) // 2, generator=gen, dtype=torch.float64) * 0.4
    c0, lam, gam = (t.float().to(dev) for t in go.expand_factor(factor, query_heads=hq, kernel_eps=0.05))
    labels = labels.to(dev)
    dout = torch.randn(b, hq, n, 64, generator=gen).to(dt).to(dev)
    kw = dict(scale=0.125, floor=0.0, precision=precision)

    def run():
        out, num, den, saved = _native.forward(q, k, v, labels, c0, lam, gam, **kw)
        grads = _native.backward(q, k, v, labels, c0, lam, gam, num, den, saved, dout, None, None,
                                 need_q=True, need_k=True, need_v=True, need_coef=True, **kw)
        return [out, num, den, *grads]

    eager = [t.clone() for t in run()]  # also creates the second stream outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        run()  # warm-up on the capture stream
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        captured = run()
    filler = torch.randn(1 << 20, device=dev)
    for rep in range(3):
        filler.mul_(1.0001).add_(0.5)  # other eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(captured, eager)):
            assert torch.equal(got, want), f"replay {rep}: output {i} differs from the eager run"
