"""The backward's second stream as the caller sees it: one stream.

``oal_backward`` forks the denominator kernels, most of the intra-chunk VJP and
most or all of the query-side fold onto a stream of the library's own, makes the caller's stream wait for events the second
stream recorded before the key-side fold and before the rest of the query-side
fold and the coefficient reductions, and joins it back into the caller's stream
before it returns.
These tests call it on caller-created streams (not the default one), from two
streams in turn, and consume the gradients on the caller's stream right after
the call with no synchronization in between. Every result must be bitwise
equal to the same call on the default stream, so a missing join would show up
as a read of a gradient that is not yet written.
"""

import pytest
import torch

from oal_amd import _native
from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _inputs(dev, n=1000, seed=43, b=2, g=8):
    gen = torch.Generator().manual_seed(seed)
    hq, hkv = 14, 2
    dt = torch.bfloat16
    q = (torch.randn(b, hq, n, 64, generator=gen) * 0.5).to(dt).to(dev)
    k = (torch.randn(b, hkv, n, 64, generator=gen) * 0.5).to(dt).to(dev)
    v = torch.randn(b, hkv, n, 64, generator=gen).to(dt).to(dev)
    labels = torch.randint(0, g, (hq, 64), generator=gen, dtype=torch.int32)
    labels[:, :g] = torch.arange(g, dtype=torch.int32)
    factor = torch.randn(hq, (g + 1) * (g + 2) // 2, generator=gen, dtype=torch.float64) * 0.4
    c0, lam, gam = (t.float().to(dev) for t in go.expand_factor(factor, query_heads=hq, kernel_eps=0.05))
    dout = torch.randn(b, hq, n, 64, generator=gen).to(dt).to(dev)
    return q, k, v, labels.to(dev), c0, lam, gam, dout


def _step(inp, precision="bf16"):
    q, k, v, labels, c0, lam, gam, dout = inp
    kw = dict(scale=0.125, floor=0.0, precision=precision)
    out, num, den, saved = _native.forward(q, k, v, labels, c0, lam, gam, **kw)
    grads = _native.backward(q, k, v, labels, c0, lam, gam, num, den, saved, dout, None, None,
                             need_q=True, need_k=True, need_v=True, need_coef=True, **kw)
    # consumed on the caller's stream at once: copies enqueued after the call
    return [t.clone() for t in (out, num, den, *grads)]


@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_backward_on_caller_streams_is_joined_before_the_next_work(precision):
    """bf16: the matrix-core backward's fork; fp32: the fp32 route's forward and
    backward forks."""
    dev = _dev()
    inp = _inputs(dev)
    ref = _step(inp, precision)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    results = []
    for rep in range(4):
        st = streams[rep % 2]
        st.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(st):
            res = _step(inp, precision)
            # more work on the same stream right behind the copies
            res.append(res[3].float().sum())
        results.append((st, res))
    torch.cuda.synchronize()
    names = ["out", "num", "den", "dq", "dk", "dv", "dc0", "dlam", "dgam"]
    for rep, (_, res) in enumerate(results):
        for name, a, r in zip(names, res, ref):
            assert torch.equal(a, r), f"call {rep}: {name} differs from the default-stream call"
        assert torch.equal(res[-1], ref[3].float().sum())


@pytest.mark.parametrize("n, b, groups", [(8300, 1, 8), (1000, 2, 12)])
def test_other_stream_arrangements_are_joined(n, b, groups):
    """Above 128 chunks per unit (N = 8300: 130) the denominator kernels follow
    the scan on the caller's stream and the query-side fold runs whole on the
    second stream; with more than 8 groups (per-pair coefficients) the dv
    kernel and a quarter of the fold stay on the caller's stream. Each call on
    a caller-created stream must equal the default-stream call bitwise."""
    dev = _dev()
    inp = _inputs(dev, n=n, seed=7, b=b, g=groups)
    ref = _step(inp)
    torch.cuda.synchronize()
    st = torch.cuda.Stream(dev)
    results = []
    for _ in range(2):
        st.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(st):
            res = _step(inp)
            res.append(res[4].float().sum())
        results.append(res)
    torch.cuda.synchronize()
    names = ["out", "num", "den", "dq", "dk", "dv", "dc0", "dlam", "dgam"]
    for rep, res in enumerate(results):
        for name, a, r in zip(names, res, ref):
            assert torch.equal(a, r), f"call {rep}: {name} differs from the default-stream call"
        assert torch.equal(res[-1], ref[4].float().sum())


def test_two_caller_streams_with_their_own_inputs():
    dev = _dev()
    inp_a, inp_b = _inputs(dev, n=700, seed=1), _inputs(dev, n=900, seed=2)
    ref_a, ref_b = _step(inp_a), _step(inp_b)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    sa.wait_stream(torch.cuda.current_stream(dev))
    sb.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(sa):
        res_a = _step(inp_a)
    with torch.cuda.stream(sb):
        res_b = _step(inp_b)
    torch.cuda.synchronize()
    for a, r in zip(res_a, ref_a):
        assert torch.equal(a, r)
    for b_, r in zip(res_b, ref_b):
        assert torch.equal(b_, r)
