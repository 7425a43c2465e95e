"""The registered operators (oal_amd/ops.py) on the GPU: torch.library.opcheck
(schema, autograd registration, fake kernel against the real one, AOT dispatch
with static shapes), results identical to the autograd Function path, and a
forward plus backward traced into a graph of the two operators."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from oal_amd import ops
from oal_amd.hd_block_gemm_autograd import grouped_oal
from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _inputs(dev, dtype, n=200, dv=64):
    gen = torch.Generator().manual_seed(17)
    b, hq, hkv, g = 1, 14, 2, 8
    q = (torch.randn(b, hq, n, 64, generator=gen) * 0.5).to(dtype)
    k = (torch.randn(b, hkv, n, 64, generator=gen) * 0.5).to(dtype)
    v = torch.randn(b, hkv, n, dv, generator=gen).to(dtype)
    labels = torch.randint(0, g, (hq, 64), generator=gen, dtype=torch.int32)
    labels[:, :g] = torch.arange(g, dtype=torch.int32)
    factor = torch.randn(hq, (g + 1) * (g + 2) // 2, generator=gen, dtype=torch.float64) * 0.4
    c0, lam, gam = (t.float() for t in go.expand_factor(factor, query_heads=hq, kernel_eps=0.05))
    return [t.to(dev) for t in (q, k, v, labels, c0, lam, gam)]


@pytest.mark.parametrize("dtype,precision", [(torch.bfloat16, "bf16"), (torch.float32, "fp32")])
def test_opcheck_forward(dtype, precision):
    dev = _dev()
    q, k, v, labels, c0, lam, gam = _inputs(dev, dtype)
    for t in (q, k, v, c0, lam, gam):
        t.requires_grad_()
    torch.library.opcheck(
        torch.ops.oal_amd.forward.default, (q, k, v, labels, c0, lam, gam, 0.125, 0.0, precision),
        test_utils=("test_schema", "test_autograd_registration", "test_faketensor", "test_aot_dispatch_static"))


def test_opcheck_backward():
    dev = _dev()
    q, k, v, labels, c0, lam, gam = _inputs(dev, torch.bfloat16)
    out, num, den, saved = torch.ops.oal_amd.forward(q, k, v, labels, c0, lam, gam, 0.125, 0.0, "bf16")
    dout = torch.randn_like(out)
    torch.library.opcheck(
        torch.ops.oal_amd.backward.default,
        (q, k, v, labels, c0, lam, gam, num, den, saved, dout, None, None, 0.125, 0.0, True, True, True, True,
         "bf16"),
        test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("dtype,precision", [(torch.bfloat16, "bf16"), (torch.float32, "fp32")])
def test_operator_path_equals_the_function_path(dtype, precision):
    dev = _dev()
    base = _inputs(dev, dtype, dv=48)
    results = []
    for fn in (grouped_oal, ops.grouped_oal_op):
        q, k, v, labels, c0, lam, gam = (t.clone() for t in base)
        for t in (q, k, v, c0, lam, gam):
            t.requires_grad_()
        out, num, den = fn(q, k, v, labels, c0, lam, gam, scale=0.125, floor=0.0, precision=precision)
        gen = torch.Generator().manual_seed(3)
        dout = torch.randn(out.shape, generator=gen).to(dev, out.dtype)
        dden = torch.randn(den.shape, generator=gen).to(dev)
        ((out * dout).sum() + (den * dden).sum()).backward()
        torch.cuda.synchronize()
        results.append([out, num, den, q.grad, k.grad, v.grad, c0.grad, lam.grad, gam.grad])
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_make_fx_traces_forward_and_backward():
    dev = _dev()

    def step(q, k, v, labels, c0, lam, gam, dout):
        out, _, _ = ops.grouped_oal_op(q, k, v, labels, c0, lam, gam, scale=0.125, floor=0.0, precision="bf16")
        return torch.autograd.grad(out, (q, k, v, lam), dout)

    with FakeTensorMode():
        bf = dict(device=dev, dtype=torch.bfloat16)
        q, k, v = torch.empty(1, 14, 200, 64, **bf), torch.empty(1, 2, 200, 64, **bf), torch.empty(1, 2, 200, 48, **bf)
        labels = torch.zeros(14, 64, device=dev, dtype=torch.int32)
        c0, lam, gam = (torch.empty(*s_, device=dev) for s_ in ((14,), (14, 8), (14, 8, 8)))
        for t in (q, k, v, lam):
            t.requires_grad_()
        dout = torch.empty(1, 14, 200, 48, **bf)
        gm = make_fx(step, tracing_mode="fake")(q, k, v, labels, c0, lam, gam, dout)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert "oal_amd.forward.default" in targets
    assert "oal_amd.backward.default" in targets
