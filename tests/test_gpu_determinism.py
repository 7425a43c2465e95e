"""Run-to-run determinism: two identical fwd+bwd calls give bitwise-identical
outputs and gradients, on the fp32 route (oal_attention's "triton"/"auto" and
"reference" executions) and on the bf16 matrix-core route. Every reduction in
the library has a fixed order (partial buffers summed in order, no atomics;
the fp32 kernels' four lanes of a token add to its gradient row in turn)."""

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.parametrize("precision,dtype,n", [("fp32", torch.float32, 777), ("fp32", torch.bfloat16, 320),
                                               ("bf16", torch.bfloat16, 1000)])
def test_two_runs_are_bitwise_identical(precision, dtype, n):
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    dev = _dev()
    inp = go.config_inputs(1, batch=1, seq_len=n, seed=17)

    def run():
        q, k, v = (inp[x].to(dtype).to(dev).requires_grad_() for x in ("q", "k", "v"))
        c0, lam, gam = (inp[x].to(dev).requires_grad_() for x in ("c0", "lam", "gam"))
        out, num, den = grouped_oal(q, k, v, inp["groups"].to(dev), c0, lam, gam, scale=inp["scale"], floor=0.0,
                                    precision=precision)
        g = torch.randn(num.shape, generator=torch.Generator().manual_seed(2)).to(dev)
        (num * g).sum().backward()
        torch.cuda.synchronize()
        return [out, num, den] + [t.grad for t in (q, k, v, c0, lam, gam)]

    first, second = run(), run()
    for name, a, b in zip(("out", "num", "den", "dq", "dk", "dv", "dc0", "dlam", "dgam"), first, second):
        assert torch.equal(a, b), (precision, name)
