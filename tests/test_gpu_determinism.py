"""Run-to-run determinism: two identical fwd+bwd calls give bitwise-identical
outputs and gradients, on the fp32 route (oal_attention's "triton"/"auto" and
"reference" executions) and on the bf16 matrix-core route, for 8 groups (the
group-sum intra-chunk kernels), 12 groups and 64 groups (per-pair
coefficients; the fp32 route's scalar kernels, the bf16 route's feature-form
local kernels and their per-head dk partials). Every reduction in the library
has a fixed order (partial buffers summed in order, no atomics; the fp32
scalar kernels' four lanes of a token add to its gradient row in turn)."""

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _inputs(gcount, n, seed):
    """8 groups: the configuration-1 inputs. 12 groups: random labels and a
    factor. 64 groups: one group per dimension (labels d -> d), the per-pair
    layout of the reference-contract HD Function."""
    if gcount == 8:
        inp = go.config_inputs(1, batch=1, seq_len=n, seed=seed)
        return {x: inp[x] for x in ("q", "k", "v", "groups", "c0", "lam", "gam", "scale")}
    gen = torch.Generator().manual_seed(seed)
    hq, hkv = 14, 2
    q = torch.randn((1, hq, n, 64), generator=gen) * 0.6
    k = torch.randn((1, hkv, n, 64), generator=gen) * 0.6
    v = torch.randn((1, hkv, n, 64), generator=gen)
    if gcount == 64:
        labels = torch.arange(64, dtype=torch.int32).unsqueeze(0).expand(hq, -1).contiguous()
        scale_f = 0.05
    else:
        labels = torch.randint(0, gcount, (hq, 64), generator=gen, dtype=torch.int32)
        labels[:, :gcount] = torch.arange(gcount, dtype=torch.int32)
        scale_f = 0.3
    side = gcount + 1
    factor = torch.randn((hq, side * (side + 1) // 2), generator=gen, dtype=torch.float64) * scale_f
    c0, lam, gam = go.expand_factor(factor, query_heads=hq, kernel_eps=0.05)
    return {"q": q, "k": k, "v": v, "groups": labels, "c0": c0.float(), "lam": lam.float(), "gam": gam.float(),
            "scale": 0.125}


@pytest.mark.parametrize("precision,dtype,n,gcount", [
    ("fp32", torch.float32, 777, 8), ("fp32", torch.bfloat16, 320, 8), ("bf16", torch.bfloat16, 1000, 8),
    ("fp32", torch.float32, 450, 12), ("bf16", torch.bfloat16, 450, 12),
    ("fp32", torch.float32, 300, 64), ("bf16", torch.bfloat16, 520, 64),
])
def test_two_runs_are_bitwise_identical(precision, dtype, n, gcount):
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    dev = _dev()
    inp = _inputs(gcount, n, seed=17)
    print(f"determinism: precision={precision} dtype={dtype} N={n} groups={gcount}", flush=True)

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
        assert torch.isfinite(a.float()).all(), (precision, gcount, name)
        assert torch.equal(a, b), (precision, gcount, name)
