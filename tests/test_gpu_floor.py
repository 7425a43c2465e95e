"""The normalization floor on the GPU, both routes, against the oracle.

out = num / max(den, floor), and the VJP masks the output-gradient part of the
denominator gradient where den < floor (reference
hd_block_gemm_normalization_ops.py:13-71; the oracle's floor branch is pinned
against autograd of the clamped denominator in tests/test_oracle.py). Here the
floor sits near the 30th percentile of the oracle's denominators, so about a
third of the tokens take each branch. The upstream output gradient is zeroed on
the few tokens whose denominator lies within 2% of the floor: there the mask is
a step in den, and the bf16 route's rounding may put a token on the other side.
"""

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-5, "bf16": 2e-2}


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_floor_forward_and_backward_match_oracle(precision):
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    dev = _dev()
    gen = torch.Generator().manual_seed(21)
    b, hq, hkv, n, g = 1, 14, 2, 512, 8
    q = torch.randn((b, hq, n, 64), generator=gen) * 0.5
    k = torch.randn((b, hkv, n, 64), generator=gen) * 0.5
    v = torch.randn((b, hkv, n, 64), generator=gen)
    labels = torch.randint(0, g, (hq, 64), generator=gen, dtype=torch.int32)
    labels[:, :g] = torch.arange(g, dtype=torch.int32)
    factor = torch.randn((hq, (g + 1) * (g + 2) // 2), generator=gen, dtype=torch.float64) * 0.4
    c0, lam, gam = go.expand_factor(factor, query_heads=hq, kernel_eps=0.05)
    if precision == "bf16":
        q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    qd, kd, vd = (t.double() for t in (q, k, v))
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=0.125, head_dim=64)
    _, num0, den0 = go.chunked_forward(qd, kd, vd, wq, chunk=64)
    floor = float(den0.flatten().sort().values[int(0.3 * den0.numel())]) * 1.0001
    below = float((den0 < floor).double().mean())
    print(f"floor {floor:.4g}: {below:.1%} of the tokens below it", flush=True)
    assert 0.2 < below < 0.4
    near = ((den0 / floor - 1.0).abs() < 0.02)
    print(f"{int(near.sum())} tokens within 2% of the floor (output gradient zeroed there)", flush=True)
    dout = torch.randn((b, hq, n, 64), generator=gen) * (~near).double().float()
    dden = torch.randn((b, hq, n, 1), generator=gen)

    ts = [t.to(dev).requires_grad_() for t in (q, k, v)]
    cs = [t.float().to(dev).requires_grad_() for t in (c0, lam, gam)]
    out, num, den = grouped_oal(*ts, labels.to(dev), *cs, scale=0.125, floor=floor, precision=precision)
    ((out.float() * dout.to(dev)).sum() + (den * dden.to(dev)).sum()).backward()
    torch.cuda.synchronize()

    out_r, num_r, den_r = go.chunked_forward(qd, kd, vd, wq, chunk=64, floor=floor)
    dq_r, dk_r, dv_r, dwq_r = go.chunked_backward(qd, kd, vd, wq, num_r, den_r, dout.double(), None,
                                                  dden.double(), floor=floor)
    dc0_r, dlam_r, dgam_r = go.coefficient_gradients_from_wq(dwq_r, labels, g, scale=0.125, head_dim=64)
    dgam_r = go.symmetrize_gamma_gradient(dgam_r)
    errs = {name: rel(got, want) for name, got, want in (
        ("out", out, out_r), ("num", num, num_r), ("den", den, den_r), ("dq", ts[0].grad, dq_r),
        ("dk", ts[1].grad, dk_r), ("dv", ts[2].grad, dv_r), ("dc0", cs[0].grad, dc0_r),
        ("dlam", cs[1].grad, dlam_r), ("dgam", cs[2].grad, dgam_r))}
    print(f"floor {precision}: " + " ".join(f"{k_}={e:.2e}" for k_, e in errs.items()), flush=True)
    assert all(e <= TOL[precision] for e in errs.values()), errs
