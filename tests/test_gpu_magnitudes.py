"""Operand magnitudes far from 1 on the bf16 matrix-core route, against the oracle.

The route rounds its chunk states, features and operands to bf16 and
accumulates in fp32. These cases put the states, the query rows and the
coefficients far from order one (large and small states, large and small q, the
coefficients' factor scaled up and down) and check every output and gradient at
the bf16 bar (rel-L2 2e-2): nothing may overflow, underflow or lose its relative
precision on the way. Scaled inputs are rounded to bf16 before both sides see
them, so the oracle and the kernels read identical values.
"""

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu

BAR = 2e-2

CASES = {
    # name: (q multiplier, k multiplier, v multiplier, factor multiplier). q and
    # k move inversely, so that the group sums s_g stay of order one: with
    # kappa close to its constant c0 the constant's gradient is the small
    # difference of two near-equal sums and no bf16 route can resolve it.
    "large_state": (1.0 / 32, 32.0, 1000.0, 1.0),
    "small_state": (64.0, 1.0 / 64, 1.0 / 4096, 1.0),
    "large_q": (300.0, 1.0 / 300, 1.0, 1.0),
    "small_q": (1e-4, 1e4, 1.0, 1.0),
    "large_coefficients": (1.0, 1.0, 1.0, 8.0),
    "small_coefficients": (1.0, 1.0, 1.0, 1.0 / 8),
}


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("case", sorted(CASES))
def test_scaled_operands_match_oracle(case):
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    mq, mk, mv, mf = CASES[case]
    dev = _dev()
    gen = torch.Generator().manual_seed(31)
    b, hq, hkv, n, g = 1, 14, 2, 512, 8
    q = (torch.randn((b, hq, n, 64), generator=gen) * 0.5 * mq).to(torch.bfloat16)
    k = (torch.randn((b, hkv, n, 64), generator=gen) * 0.5 * mk).to(torch.bfloat16)
    v = (torch.randn((b, hkv, n, 64), generator=gen) * mv).to(torch.bfloat16)
    labels = torch.randint(0, g, (hq, 64), generator=gen, dtype=torch.int32)
    labels[:, :g] = torch.arange(g, dtype=torch.int32)
    # a PSD factor (every denominator positive, as the reference's public entry
    # points guarantee)
    factor = torch.randn((hq, (g + 1) * (g + 2) // 2), generator=gen, dtype=torch.float64) * 0.4 * mf
    c0, lam, gam = go.expand_factor(factor, query_heads=hq, kernel_eps=0.05 * mf * mf)
    qd, kd, vd = (t.double() for t in (q, k, v))
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=0.125, head_dim=64)
    out_r, num_r, den_r = go.chunked_forward(qd, kd, vd, wq, chunk=64)
    assert float(den_r.min()) > 0.0
    dout = torch.randn((b, hq, n, 64), generator=gen)
    dq_r, dk_r, dv_r, dwq_r = go.chunked_backward(qd, kd, vd, wq, num_r, den_r, dout.double(), None, None)
    dc0_r, dlam_r, dgam_r = go.coefficient_gradients_from_wq(dwq_r, labels, g, scale=0.125, head_dim=64)
    dgam_r = go.symmetrize_gamma_gradient(dgam_r)

    ts = [t.to(dev).requires_grad_() for t in (q, k, v)]
    cs = [t.float().to(dev).requires_grad_() for t in (c0, lam, gam)]
    out, num, den = grouped_oal(*ts, labels.to(dev), *cs, scale=0.125, floor=0.0, precision="bf16")
    (out.float() * dout.to(dev)).sum().backward()
    torch.cuda.synchronize()
    errs = {name: rel(got, want) for name, got, want in (
        ("out", out, out_r), ("num", num, num_r), ("den", den, den_r), ("dq", ts[0].grad, dq_r),
        ("dk", ts[1].grad, dk_r), ("dv", ts[2].grad, dv_r), ("dc0", cs[0].grad, dc0_r),
        ("dlam", cs[1].grad, dlam_r), ("dgam", cs[2].grad, dgam_r))}
    print(f"{case}: " + " ".join(f"{k_}={e:.2e}" for k_, e in errs.items()), flush=True)
    assert all(e <= BAR for e in errs.values()), errs
    for t in (out, num, den, ts[0].grad, ts[1].grad, ts[2].grad):
        assert bool(torch.isfinite(t).all())
