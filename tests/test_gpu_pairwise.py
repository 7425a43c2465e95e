"""Per-pair coefficients on the matrix cores (more than 8 groups), GPU parity.

The reference-contract HD Function takes logical per-pair coefficients
(a [Hq], b [Hq, D], c [Hq, D(D+1)/2]; hd_block_gemm_autograd.py:85-204). With a
``bf16_tensorcore`` plan it runs the bf16 matrix-core path with one group per
dimension (G = 64): the state contractions on per-slot weights as for grouped
coefficients, and the intra-chunk local score in feature form, phi_Q . phi_K^T
on the matrix cores (hd_block_gemm_runtime.py:530-540), with its feature-form
VJP. Compared with the fp32 oracle (oracle/grouped_oracle.py, per-feature
coefficients of the identity labelling) on the bf16-rounded q, k, v, fwd+bwd at
D = 64, Hq = 14, Hkv = 2, up to the configuration-2 shape (B = 4, N = 4096):
rel-L2 <= 2e-2 (the bf16-mode bar) on out, num, den, dq, dk, dv, da, db and dc.

The coefficients come from a random lower-triangular factor over [1, x]
(x = scale q o k), so kappa = ||[1, x] L||^2 + eps > 0 and every denominator is
positive (the plan's positivity check runs). A grouped case with 12 groups
takes the same feature-form path.
"""

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _logical_coefficients(hq, d, gen, eps=1e-3):
    """(a, b, c) of kappa = [1, x] M [1, x]^T + eps, M = L L^T, c without multiplicity."""
    a, b, c = [], [], []
    rows, cols = torch.tril_indices(d, d)
    for _ in range(hq):
        low = torch.tril(torch.randn(d + 1, d + 1, generator=gen, dtype=torch.float64) * 0.08)
        low.diagonal().copy_(0.4 + 0.3 * torch.rand(d + 1, generator=gen, dtype=torch.float64))
        m = low @ low.T
        a.append(m[0, 0] + eps)
        b.append(2 * m[0, 1:])
        c.append(m[1:, 1:][rows, cols])
    return torch.stack(a).float(), torch.stack(b).float(), torch.stack(c).float()


def _oracle(q32, k32, v32, a, b, c, scale, dout):
    """Oracle fwd+bwd with the identity labelling; gradients mapped to (a, b, c)."""
    hq, d = b.shape
    labels = torch.arange(d, dtype=torch.int32).unsqueeze(0).expand(hq, -1).contiguous()
    rows, cols = torch.tril_indices(d, d)
    gam = torch.zeros(hq, d, d, dtype=torch.float64)
    gam[:, rows, cols] = c.double()
    gam[:, cols, rows] = c.double()
    wq = go.feature_coefficients(labels, a.double(), b.double(), gam, scale=scale, head_dim=d)
    qd, kd, vd = (t.double() for t in (q32, k32, v32))
    out, num, den = go.chunked_forward(qd, kd, vd, wq, chunk=64)
    dq, dk, dv, dwq = go.chunked_backward(qd, kd, vd, wq, num, den, dout.double(), None, None)
    mult = torch.where(rows == cols, 1.0, 2.0).double()
    da = dwq[:, 0]
    db = dwq[:, 1:1 + d] * scale
    dc = dwq[:, 1 + d:] * mult * scale * scale
    return (out, num, den), (dq, dk, dv, da, db, dc)


@pytest.mark.parametrize("batch,n", [(1, 1024), (2, 1000), (4, 4096)])
def test_hd_function_bf16_plan_per_pair_coefficients_match_oracle(batch, n):
    from oal_amd.hd_block_gemm import build_hd_block_gemm_plan, canonical_pair_layout
    from oal_amd.hd_block_gemm_autograd import _hd_parallel_block_gemm_autograd

    dev = _dev()
    gen = torch.Generator().manual_seed(31 + n)
    hq, hkv, d = 14, 2, 64
    q = torch.randn(batch, hq, n, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(batch, hkv, n, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(batch, hkv, n, d, generator=gen).to(torch.bfloat16)
    a, b, c = _logical_coefficients(hq, d, gen)
    scale = d ** -0.5
    ts = [t.to(dev).requires_grad_() for t in (q, k, v, a, b, c)]
    plan = build_hd_block_gemm_plan(ts[0], ts[1], ts[2], precision="bf16_tensorcore",
                                    requested_gradient_mask=(True,) * 6)
    out, num, den = _hd_parallel_block_gemm_autograd(*ts, scale=scale, eps=1e-30, layout=canonical_pair_layout(d),
                                                     plan=plan)
    dout = torch.randn(out.shape, generator=gen).to(torch.bfloat16)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    (out_r, num_r, den_r), grads_r = _oracle(q.float(), k.float(), v.float(), a, b, c, scale, dout.float())
    errs = {"out": rel(out.float(), out_r), "num": rel(num, num_r), "den": rel(den, den_r)}
    for name, t, r in zip(("dq", "dk", "dv", "da", "db", "dc"), ts, grads_r):
        errs[name] = rel(t.grad, r)
    print(f"per-pair bf16 B={batch} N={n}: " + " ".join(f"{k_}={e:.2e}" for k_, e in errs.items()), flush=True)
    assert all(e <= BF16_TOL for e in errs.values()), errs


def test_grouped_function_with_12_groups_takes_the_feature_form_path():
    from oal_amd.hd_block_gemm_autograd import _GroupedOALFunction

    dev = _dev()
    gen = torch.Generator().manual_seed(5)
    bsz, hq, hkv, n, d, g = 1, 14, 2, 700, 64, 12
    q = (torch.randn(bsz, hq, n, d, generator=gen) * 0.7).to(torch.bfloat16)
    k = (torch.randn(bsz, hkv, n, d, generator=gen) * 0.7).to(torch.bfloat16)
    v = torch.randn(bsz, hkv, n, d, generator=gen).to(torch.bfloat16)
    labels = torch.randint(0, g, (hq, d), generator=gen, dtype=torch.int32)
    labels[:, :g] = torch.arange(g, dtype=torch.int32)
    side = g + 1
    factor = torch.randn(hq, side * (side + 1) // 2, generator=gen, dtype=torch.float64) * 0.3
    c0, lam, gam = go.expand_factor(factor, query_heads=hq, kernel_eps=0.05)
    c0d, lamd, gamd = (t.float().to(dev).requires_grad_() for t in (c0, lam, gam))
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    out, num, den = _GroupedOALFunction.apply(qd, kd, vd, c0d, lamd, gamd, labels.to(dev), 0.125, 0.0, "bf16")
    dnum = torch.randn(num.shape, generator=gen)
    (num * dnum.to(dev)).sum().backward()
    torch.cuda.synchronize()
    wq = go.feature_coefficients(labels, c0.double(), lam.double(), gam.double(), scale=0.125, head_dim=d)
    q32, k32, v32 = (t.double() for t in (q, k, v))
    _, num_r, den_r = go.chunked_forward(q32, k32, v32, wq, chunk=64)
    dq_r, dk_r, dv_r, dwq_r = go.chunked_backward(q32, k32, v32, wq, num_r, den_r, None, dnum.double(), None)
    dc0_r, dlam_r, dgam_r = go.coefficient_gradients_from_wq(dwq_r, labels, g, scale=0.125, head_dim=d)
    dgam_r = go.symmetrize_gamma_gradient(dgam_r)
    errs = {"num": rel(num, num_r), "den": rel(den, den_r), "dq": rel(qd.grad, dq_r), "dk": rel(kd.grad, dk_r),
            "dv": rel(vd.grad, dv_r), "dc0": rel(c0d.grad, dc0_r), "dlam": rel(lamd.grad, dlam_r),
            "dgam": rel(gamd.grad, dgam_r)}
    print("grouped G=12 bf16 (feature-form local): " + " ".join(f"{k_}={e:.2e}" for k_, e in errs.items()),
          flush=True)
    assert all(e <= BF16_TOL for e in errs.values()), errs
