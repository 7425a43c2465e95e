"""GPU parity at the full benchmark shapes (configurations 1, 2 and 3), bf16 matrix-core path.

The fp32 chunked oracle (oracle/grouped_oracle.py) runs these shapes in seconds on
the host cores, so the comparison is made on every output and gradient, not on
a sample:

* config 1: B=1, Hq=14, Hkv=2, N=4096, d=64, forward;
* config 2: B=4, same heads, N=4096, forward + backward through the grouped
  autograd Function with dO ~ N(0,1) in bf16 (dq, dk, dv, dc0, dlam, dGam);
* config 3: B=1, N=32768, forward + backward (long-context state carry).

Tolerance (the bf16-mode bar): rel-L2 <= 2e-2 against the fp32
oracle evaluated on the same bf16-rounded q, k, v.

The config coefficients (c0 = 1, lam ~ U(0.5, 1.5), Gam_gh ~ U(0, 0.5) for g <= h,
mirrored) are not PSD: every head's Gam has a negative eigenvalue, and the oracle
finds 1, 19 and 7 tokens with den <= 0 at configs 1, 2 and 3 (min den -2.08,
-3.50, -0.94). The reference's HD runtime raises on such an output
(hd_block_gemm_runtime.py:392-408); its public entry points take a PSD factor
and cannot receive these coefficients at all. The tests time and compare the
operator on them anyway, with two masks whose excluded-token counts are printed
and bounded by 0.1%: `out` is compared where the oracle's |den| > 1 (4, 36 and
16 tokens excluded; elsewhere out = num / den is ill-conditioned), and the
upstream dO is kept on tokens whose denominator is not a near-cancelling sum
(26 and 107 tokens excluded at configs 1 and 2, 41 at config 3).
"""

import os
import time

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))
    return torch.device("cuda:0")


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _assert_few_excluded(keep, what, bound=1e-3):
    dropped = int((~keep).sum())
    print(f"{what}: {dropped} of {keep.numel()} tokens excluded", flush=True)
    assert dropped <= bound * keep.numel(), (what, dropped, keep.numel())
    return dropped


def _well_conditioned(q32, k32, v32, wq, den_r, max_cond=20.0):
    _, _, den_abs = go.chunked_forward(q32.abs(), k32.abs(), v32, wq.abs(), chunk=64)
    keep = (den_r.abs() > 1.0) & (den_abs <= max_cond * den_r.abs())
    _assert_few_excluded(keep, "dO conditioning")
    return keep


def _inputs(config, dev):
    inp = go.config_inputs(config)
    q32, k32, v32 = (inp[n].to(torch.bfloat16).float() for n in ("q", "k", "v"))
    wq = go.feature_coefficients(inp["groups"], inp["c0"], inp["lam"], inp["gam"], scale=inp["scale"], head_dim=64)
    return inp, q32, k32, v32, wq


def _forward_errors(out, num, den, out_r, num_r, den_r):
    nonpos = int((den_r <= 0).sum())
    print(f"oracle den <= 0 on {nonpos} tokens (the reference would raise on this input)", flush=True)
    ok = den_r.abs() > 1.0
    _assert_few_excluded(ok, "out comparison")
    ok = ok.expand_as(out_r)
    return {"num": rel(num, num_r), "den": rel(den, den_r), "out": rel(out.float().cpu()[ok], out_r[ok])}


def test_config1_forward_full_shape():
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    dev = _dev()
    inp, q32, k32, v32, wq = _inputs(1, dev)
    args = [t.to(torch.bfloat16).to(dev) for t in (q32, k32, v32)]
    args += [inp[n].to(dev) for n in ("groups", "c0", "lam", "gam")]
    out, num, den = grouped_oal(*args, scale=inp["scale"], floor=0.0, precision="bf16")
    torch.cuda.synchronize()
    out_r, num_r, den_r = go.chunked_forward(q32, k32, v32, wq, chunk=64)
    errs = _forward_errors(out, num, den, out_r, num_r, den_r)
    print("config 1 forward rel-L2:", {k: f"{e:.2e}" for k, e in errs.items()}, flush=True)
    assert all(e <= BF16_TOL for e in errs.values()), errs


def _fwd_bwd_case(config):
    from oal_amd.hd_block_gemm_autograd import _GroupedOALFunction

    dev = _dev()
    inp, q32, k32, v32, wq = _inputs(config, dev)
    qb, kb, vb = (t.to(torch.bfloat16).to(dev).requires_grad_() for t in (q32, k32, v32))
    c0, lam, gam = (inp[n].to(dev).requires_grad_() for n in ("c0", "lam", "gam"))
    labels = inp["groups"].to(dev)
    t0 = time.perf_counter()
    out, num, den = _GroupedOALFunction.apply(qb, kb, vb, c0, lam, gam, labels, inp["scale"], 0.0, "bf16")
    torch.cuda.synchronize()
    out_r, num_r, den_r = go.chunked_forward(q32, k32, v32, wq, chunk=64)
    fwd = _forward_errors(out, num, den, out_r, num_r, den_r)
    gen = torch.Generator().manual_seed(11)
    mask = _well_conditioned(q32, k32, v32, wq, den_r).float()
    dout = torch.randn(out.shape, generator=gen).to(torch.bfloat16).float() * mask
    out.backward(dout.to(torch.bfloat16).to(dev))
    torch.cuda.synchronize()
    dq_r, dk_r, dv_r, dwq_r = go.chunked_backward(q32, k32, v32, wq, num_r, den_r, dout, None, None)
    dc0_r, dlam_r, dgam_r = go.coefficient_gradients_from_wq(dwq_r, inp["groups"], 8, scale=inp["scale"],
                                                             head_dim=64)
    dgam_r = go.symmetrize_gamma_gradient(dgam_r)
    errs = dict(fwd)
    for name, got, want in (("dq", qb.grad, dq_r), ("dk", kb.grad, dk_r), ("dv", vb.grad, dv_r),
                            ("dc0", c0.grad, dc0_r), ("dlam", lam.grad, dlam_r), ("dgam", gam.grad, dgam_r)):
        errs[name] = rel(got, want)
    print(f"config {config} fwd+bwd rel-L2 (kept dO on {mask.mean().item():.3f} of tokens, "
          f"{time.perf_counter() - t0:.1f}s):", {k: f"{e:.2e}" for k, e in errs.items()}, flush=True)
    assert all(e <= BF16_TOL for e in errs.values()), errs


def test_config2_forward_backward_full_shape():
    _fwd_bwd_case(2)


def test_config3_long_context_forward_backward():
    _fwd_bwd_case(3)
