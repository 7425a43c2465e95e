"""Pins the CPU oracle (oracle/grouped_oracle.py) before it is trusted.

Each check is chosen so that a plausible mistake fails it: the reference's
own golden fixtures; three independent formulations agreeing (token-pair
group-sum form, token-cumulative state form, chunked feature form);
autograd gradcheck; closed-form backward vs autograd; known-answer factor
expansion; and invariants the mathematics fixes.
"""

import json
import math
import os

import pytest
import torch

from oracle import grouped_oracle as go

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _fixture(name):
    with open(os.path.join(GOLDEN, name)) as fh:
        return json.load(fh)


def _fixture_case(fx):
    q = torch.tensor(fx["q"], dtype=torch.float64)
    k = torch.tensor(fx["k"], dtype=torch.float64)
    v = torch.tensor(fx["v"], dtype=torch.float64)
    hq, d = fx["query_heads"], fx["head_dimension"]
    labels = torch.zeros((hq, d), dtype=torch.int32)
    for h, groups in enumerate(fx["groups"]):
        for gid, dims in enumerate(groups):
            for dim in dims:
                labels[h, dim] = gid
    factor = torch.tensor(fx["packed_lower_triangular"], dtype=torch.float64)
    return q, k, v, labels, factor


@pytest.mark.parametrize("name", ["two_groups.json", "different_active_group_counts.json"])
def test_oracle_matches_reference_golden_fixtures(name):
    fx = _fixture(name)
    q, k, v, labels, factor = _fixture_case(fx)
    eps, scale = fx["kernel_eps"], fx["scale"]
    num_e = torch.tensor(fx["numerator"], dtype=torch.float64)
    den_e = torch.tensor(fx["denominator"], dtype=torch.float64)
    out_e = torch.tensor(fx["output"], dtype=torch.float64)
    c0, lam, gam = go.expand_factor(factor, query_heads=q.shape[1], kernel_eps=eps)
    num, den = go.materialized_forward(q, k, v, labels, c0, lam, gam, scale=scale)
    torch.testing.assert_close(num, num_e, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(den, den_e, atol=1e-12, rtol=1e-12)
    out, num2, den2 = go.dense_forward(q, k, v, labels, factor, scale=scale, kernel_eps=eps)
    torch.testing.assert_close(out, out_e, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(num2, num_e, atol=1e-12, rtol=1e-12)
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=scale, head_dim=q.shape[-1])
    out3, num3, den3 = go.chunked_forward(q, k, v, wq, chunk=1)
    torch.testing.assert_close(out3, out_e, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(den3, den_e, atol=1e-12, rtol=1e-12)


def _random_case(b=2, hq=4, hkv=2, n=13, d=6, dv=5, gmax=3, seed=7):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((b, hq, n, d), generator=gen, dtype=torch.float64)
    k = torch.randn((b, hkv, n, d), generator=gen, dtype=torch.float64)
    v = torch.randn((b, hkv, n, dv), generator=gen, dtype=torch.float64)
    labels = torch.randint(0, gmax, (hq, d), generator=gen, dtype=torch.int32)
    for h in range(hq):  # continuous prefix of ids, as the public contract requires
        labels[h, :gmax] = torch.arange(gmax, dtype=torch.int32)
    side = gmax + 1
    factor = torch.randn((hq, side * (side + 1) // 2), generator=gen, dtype=torch.float64) * 0.5
    return q, k, v, labels, factor


def test_three_formulations_agree_with_gqa_and_ragged_chunks():
    q, k, v, labels, factor = _random_case()
    scale, eps = 0.37, 0.07
    c0, lam, gam = go.expand_factor(factor, query_heads=4, kernel_eps=eps)
    out_d, num_d, den_d = go.dense_forward(q, k, v, labels, factor, scale=scale, kernel_eps=eps)
    num_m, den_m = go.materialized_forward(q, k, v, labels, c0, lam, gam, scale=scale)
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=scale, head_dim=q.shape[-1])
    for chunk in (1, 4, 5, 13, 64):
        out_c, num_c, den_c = go.chunked_forward(q, k, v, wq, chunk=chunk)
        torch.testing.assert_close(num_c, num_d, atol=1e-11, rtol=1e-10)
        torch.testing.assert_close(den_c, den_d, atol=1e-11, rtol=1e-10)
        torch.testing.assert_close(out_c, out_d, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(num_m, num_d, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(den_m, den_d, atol=1e-11, rtol=1e-10)


def test_nonsymmetric_gamma_pair_form_matches_materialized():
    # The reference routes pair (r, c), r >= c, through Gam[g(r), g(c)] only.
    q, k, v, labels, _ = _random_case(seed=3)
    gen = torch.Generator().manual_seed(11)
    c0 = torch.rand(4, generator=gen, dtype=torch.float64) + 1
    lam = torch.rand((4, 3), generator=gen, dtype=torch.float64)
    gam = torch.rand((4, 3, 3), generator=gen, dtype=torch.float64)
    num_m, den_m = go.materialized_forward(q, k, v, labels, c0, lam, gam, scale=0.3)
    num_p, den_p = go.dense_forward_coefficients(q, k, v, labels, c0, lam, gam, scale=0.3)
    torch.testing.assert_close(num_m, num_p, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(den_m, den_p, atol=1e-11, rtol=1e-10)
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=0.3, head_dim=q.shape[-1])
    _, num_c, den_c = go.chunked_forward(q, k, v, wq, chunk=4)
    torch.testing.assert_close(num_c, num_p, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(den_c, den_p, atol=1e-11, rtol=1e-10)


def test_materialized_forward_passes_gradcheck():
    q, k, v, labels, factor = _random_case(b=1, hq=2, hkv=1, n=3, d=3, dv=2, gmax=2)
    fac = factor.clone().requires_grad_()
    qkv = [t.clone().requires_grad_() for t in (q, k, v)]

    def fn(qq, kk, vv, ff):
        c0, lam, gam = go.expand_factor(ff, query_heads=2, kernel_eps=0.1)
        num, den = go.materialized_forward(qq, kk, vv, labels, c0, lam, gam, scale=0.4)
        return num / den

    assert torch.autograd.gradcheck(fn, (*qkv, fac), atol=1e-6, rtol=1e-4)


@pytest.mark.parametrize("use_dnum", [False, True])
def test_closed_form_chunked_backward_matches_autograd(use_dnum):
    q, k, v, labels, _ = _random_case(seed=5)
    gen = torch.Generator().manual_seed(2)
    c0 = (torch.rand(4, generator=gen, dtype=torch.float64) + 2).requires_grad_()
    lam = torch.rand((4, 3), generator=gen, dtype=torch.float64).requires_grad_()
    g0 = torch.rand((4, 3, 3), generator=gen, dtype=torch.float64)
    gam = (0.5 * (g0 + g0.transpose(-1, -2))).requires_grad_()
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
    scale = 0.3
    num, den = go.dense_forward_coefficients(qa, ka, va, labels, c0, lam, gam, scale=scale)
    out = num / den
    dout = torch.randn(out.shape, generator=gen, dtype=torch.float64)
    dnum = torch.randn(num.shape, generator=gen, dtype=torch.float64) if use_dnum else None
    dden = torch.randn(den.shape, generator=gen, dtype=torch.float64) if use_dnum else None
    loss = (out * dout).sum()
    if use_dnum:
        loss = loss + (num * dnum).sum() + (den * dden).sum()
    loss.backward()
    wq = go.feature_coefficients(labels, c0.detach(), lam.detach(), gam.detach(), scale=scale, head_dim=6)
    _, num_c, den_c = go.chunked_forward(q, k, v, wq, chunk=4)
    dq, dk, dv, dwq = go.chunked_backward(q, k, v, wq, num_c, den_c, dout, dnum, dden, chunk=4)
    torch.testing.assert_close(dq, qa.grad, atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(dk, ka.grad, atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(dv, va.grad, atol=1e-10, rtol=1e-9)
    dc0, dlam, dgam = go.coefficient_gradients_from_wq(dwq, labels, 3, scale=scale, head_dim=6)
    torch.testing.assert_close(dc0, c0.grad, atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(dlam, lam.grad, atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(dgam, gam.grad, atol=1e-10, rtol=1e-9)


def _floor_between(den: torch.Tensor, quantile: float) -> float:
    """A floor between two sorted denominators near the given quantile, at the
    middle of the widest gap there, so that no denominator sits on it."""
    vals = den.detach().flatten().sort().values
    lo = int(quantile * (vals.numel() - 1))
    window = range(max(lo - 8, 0), min(lo + 8, vals.numel() - 1))
    best = max(window, key=lambda i: float(vals[i + 1] - vals[i]))
    return float(0.5 * (vals[best] + vals[best + 1]))


def test_floor_branch_matches_autograd_of_clamped_denominator():
    # reference hd_block_gemm_normalization_ops.py:13-71: out = num / max(den, eps), and the
    # VJP masks the dout part of the denominator gradient where den < eps (the gradient of
    # clamp_min), while dden is added unmasked
    q, k, v, labels, _ = _random_case(seed=11)
    gen = torch.Generator().manual_seed(4)
    c0 = torch.rand(4, generator=gen, dtype=torch.float64) + 2
    lam = torch.rand((4, 3), generator=gen, dtype=torch.float64)
    g0 = torch.rand((4, 3, 3), generator=gen, dtype=torch.float64)
    gam = 0.5 * (g0 + g0.transpose(-1, -2))
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
    c0a, lama, gama = (t.clone().requires_grad_() for t in (c0, lam, gam))
    scale = 0.3
    num, den = go.dense_forward_coefficients(qa, ka, va, labels, c0a, lama, gama, scale=scale)
    floor = _floor_between(den, 0.4)
    below = int((den < floor).sum())
    assert 0.2 * den.numel() < below < 0.6 * den.numel()
    out = num / den.clamp_min(floor)
    dout = torch.randn(out.shape, generator=gen, dtype=torch.float64)
    dnum = torch.randn(num.shape, generator=gen, dtype=torch.float64)
    dden = torch.randn(den.shape, generator=gen, dtype=torch.float64)
    ((out * dout).sum() + (num * dnum).sum() + (den * dden).sum()).backward()
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=scale, head_dim=6)
    out_c, num_c, den_c = go.chunked_forward(q, k, v, wq, chunk=4, floor=floor)
    torch.testing.assert_close(out_c, out.detach(), atol=1e-12, rtol=1e-11)
    dq, dk, dv, dwq = go.chunked_backward(q, k, v, wq, num_c, den_c, dout, dnum, dden, chunk=4, floor=floor)
    torch.testing.assert_close(dq, qa.grad, atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(dk, ka.grad, atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(dv, va.grad, atol=1e-10, rtol=1e-9)
    dc0, dlam, dgam = go.coefficient_gradients_from_wq(dwq, labels, 3, scale=scale, head_dim=6)
    torch.testing.assert_close(dc0, c0a.grad, atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(dlam, lama.grad, atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(dgam, gama.grad, atol=1e-10, rtol=1e-9)
    # the mask matters: without it (the floor's gradient passed through) dq differs
    dq0, _, _, _ = go.chunked_backward(q, k, v, wq, num_c, den_c.clamp_min(floor), dout, dnum, dden, chunk=4,
                                       floor=0.0)
    assert (dq0 - qa.grad).abs().max() > 1e-3


def test_factor_expansion_known_answer():
    # tests/operators/test_grouped_quadratic.py:476-488
    factor = torch.tensor((1.1, 0.5, 0.9, 0.4, 0.8, 0.7), dtype=torch.float64)
    c0, lam, gam = go.expand_factor(factor, query_heads=1, kernel_eps=0.07)
    lower = torch.tensor(((1.1, 0.0, 0.0), (0.5, 0.9, 0.0), (0.4, 0.8, 0.7)), dtype=torch.float64)
    m = lower @ lower.T
    torch.testing.assert_close(c0, m[0, 0].view(1) + 0.07)
    torch.testing.assert_close(lam, 2 * m[0, 1:].view(1, 2))
    torch.testing.assert_close(gam, m[1:, 1:].view(1, 2, 2))


def test_invariants_token0_zero_query_and_gqa_repeat():
    q, k, v, labels, factor = _random_case(seed=9)
    c0, lam, gam = go.expand_factor(factor, query_heads=4, kernel_eps=0.05)
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=0.3, head_dim=6)
    out, num, den = go.chunked_forward(q, k, v, wq, chunk=4)
    # token 0 attends only to itself
    torch.testing.assert_close(out[:, :, 0], v.repeat_interleave(2, dim=1)[:, :, 0])
    # q = 0 -> kappa == c0 -> causal running mean of v
    out0, _, _ = go.chunked_forward(torch.zeros_like(q), k, v, wq, chunk=4)
    counts = torch.arange(1, q.shape[2] + 1, dtype=torch.float64)[None, None, :, None]
    mean = v.cumsum(2) / counts
    torch.testing.assert_close(out0, mean.repeat_interleave(2, dim=1), atol=1e-12, rtol=1e-12)
    # native GQA equals K/V repeated per query head
    outr, _, _ = go.chunked_forward(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), wq, chunk=4)
    torch.testing.assert_close(out, outr, atol=1e-12, rtol=1e-12)


def test_config_generators_shapes_and_group_sizes():
    inp = go.config_inputs(1, seq_len=32)
    assert inp["q"].shape == (1, 14, 32, 64) and inp["k"].shape == (1, 2, 32, 64)
    counts = torch.bincount(inp["groups"][0].long(), minlength=8)
    assert sorted(counts.tolist()) == sorted(go.UNEVEN_GROUP_SIZES)
    assert torch.allclose(inp["gam"], inp["gam"].transpose(-1, -2))
    inp0 = go.config_inputs(0)
    assert inp0["q"].shape == (1, 1, 256, 64)
    assert abs(inp0["q"].std().item() - 1 / math.sqrt(8)) < 0.02
