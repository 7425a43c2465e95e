"""FP64 route (``oal_f64.hip``): ``oal_attention(execution="reference")`` with a
float64 working dtype, and the grouped float64 Function.

The first tests restate, on the HIP device, the reference's own float64 tests of
that execution (``tests/operators/test_grouped_quadratic.py:136-330``): the dense
oracle match at atol 1e-11 / rtol 1e-10, partition independence, the cross-group
coefficient, group/factor broadcasting, the factor and q/k/v gradients at atol
1e-10 / rtol 1e-9, gradcheck, and the padded factor entries. The oracle is
``oracle/grouped_oracle.py`` (``dense_forward``, pinned to the reference's golden
fixtures), run on the CPU in float64. The later tests take multi-tile, ragged,
GQA shapes with 64 features, 8 and 64 groups, every upstream gradient and the
coefficient gradients (dGam in the symmetric convention).
"""

from __future__ import annotations

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def _case(*, batch=2, query_heads=4, key_heads=2, sequence=3, dimension=4, value_dimension=3):
    gen = torch.Generator().manual_seed(20260802)
    return (
        torch.randn(batch, query_heads, sequence, dimension, generator=gen, dtype=torch.float64),
        torch.randn(batch, key_heads, sequence, dimension, generator=gen, dtype=torch.float64),
        torch.randn(batch, key_heads, sequence, value_dimension, generator=gen, dtype=torch.float64),
    )


def _two_group_mapping(query_heads=4, dimension=4):
    mapping = torch.ones((query_heads, dimension), dtype=torch.int32)
    mapping[:, :2] = 0
    return mapping


FIXED_TWO_GROUP = (1.0, 0.5, 0.5, 0.5, 0.5, 0.0)
CROSS_GROUP = (1.1, 0.5, 0.9, 0.4, 0.8, 0.7)


def _oal(q, k, v, groups, factor, **kw):
    from oal_amd import oal_attention

    dev = _dev()
    return oal_attention(q.to(dev), k.to(dev), v.to(dev), groups.to(dev), factor.to(dev), execution="reference", **kw)


def test_matches_dense_oracle_in_float64():
    q, k, v = _case()
    groups = _two_group_mapping()
    factor = torch.tensor(CROSS_GROUP, dtype=torch.float64)
    out, num, den = _oal(q, k, v, groups, factor, scale=0.37, kernel_eps=0.07, return_unnormalized=True)
    assert out.dtype == num.dtype == den.dtype == torch.float64
    out_r, num_r, den_r = go.dense_forward(q, k, v, groups, factor, scale=0.37, kernel_eps=0.07)
    torch.testing.assert_close(out.cpu(), out_r, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(num.cpu(), num_r, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(den.cpu(), den_r, atol=1e-11, rtol=1e-10)
    assert bool((den > 0).all())


def test_output_does_not_depend_on_a_legal_group_partition():
    q, k, v = _case(query_heads=1, key_heads=1)
    factor = torch.tensor(FIXED_TWO_GROUP, dtype=torch.float64)
    out_a = _oal(q, k, v, torch.tensor((0, 0, 1, 1), dtype=torch.int64), factor)
    out_b = _oal(q, k, v, torch.tensor((0, 1, 0, 1), dtype=torch.int64), factor)
    torch.testing.assert_close(out_a, out_b, atol=1e-11, rtol=1e-10)


def test_cross_group_coefficient_changes_result():
    q, k, v = _case(query_heads=1, key_heads=1)
    groups = torch.tensor((0, 0, 1, 1), dtype=torch.int32)
    factor = torch.tensor(CROSS_GROUP, dtype=torch.float64)
    no_cross = factor.clone()
    no_cross[3] = 0.0
    assert not torch.allclose(_oal(q, k, v, groups, factor), _oal(q, k, v, groups, no_cross))


@pytest.mark.parametrize("group_shape", ["shared", "per_head"])
@pytest.mark.parametrize("factor_shape", ["shared", "per_head"])
def test_group_and_factor_broadcast_combinations(group_shape, factor_shape):
    q, k, v = _case()
    groups = _two_group_mapping()
    factor = torch.tensor(CROSS_GROUP, dtype=torch.float64)
    passed_groups = groups[0] if group_shape == "shared" else groups
    passed_factor = factor if factor_shape == "shared" else factor.expand(q.shape[1], -1).clone()
    out = _oal(q, k, v, passed_groups, passed_factor)
    out_r, _, _ = go.dense_forward(q, k, v, passed_groups, passed_factor, scale=q.shape[-1] ** -0.5,
                                   kernel_eps=1e-6)
    torch.testing.assert_close(out.cpu(), out_r, atol=1e-11, rtol=1e-10)


def test_factor_and_qkv_gradients_match_dense_oracle():
    dev = _dev()
    q, k, v = _case(batch=1)
    groups = _two_group_mapping()
    factor = torch.tensor(CROSS_GROUP, dtype=torch.float64)
    upstream = torch.randn(q.shape[:-1] + (v.shape[-1],), generator=torch.Generator().manual_seed(5),
                           dtype=torch.float64)
    leaves = [t.to(dev).requires_grad_() for t in (q, k, v, factor)]
    from oal_amd import oal_attention

    out = oal_attention(*leaves[:3], groups.to(dev), leaves[3], scale=0.31, kernel_eps=0.09, execution="reference")
    out.backward(upstream.to(dev))
    ref = [t.clone().requires_grad_() for t in (q, k, v, factor)]
    out_r, _, _ = go.dense_forward(*ref[:3], groups, ref[3], scale=0.31, kernel_eps=0.09)
    out_r.backward(upstream)
    for name, a, r in zip(("q", "k", "v", "factor"), leaves, ref):
        torch.testing.assert_close(a.grad.cpu(), r.grad, atol=1e-10, rtol=1e-9, msg=f"d{name}")


def test_reference_execution_passes_gradcheck_on_the_device():
    from oal_amd import oal_attention

    dev = _dev()
    q, k, v = _case(batch=1, query_heads=1, key_heads=1, sequence=2, dimension=2, value_dimension=1)
    q, k, v = (t.to(dev).requires_grad_() for t in (q, k, v))
    factor = torch.tensor((1.0, 0.4, 0.8, 0.2, 0.3, 0.7), dtype=torch.float64, device=dev, requires_grad=True)
    groups = torch.tensor((0, 1), dtype=torch.int32, device=dev)

    def function(query, key, value, live_factor):
        return oal_attention(query, key, value, groups, live_factor, kernel_eps=0.1, execution="reference")

    assert torch.autograd.gradcheck(function, (q, k, v, factor), atol=1e-6, rtol=1e-4)


def test_broadcast_factor_gradient_reduces_across_query_heads():
    from oal_amd import oal_attention

    dev = _dev()
    q, k, v = (t.to(dev) for t in _case(batch=1))
    groups = _two_group_mapping().to(dev)
    shared = torch.tensor(CROSS_GROUP, dtype=torch.float64, device=dev, requires_grad=True)
    oal_attention(q, k, v, groups, shared, execution="reference").square().sum().backward()
    per_head = torch.tensor(CROSS_GROUP, dtype=torch.float64, device=dev).expand(q.shape[1], -1).clone()
    per_head.requires_grad_()
    oal_attention(q, k, v, groups, per_head, execution="reference").square().sum().backward()
    torch.testing.assert_close(shared.grad, per_head.grad.sum(dim=0), atol=1e-10, rtol=1e-9)


def test_inactive_padded_factor_entries_do_not_change_output_or_gradient():
    from oal_amd import oal_attention

    dev = _dev()
    q, k, v = (t.to(dev) for t in _case(query_heads=2, key_heads=1))
    groups = torch.tensor(((0, 0, 1, 1), (0, 0, 0, 0)), dtype=torch.int32, device=dev)
    factor = torch.tensor(CROSS_GROUP, dtype=torch.float64, device=dev).expand(2, -1).clone().requires_grad_()
    out = oal_attention(q, k, v, groups, factor, execution="reference")
    out[:, 1].square().sum().backward()
    assert torch.equal(factor.grad[0], torch.zeros_like(factor.grad[0]))
    torch.testing.assert_close(factor.grad[1, 3:], torch.zeros_like(factor.grad[1, 3:]))
    changed = factor.detach().clone()
    changed[1, 3:] = 9.0
    out_changed = oal_attention(q, k, v, groups, changed, execution="reference")
    torch.testing.assert_close(out_changed[:, 1], out[:, 1].detach(), atol=1e-11, rtol=1e-10)


def _grouped_case(b, hq, hkv, n, labels_of, g, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, n, 64, generator=gen, dtype=torch.float64) * 0.5
    k = torch.randn(b, hkv, n, 64, generator=gen, dtype=torch.float64) * 0.5
    v = torch.randn(b, hkv, n, 64, generator=gen, dtype=torch.float64)
    labels = labels_of(gen)
    low = torch.tril(torch.randn(hq, g + 1, g + 1, generator=gen, dtype=torch.float64) * 0.15)
    low.diagonal(dim1=-2, dim2=-1).copy_(0.5 + 0.3 * torch.rand(hq, g + 1, generator=gen, dtype=torch.float64))
    m = low @ low.transpose(-1, -2)
    return q, k, v, labels, m[:, 0, 0] + 1e-3, 2.0 * m[:, 0, 1:], m[:, 1:, 1:].contiguous()


@pytest.mark.parametrize("groups", [8, 64])
def test_grouped_function_fwd_bwd_multi_tile_ragged_gqa(groups):
    from oal_amd.hd_block_gemm_autograd import grouped_oal_f64

    dev = _dev()
    b, hq, hkv, n = (2, 4, 2, 70) if groups == 8 else (1, 2, 1, 70)
    if groups == 8:
        def labels_of(gen):
            return go.seeded_groups(64, go.UNEVEN_GROUP_SIZES, gen).unsqueeze(0).expand(hq, -1).contiguous()
    else:
        def labels_of(gen):
            return torch.arange(64, dtype=torch.int32).unsqueeze(0).expand(hq, -1).contiguous()
    q, k, v, labels, c0, lam, gam = _grouped_case(b, hq, hkv, n, labels_of, groups, seed=groups)
    scale = 0.125
    leaves = [t.to(dev).requires_grad_() for t in (q, k, v, c0, lam, gam)]
    out, num, den = grouped_oal_f64(leaves[0], leaves[1], leaves[2], labels.to(dev), *leaves[3:], scale=scale)
    gen = torch.Generator().manual_seed(7)
    dout = torch.randn(out.shape, generator=gen, dtype=torch.float64)
    dnum = torch.randn(num.shape, generator=gen, dtype=torch.float64)
    dden = torch.randn(den.shape, generator=gen, dtype=torch.float64)
    torch.autograd.backward((out, num, den), (dout.to(dev), dnum.to(dev), dden.to(dev)))

    ref = [t.clone().requires_grad_() for t in (q, k, v, c0, lam, gam)]
    num_r, den_r = go.dense_forward_coefficients(ref[0], ref[1], ref[2], labels, *ref[3:], scale=scale)
    out_r = num_r / den_r
    torch.autograd.backward((out_r, num_r, den_r), (dout, dnum, dden))

    def rel(a, r):
        return float((a.detach().cpu() - r.detach()).norm() / r.detach().norm())

    errs = {"out": rel(out, out_r), "num": rel(num, num_r), "den": rel(den, den_r)}
    for name, a, r in zip(("dq", "dk", "dv", "dc0", "dlam"), leaves, ref):
        errs[name] = rel(a.grad, r.grad)
    errs["dgam"] = rel(leaves[5].grad, go.symmetrize_gamma_gradient(ref[5].grad))
    print(f"fp64 route, {groups} groups, B={b} Hq={hq} Hkv={hkv} N={n}: "
          + " ".join(f"{k_}={e:.1e}" for k_, e in errs.items()), flush=True)
    for name, e in errs.items():
        assert e <= 1e-11, (name, e)


def test_partial_requests_and_reruns_are_bitwise_identical():
    from oal_amd import _native
    from oal_amd.hd_block_gemm_autograd import pad_labels

    dev = _dev()
    hq = 4
    q, k, v, labels, c0, lam, gam = _grouped_case(
        1, hq, 2, 90, lambda gen: go.seeded_groups(64, (10, 20, 34), gen).unsqueeze(0).expand(hq, -1).contiguous(),
        3, seed=2)
    q, k, v, c0, lam, gam = (t.to(dev).contiguous() for t in (q, k, v, c0, lam, gam))
    lab = pad_labels(labels.to(dev), hq)
    out, num, den = _native.forward_f64(q, k, v, lab, c0, lam, gam, scale=0.2)
    out2, num2, den2 = _native.forward_f64(q, k, v, lab, c0, lam, gam, scale=0.2)
    assert torch.equal(out, out2) and torch.equal(num, num2) and torch.equal(den, den2)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(1), dtype=torch.float64).to(dev)
    full = _native.backward_f64(q, k, v, lab, c0, lam, gam, num, den, dout, None, None, scale=0.2, need_q=True,
                                need_kv=True, need_coef=True)
    again = _native.backward_f64(q, k, v, lab, c0, lam, gam, num, den, dout, None, None, scale=0.2, need_q=True,
                                 need_kv=True, need_coef=True)
    only_q = _native.backward_f64(q, k, v, lab, c0, lam, gam, num, den, dout, None, None, scale=0.2, need_q=True,
                                  need_kv=False, need_coef=False)
    only_coef = _native.backward_f64(q, k, v, lab, c0, lam, gam, num, den, dout, None, None, scale=0.2,
                                     need_q=False, need_kv=False, need_coef=True)
    for a, b_ in zip(full, again):
        assert torch.equal(a, b_)
    assert torch.equal(only_q[0], full[0]) and only_q[1] is None and only_q[3] is None
    for i in (3, 4, 5):
        assert torch.equal(only_coef[i], full[i])
