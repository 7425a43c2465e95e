"""Non-positive denominators and the reference execution on the GPU.

The BASELINE config coefficients (c0 = 1, lam ~ U(0.5, 1.5), Gam_gh ~ U(0, 0.5)
for g <= h, mirrored) are not PSD, and the fp32 oracle finds one token with
den <= 0 at config 1 (tests/test_config_denominators.py pins the counts). The
reference refuses such an output: its HD runtime checks den > 0 after the
forward (hd_block_gemm_runtime.py:392-408), and its public entry points
(oal_attention, grouped_causal_attention) take a packed PSD factor, so that
kappa = ||[1, s] L||^2 + eps > 0 and no factor can carry these coefficients.

* The logical-coefficient HD Function with a plan raises on the config-1 inputs,
  as the reference's does.
* The grouped Function the benchmark times has no positivity check (as the
  reference's private candidate route); it returns the non-positive
  denominators, which are printed.
* oal_attention / grouped_causal_attention with a PSD factor give den > 0 on
  every token of the same q, k, v.
* oal_attention(execution="reference") runs the fp32 HIP kernels on ROCm tensors
  (the reference's pure-torch route, used by its quality sessions on GPU
  tensors, qwen_lora_experiment/attention/grouped.py:125-152): rel-L2 <= 1e-5
  against the fp32 oracle, bf16 inputs included (cast to fp32 as the reference
  does).
"""

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _config1(dev):
    inp = go.config_inputs(1)
    qb, kb, vb = (inp[n].to(torch.bfloat16).to(dev) for n in ("q", "k", "v"))
    return inp, qb, kb, vb


def _logical(inp, dev):
    """(a, b, c) of the reference HD family: a = c0, b_d = lam[g(d)], c_p(r,c) = Gam[g(r)][g(c)]."""
    labels = inp["groups"].long()
    hq = labels.shape[0]
    rows, cols = torch.tril_indices(64, 64)
    a = inp["c0"].clone()
    b = torch.gather(inp["lam"], 1, labels)
    gam = inp["gam"]
    c = torch.stack([gam[h][labels[h][rows], labels[h][cols]] for h in range(hq)])
    return a.to(dev), b.to(dev), c.to(dev)


def test_config1_inputs_raise_through_the_hd_function_like_the_reference():
    from oal_amd.hd_block_gemm import build_hd_block_gemm_plan, canonical_pair_layout
    from oal_amd.hd_block_gemm_autograd import _hd_parallel_block_gemm

    dev = _dev()
    inp, qb, kb, vb = _config1(dev)
    a, b, c = _logical(inp, dev)
    plan = build_hd_block_gemm_plan(qb, kb, vb, precision="bf16_tensorcore", requested_gradient_mask=(False,) * 6)
    assert plan.require_positive_denominator
    with pytest.raises(RuntimeError, match="strictly positive"):
        _hd_parallel_block_gemm(qb, kb, vb, a, b, c, scale=inp["scale"], eps=1e-30,
                                layout=canonical_pair_layout(64), plan=plan)


def test_bench_route_returns_the_nonpositive_denominators():
    from oal_amd.hd_block_gemm_autograd import _GroupedOALFunction

    dev = _dev()
    inp, qb, kb, vb = _config1(dev)
    c0, lam, gam, labels = (inp[n].to(dev) for n in ("c0", "lam", "gam", "groups"))
    with torch.no_grad():
        _, _, den = _GroupedOALFunction.apply(qb, kb, vb, c0, lam, gam, labels, inp["scale"], 0.0, "bf16")
    q32, k32, v32 = (t.float().cpu() for t in (qb, kb, vb))
    wq = go.feature_coefficients(inp["groups"], inp["c0"], inp["lam"], inp["gam"], scale=inp["scale"], head_dim=64)
    _, _, den_r = go.chunked_forward(q32, k32, v32, wq, chunk=64)
    got, want = int((den <= 0).sum()), int((den_r <= 0).sum())
    print(f"config 1: den <= 0 on {got} tokens (oracle: {want}), min den {float(den.min()):.3f} "
          f"(oracle {float(den_r.min()):.3f})", flush=True)
    assert want == 1
    # the sign of a near-zero denominator is at the mercy of bf16 rounding; the
    # most negative one is not
    assert float(den.min()) < 0
    assert abs(float(den.min()) - float(den_r.min())) <= 0.5


def _psd_factor(hq, gen):
    side = 9
    rows = []
    for _ in range(hq):
        low = torch.tril(torch.randn((side, side), generator=gen) * 0.15)
        low.diagonal().copy_(0.5 + 0.5 * torch.rand(side, generator=gen))
        r, c = torch.tril_indices(side, side)
        rows.append(low[r, c])
    return torch.stack(rows).float()


def test_public_entry_points_with_a_psd_factor_have_positive_denominators():
    from oal_amd import oal_attention
    from oal_amd.hd_attention import grouped_causal_attention

    dev = _dev()
    inp, qb, kb, vb = _config1(dev)
    factor = _psd_factor(14, torch.Generator().manual_seed(3)).to(dev)
    groups = inp["groups"].to(dev)
    _, _, den = oal_attention(qb, kb, vb, groups, factor, return_unnormalized=True)
    assert bool((den > 0).all())
    _, _, den2 = grouped_causal_attention(qb, kb, vb, groups, factor, precision="bf16_tensorcore")
    assert bool((den2 > 0).all())
    print(f"PSD factor on the config-1 q, k, v: min den {float(den.min()):.3f} (fp32 route), "
          f"{float(den2.min()):.3f} (bf16 matrix cores)", flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_execution_runs_the_fp32_kernels_on_rocm(dtype):
    from oal_amd import oal_attention

    dev = _dev()
    gen = torch.Generator().manual_seed(8)
    b, hq, hkv, n = 1, 14, 2, 200
    q = (torch.randn(b, hq, n, 64, generator=gen) * 0.5).to(dtype)
    k = (torch.randn(b, hkv, n, 64, generator=gen) * 0.5).to(dtype)
    v = torch.randn(b, hkv, n, 64, generator=gen).to(dtype)
    labels = go.seeded_groups(64, go.UNEVEN_GROUP_SIZES, gen).unsqueeze(0).expand(hq, -1).contiguous()
    factor = _psd_factor(hq, gen)
    out, num, den = oal_attention(q.to(dev), k.to(dev), v.to(dev), labels.to(dev), factor.to(dev),
                                  execution="reference", return_unnormalized=True)
    assert out.dtype == dtype and num.dtype == torch.float32 and den.shape == (b, hq, n, 1)
    c0, lam, gam = go.expand_factor(factor.double(), query_heads=hq, kernel_eps=1e-6)
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=0.125, head_dim=64)
    out_r, num_r, den_r = go.chunked_forward(q.double(), k.double(), v.double(), wq, chunk=64)
    errs = {"num": rel(num, num_r), "den": rel(den, den_r), "out": rel(out.float(), out_r)}
    print(f"execution='reference' ({dtype}): " + " ".join(f"{k_}={e:.2e}" for k_, e in errs.items()), flush=True)
    assert errs["num"] <= FP32_TOL and errs["den"] <= FP32_TOL
    # out is stored in the input dtype
    assert errs["out"] <= (FP32_TOL if dtype == torch.float32 else 1e-2)
