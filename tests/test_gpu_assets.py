"""The reference's released grouping (layers 0, 7, 12 of configs/oal_qwen_n4096.json,
tests/golden/oal_qwen_asset_subset.json) through the HIP operator on the GPU.

Each layer's [14, 64] labels and padded [14, 45] factor go through
oal_attention(execution="triton") (fp32 kernels; rel-L2 <= 1e-5) and through the
HD family's grouped_causal_attention with precision "bf16_tensorcore" (matrix
cores; rel-L2 <= 2e-2), against the dense token-pair oracle in fp64 with the
asset's epsilon and scale 64^-1/2.
"""

import os

import pytest
import torch

from oal_amd.group_assets import load_oal_group_asset
from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "oal_qwen_asset_subset.json")


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("layer", [0, 7, 12])
def test_asset_layer_through_hip_operator_matches_dense_oracle(layer):
    from oal_amd import oal_attention
    from oal_amd.hd_attention import grouped_causal_attention

    dev = _dev()
    asset = load_oal_group_asset(GOLDEN)
    groups = asset.dim_groups_for_layer(layer)
    factor = asset.packed_grouped_factor_for_layer(layer)
    gen = torch.Generator().manual_seed(layer)
    q = torch.randn((1, 14, 200, 64), generator=gen)
    k = torch.randn((1, 2, 200, 64), generator=gen)
    v = torch.randn((1, 2, 200, 64), generator=gen)
    scale = 64 ** -0.5
    out_r, num_r, den_r = go.dense_forward(q.double(), k.double(), v.double(), groups, factor.double(), scale=scale,
                                           kernel_eps=asset.epsilon)
    out, num, den = oal_attention(q.to(dev), k.to(dev), v.to(dev), groups.to(dev), factor.to(dev), scale=scale,
                                  kernel_eps=asset.epsilon, execution="triton", return_unnormalized=True)
    e32 = {"out": _rel(out, out_r), "num": _rel(num, num_r), "den": _rel(den, den_r)}
    qb, kb, vb = (t.to(torch.bfloat16) for t in (q, k, v))
    out_rb, _, _ = go.dense_forward(qb.double(), kb.double(), vb.double(), groups, factor.double(), scale=scale,
                                    kernel_eps=asset.epsilon)
    outb, numb, denb = grouped_causal_attention(qb.to(dev), kb.to(dev), vb.to(dev), groups.to(dev), factor.to(dev),
                                                scale=scale, kernel_eps=asset.epsilon, precision="bf16_tensorcore")
    e16 = _rel(outb.float(), out_rb)
    print(f"asset layer {layer}: fp32 {e32}, bf16 out {e16:.2e}")
    assert all(e <= 1e-5 for e in e32.values()), e32
    assert e16 <= 2e-2


@pytest.mark.parametrize("layer", [0, 12])
def test_asset_layer_backward_bf16_matches_dense_oracle(layer):
    """The released groupings (2..5 active groups in a factor padded to Gmax = 8)
    through the matrix-core backward: dq, dk, dv and the factor gradient against
    autograd of the fp64 dense oracle on the same bf16-rounded q, k, v and dO.
    kappa = ||[1, z] L||^2 + eps is positive for every pair, so every denominator
    is a sum of positive terms and the whole upstream gradient is kept.
    Tolerance rel-L2 <= 2e-2 (bf16 mode)."""
    from oal_amd.hd_attention import grouped_causal_attention

    dev = _dev()
    asset = load_oal_group_asset(GOLDEN)
    groups = asset.dim_groups_for_layer(layer)
    factor = asset.packed_grouped_factor_for_layer(layer)
    gen = torch.Generator().manual_seed(100 + layer)
    q, k, v = (torch.randn(shape, generator=gen).to(torch.bfloat16)
               for shape in ((1, 14, 160, 64), (1, 2, 160, 64), (1, 2, 160, 64)))
    dout = torch.randn((1, 14, 160, 64), generator=gen)
    scale = 64 ** -0.5
    ref = [t.double().requires_grad_() for t in (q, k, v, factor)]
    out_r, _, _ = go.dense_forward(ref[0], ref[1], ref[2], groups, ref[3], scale=scale, kernel_eps=asset.epsilon)
    (out_r * dout.double()).sum().backward()
    ins = [t.to(dev).requires_grad_() for t in (q, k, v, factor)]
    out, _, _ = grouped_causal_attention(ins[0], ins[1], ins[2], groups.to(dev), ins[3], scale=scale,
                                         kernel_eps=asset.epsilon, precision="bf16_tensorcore")
    (out.float() * dout.to(dev)).sum().backward()
    errs = {name: _rel(x.grad.float(), r.grad) for name, x, r in zip(("dq", "dk", "dv", "dfactor"), ins, ref)}
    errs["out"] = _rel(out.float(), out_r)
    print(f"asset layer {layer} bf16 backward rel-L2: " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()),
          flush=True)
    assert all(e <= 2e-2 for e in errs.values()), errs
