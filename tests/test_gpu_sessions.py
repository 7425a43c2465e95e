"""Reference-quality execution on the GPU (the reference's attention/grouped.py:261-441).

* The N=128 alignment guard runs each layer of the released asset subset
  (tests/golden/oal_qwen_asset_subset.json: layers 0, 7, 12) and the layers of a
  seeded model through the fp32 kernels ("reference") and the bf16 matrix-core
  kernels ("triton"): the record must report allclose(atol=0.03, rtol=0.03).
* Inside grouped_quadratic_reference_session the model's forward is the fp32
  kernels' forward: bit-identical to the same model built with precision
  fp32_ieee, and within bf16 tolerance (rel-L2 <= 2e-2) of the fast execution.
"""

import os

import pytest
import torch

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "oal_qwen_asset_subset.json")


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def test_alignment_on_the_released_asset_layers():
    from oal_amd.group_assets import load_oal_group_asset
    from oal_amd.grouped_sessions import (OALParameterBank, grouped_quadratic_reference_alignment,
                                          grouped_quadratic_reference_quality_alignment)

    dev = _dev()
    asset = load_oal_group_asset(GOLDEN)
    bank = OALParameterBank.from_asset(asset)
    for layer_id in asset.layer_ids_zero_based:
        rec = grouped_quadratic_reference_alignment(parameter_bank=bank, layer_id=layer_id, device=dev, seed=layer_id)
        print(layer_id, rec, flush=True)
        assert rec["schema"] == "grouped_reference_alignment_v1" and rec["within_tolerance"]
        assert rec["sequence_length"] == 128 and rec["layer_id"] == layer_id and rec["seed"] == layer_id
        assert 0.0 < rec["mean_abs_error"] <= rec["max_abs_error"]
    rec = grouped_quadratic_reference_quality_alignment(parameter_bank=bank, layer_id=asset.layer_ids_zero_based[0],
                                                        device=dev, seed=3)
    assert rec["schema"] == "grouped_piqa_reference_alignment_v1" and rec["within_tolerance"]


def test_alignment_on_seeded_model_layers():
    from oal_amd.grouped_sessions import OALParameterBank, grouped_quadratic_reference_alignment
    from oal_amd.qwen_oal import QwenOALConfig, QwenOALModel

    dev = _dev()
    model = QwenOALModel(QwenOALConfig(vocab_size=64, hidden_size=896, intermediate_size=32, num_layers=2))
    bank = OALParameterBank.from_model(model)
    for layer_id in (0, 1):
        rec = grouped_quadratic_reference_alignment(parameter_bank=bank, layer_id=layer_id, device=dev, seed=7)
        assert rec["within_tolerance"], rec


def test_reference_session_forward_is_the_fp32_kernels():
    from oal_amd.grouped_sessions import grouped_quadratic_reference_session
    from oal_amd.qwen_oal import QwenOALConfig, QwenOALModel

    dev = _dev()
    cfg = QwenOALConfig(vocab_size=512, num_layers=2, intermediate_size=256)
    fast = QwenOALModel(cfg, seed=0).to(dev)
    exact = QwenOALModel(QwenOALConfig(vocab_size=512, num_layers=2, intermediate_size=256,
                                       precision="fp32_ieee"), seed=0).to(dev)
    tokens = torch.randint(0, cfg.vocab_size, (1, 200), generator=torch.Generator().manual_seed(1)).to(dev)
    with torch.no_grad():
        out_fast = fast(tokens)
        with grouped_quadratic_reference_session(fast, expected_layer_ids=[0, 1]):
            out_ref = fast(tokens)
        out_again = fast(tokens)
        out_exact = exact(tokens)
    err = _rel(out_fast, out_ref)
    print("fast vs reference-session logits rel-L2", err, flush=True)
    assert torch.equal(out_ref, out_exact)
    assert torch.equal(out_again, out_fast)
    assert 0.0 < err <= 2e-2
