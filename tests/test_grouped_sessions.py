"""Reference-quality sessions and parameter banks on the host (no kernel calls).

Mirrors the session contract of the reference adapter module
(qwen_lora_experiment/attention/grouped.py:261-324): the layer-id validation and
its error types, the all-or-nothing switch of the OAL layers to the reference
execution, the restore on exit (also when the block raises) and the rejection of
a session that starts with a layer already switched. The GPU side (the N=128
alignment record, and that a session's forward is the fp32 kernels' forward) is
tests/test_gpu_sessions.py.
"""

import os

import pytest
import torch

from oal_amd.group_assets import load_oal_group_asset
from oal_amd.grouped_sessions import (
    GroupedQuadraticAttentionError,
    OALParameterBank,
    grouped_quadratic_reference_alignment,
    grouped_quadratic_reference_quality_session,
    grouped_quadratic_reference_session,
)
from oal_amd.qwen_oal import QwenOALConfig, QwenOALModel

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "oal_qwen_asset_subset.json")


def _model(layers=3):
    return QwenOALModel(QwenOALConfig(vocab_size=64, hidden_size=64, intermediate_size=32, num_layers=layers))


def _modes(model):
    return [layer.attn._grouped_execution for layer in model.layers]


def test_session_switches_every_layer_and_restores():
    model = _model()
    assert _modes(model) == ["triton"] * 3
    assert {layer.attn.execution_precision() for layer in model.layers} == {"bf16_tensorcore"}
    with grouped_quadratic_reference_session(model, expected_layer_ids=[0, 1, 2]):
        assert _modes(model) == ["reference"] * 3
        assert {layer.attn.execution_precision() for layer in model.layers} == {"fp32_ieee"}
    assert _modes(model) == ["triton"] * 3
    with grouped_quadratic_reference_quality_session(model, expected_layer_ids=(0, 1, 2)):
        assert _modes(model) == ["reference"] * 3
    assert _modes(model) == ["triton"] * 3


def test_session_restores_when_the_block_raises():
    model = _model()
    with pytest.raises(KeyError):
        with grouped_quadratic_reference_session(model, expected_layer_ids=[0, 1, 2]):
            raise KeyError("scorer failed")
    assert _modes(model) == ["triton"] * 3


@pytest.mark.parametrize("ids,exc", [
    ([], ValueError), ([1, 0, 2], ValueError), ([0, 0, 1, 2], ValueError), ([0, -1], ValueError),
    ([0, 1.0, 2], ValueError), ("012", TypeError), ([0, 1], GroupedQuadraticAttentionError),
    ([0, 1, 2, 3], GroupedQuadraticAttentionError),
])
def test_session_rejects_layer_ids(ids, exc):
    model = _model()
    with pytest.raises(exc):
        with grouped_quadratic_reference_session(model, expected_layer_ids=ids):
            pass
    assert _modes(model) == ["triton"] * 3


def test_session_rejects_non_modules_and_a_partial_switch():
    with pytest.raises(TypeError):
        with grouped_quadratic_reference_session(object(), expected_layer_ids=[0]):
            pass
    with pytest.raises(GroupedQuadraticAttentionError):
        with grouped_quadratic_reference_session(torch.nn.Linear(2, 2), expected_layer_ids=[0]):
            pass
    model = _model()
    model.layers[1].attn._grouped_execution = "reference"
    with pytest.raises(GroupedQuadraticAttentionError, match="begin in Triton mode"):
        with grouped_quadratic_reference_session(model, expected_layer_ids=[0, 1, 2]):
            pass
    assert _modes(model) == ["triton", "reference", "triton"]  # left as found


def test_invalid_execution_mode_is_an_error():
    model = _model(1)
    model.layers[0].attn._grouped_execution = "auto"
    with pytest.raises(GroupedQuadraticAttentionError, match="layer=0: adapter has an invalid grouped execution mode"):
        model.layers[0].attn.execution_precision()


def test_parameter_banks_from_model_and_asset():
    model = _model()
    bank = OALParameterBank.from_model(model)
    assert bank.active_kernel_layer_ids() == (0, 1, 2)
    assert (bank.geometry.num_query_heads, bank.geometry.num_kv_heads, bank.geometry.head_dim) == (14, 2, 64)
    assert torch.equal(bank.dim_groups_for_layer(1), model.layers[1].attn.dim_groups)
    assert torch.equal(bank.packed_grouped_factor_for_layer(2), model.layers[2].attn.factor)
    assert bank.grouped_kernel_epsilon_for_runtime() == model.cfg.kernel_eps
    with pytest.raises(KeyError):
        bank.dim_groups_for_layer(3)
    asset = load_oal_group_asset(GOLDEN)
    abank = OALParameterBank.from_asset(asset)
    assert abank.active_kernel_layer_ids() == tuple(sorted(asset.layer_ids_zero_based))
    lid = asset.layer_ids_zero_based[0]
    assert torch.equal(abank.dim_groups_for_layer(lid), asset.dim_groups_for_layer(lid))
    assert abank.packed_grouped_factor_for_layer(lid).shape == (14, 45)
    assert abank.grouped_kernel_epsilon_for_runtime() == asset.epsilon


def test_alignment_seed_must_be_an_integer():
    bank = OALParameterBank.from_model(_model(1))
    with pytest.raises(TypeError):
        grouped_quadratic_reference_alignment(parameter_bank=bank, layer_id=0, device="cpu", seed=1.0)
