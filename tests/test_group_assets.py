"""Group / coefficient asset loader (oal_amd.group_assets) on the reference's own data.

tests/golden/oal_qwen_asset_subset.json holds layers 0, 7 and 12 of the released
configs/oal_qwen_n4096.json unchanged (tests/golden/make_asset_subset.py). Each head
record stores its expanded quadratic matrix M = L_active L_active^T next to the
layer-padded packed factor: that is the known answer the loader, the active
truncation and the factor -> (c0, lam, Gam) expansion are pinned against.
"""

import copy
import json
import os

import numpy as np
import pytest
import torch

from oal_amd.group_assets import FACTOR_SIZE, active_packed_length, expand_packed_lower_triangular, load_oal_group_asset
from oracle import grouped_oracle as go

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "oal_qwen_asset_subset.json")


def _raw():
    with open(GOLDEN) as fh:
        return json.load(fh)


def test_reference_asset_subset_loads_with_labels_and_padded_factors():
    asset = load_oal_group_asset(GOLDEN)
    assert asset.layer_ids_zero_based == (0, 7, 12)
    labels = asset.dim_groups()
    assert labels.shape == (3, 14, 64) and labels.dtype == torch.int32
    counts = asset.group_counts()
    raw = _raw()
    for off, layer in enumerate(asset.layer_ids_zero_based):
        factor = asset.packed_grouped_factor_for_layer(layer)
        assert factor.shape == (14, FACTOR_SIZE) and factor.dtype == torch.float32
        for h in range(14):
            rec = raw["layers"][str(layer)]["heads"][str(h)]
            gc = rec["group_count"]
            assert counts[off, h] == gc
            for g, dims in enumerate(rec["groups"]):
                assert (labels[off, h, dims] == g).all()
            n = active_packed_length(gc)
            assert torch.equal(factor[h, :n], torch.tensor(rec["packed_lower_triangular"][:n], dtype=torch.float32))
            assert (factor[h, n:] == 0).all()


def test_active_truncation_is_what_reconstructs_the_stored_matrix():
    """Heads with non-zero stored entries past the active length: the stored
    matrix equals L_active L_active^T, and the untruncated factor does not give it."""
    raw = _raw()
    tails = 0
    for layer in raw["layers"].values():
        gmax = layer["max_groups"]
        for rec in layer["heads"].values():
            gc = rec["group_count"]
            packed = rec["packed_lower_triangular"]
            stored = np.asarray(rec["expanded_quadratic_matrix"])
            active = np.zeros_like(stored)
            active[:gc + 1, :gc + 1] = expand_packed_lower_triangular(packed[:active_packed_length(gc)], gc + 1)
            assert np.allclose(active, stored, rtol=2e-5, atol=2e-5)
            if any(x != 0 for x in packed[active_packed_length(gc):]):
                tails += 1
                assert not np.allclose(expand_packed_lower_triangular(packed, gmax + 1), stored, rtol=2e-5, atol=2e-5)
    assert tails >= 8


def test_asset_factor_expands_to_the_stored_matrix_in_both_expansions():
    """c0 = M00 + eps, lam = 2 M[0, 1:], Gam = M[1:, 1:] with M the stored matrix,
    from the padded [14, 45] factor (oracle expansion and the package's own)."""
    from oal_amd.grouped_quadratic import _expand_factor_coefficients

    asset = load_oal_group_asset(GOLDEN)
    raw = _raw()
    for layer in asset.layer_ids_zero_based:
        factor = asset.packed_grouped_factor_for_layer(layer).double()
        c0, lam, gam = go.expand_factor(factor, query_heads=14, kernel_eps=asset.epsilon)
        c0b, lamb, gamb = _expand_factor_coefficients(factor, query_heads=14, gmax=8, kernel_eps=asset.epsilon,
                                                      working_dtype=torch.float64)
        for h in range(14):
            m = torch.tensor(raw["layers"][str(layer)]["heads"][str(h)]["expanded_quadratic_matrix"], dtype=torch.float64)
            s = m.shape[0]
            for got_c0, got_lam, got_gam in ((c0, lam, gam), (c0b, lamb, gamb)):
                assert abs(float(got_c0[h]) - (float(m[0, 0]) + asset.epsilon)) <= 1e-5 * max(1.0, abs(float(m[0, 0])))
                assert torch.allclose(got_lam[h, :s - 1].double(), 2 * m[0, 1:], rtol=2e-5, atol=2e-5)
                assert torch.allclose(got_gam[h, :s - 1, :s - 1].double(), m[1:, 1:], rtol=2e-5, atol=2e-5)
                assert float(got_gam[h, s - 1:].abs().sum()) == 0.0


@pytest.mark.parametrize("mutation", ["missing_key", "duplicate_dim", "uncovered_dim", "packed_length",
                                      "matrix", "group_count", "special_dims", "unknown_root"])
def test_malformed_assets_are_rejected(mutation):
    data = _raw()
    bad = copy.deepcopy(data)
    rec = bad["layers"]["0"]["heads"]["3"]
    if mutation == "missing_key":
        del rec["validation_output_mse"]
    elif mutation == "duplicate_dim":
        rec["groups"][1] = sorted(set(rec["groups"][1]) | {rec["groups"][0][0]})
    elif mutation == "uncovered_dim":
        rec["groups"][0] = rec["groups"][0][1:]
    elif mutation == "packed_length":
        rec["packed_lower_triangular"] = rec["packed_lower_triangular"][:-1]
    elif mutation == "matrix":
        rec["expanded_quadratic_matrix"][0][0] += 1e-3
    elif mutation == "group_count":
        rec["group_count"] = bad["layers"]["0"]["max_groups"] + 1
    elif mutation == "special_dims":
        rec["special_dims"] = list(reversed(rec.get("special_dims", [0, 1])))
    elif mutation == "unknown_root":
        bad["extra"] = 1
    load_oal_group_asset(data)
    with pytest.raises(ValueError):
        load_oal_group_asset(bad)


def test_model_takes_groups_and_factors_from_the_asset():
    from oal_amd.qwen_oal import QwenOALConfig, QwenOALModel

    asset = load_oal_group_asset(GOLDEN)
    model = QwenOALModel(QwenOALConfig(vocab_size=64, num_layers=13, intermediate_size=32)).load_group_asset(asset)
    for layer in asset.layer_ids_zero_based:
        attn = model.layers[layer].attn
        assert torch.equal(attn.dim_groups, asset.dim_groups_for_layer(layer))
        assert torch.equal(attn.factor, asset.packed_grouped_factor_for_layer(layer))
        assert attn.kernel_eps == asset.epsilon
