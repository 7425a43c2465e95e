"""Group / coefficient asset loader for OAL layers (the released ``configs/oal_qwen_n4096.json`` format).

Follows the reference's legacy adaptive asset contract:
* root keys and head-record keys: qwen_lora_experiment/grouped_asset_contract.py:84-106;
* head validation: legacy_group_assets.py:170-236 (group count 2..5 and at most the
  layer's ``max_groups``, an exact sorted partition of dimensions 0..63, the packed
  factor stored at the layer-padded length ``(max_groups+1)(max_groups+2)/2`` and
  truncated to the active length ``(group_count+1)(group_count+2)/2``, the stored
  ``expanded_quadratic_matrix`` reconstructed from the active factor to
  rtol = atol = 2e-5, ``special_dims`` equal to the non-zero groups in order);
* labels: grouped_initialization.py:28-38 (dimension d of group g gets label g),
  ``[L, 14, 64]`` int32;
* factors: kernel_parameters.py:115-236 (the active factor zero-padded to the public
  ``[14, 45]`` fp32 layout of Gmax = 8, ``packed_grouped_factor_for_layer``).

The active truncation matters: stored factors may carry non-zero entries past the
active length; they belong to no group and are dropped, as the reference does.
"""

from __future__ import annotations

import json
import math
import os
from dataclasses import dataclass
from typing import Mapping

import numpy as np
import torch

HEAD_DIM = 64
QUERY_HEADS = 14
GMAX = 8
FACTOR_SIZE = (GMAX + 1) * (GMAX + 2) // 2  # 45
GROUP_COUNT_RANGE = range(2, 6)
MATRIX_TOLERANCE = 2e-5

_ROOT_REQUIRED = {
    "model_name", "layer_ids_zero_based", "head_dim", "epsilon", "seq_len", "method", "objective",
    "parameterization", "train_indices", "validation_indices", "test_indices", "layers",
}
_ROOT_OPTIONAL = {"schema", "minimum_group_count"}
_HEAD_REQUIRED = {"group_count", "groups", "packed_lower_triangular", "expanded_quadratic_matrix",
                  "validation_output_mse"}
_HEAD_OPTIONAL = {"special_dims"}


def active_packed_length(group_count: int) -> int:
    """Length of a packed lower-triangular factor of side group_count + 1."""
    return (group_count + 1) * (group_count + 2) // 2


def expand_packed_lower_triangular(packed, side: int) -> np.ndarray:
    """Row-major packed lower triangle -> L L^T (float64)."""
    lower = np.zeros((side, side), dtype=np.float64)
    rows, cols = np.tril_indices(side)
    lower[rows, cols] = np.asarray(packed, dtype=np.float64)
    return lower @ lower.T


@dataclass(frozen=True)
class GroupHeadRecord:
    layer_id: int
    head_id: int
    group_count: int
    stored_gmax: int
    groups: tuple
    active_factor: tuple
    expanded_quadratic_matrix: np.ndarray
    validation_output_mse: float


@dataclass(frozen=True)
class OALGroupAsset:
    model_name: str
    layer_ids_zero_based: tuple
    head_dim: int
    epsilon: float
    seq_len: int
    heads: Mapping  # (layer_id, head_id) -> GroupHeadRecord
    num_query_heads: int = QUERY_HEADS

    def dim_groups(self) -> torch.Tensor:
        """``[L, Hq, 64]`` int32 labels of the asset's layers (build_grouped_dim_groups)."""
        labels = torch.empty((len(self.layer_ids_zero_based), self.num_query_heads, self.head_dim),
                             dtype=torch.int32)
        for off, layer in enumerate(self.layer_ids_zero_based):
            for head in range(self.num_query_heads):
                for g, dims in enumerate(self.heads[layer, head].groups):
                    labels[off, head, list(dims)] = g
        return labels

    def dim_groups_for_layer(self, layer_id: int) -> torch.Tensor:
        """``[Hq, 64]`` int32 labels of one layer."""
        return self.dim_groups()[self._offset(layer_id)].contiguous()

    def group_counts(self) -> torch.Tensor:
        """``[L, Hq]`` int32 active group counts."""
        return torch.tensor([[self.heads[layer, h].group_count for h in range(self.num_query_heads)]
                             for layer in self.layer_ids_zero_based], dtype=torch.int32)

    def packed_grouped_factor_for_layer(self, layer_id: int) -> torch.Tensor:
        """``[Hq, 45]`` fp32: each head's active factor, zero-padded to Gmax = 8."""
        self._offset(layer_id)
        rows = []
        for head in range(self.num_query_heads):
            active = torch.tensor(self.heads[layer_id, head].active_factor, dtype=torch.float32)
            rows.append(torch.cat((active, torch.zeros(FACTOR_SIZE - active.numel(), dtype=torch.float32))))
        return torch.stack(rows).contiguous()

    def _offset(self, layer_id: int) -> int:
        if layer_id not in self.layer_ids_zero_based:
            raise KeyError(f"layer {layer_id} is not in the asset (layers {list(self.layer_ids_zero_based)})")
        return self.layer_ids_zero_based.index(layer_id)


def _require_keys(obj: Mapping, required: set, optional: set, path: str) -> None:
    if not isinstance(obj, Mapping):
        raise ValueError(f"{path} must be an object")
    unknown = sorted(set(obj) - required - optional)
    if unknown:
        raise ValueError(f"{path} has unknown field(s): {', '.join(unknown)}")
    missing = sorted(required - set(obj))
    if missing:
        raise ValueError(f"{path} is missing required field(s): {', '.join(missing)}")


def _finite(value, path: str, *, nonnegative: bool = False) -> float:
    if type(value) not in (int, float) or not math.isfinite(value):
        raise ValueError(f"{path} must be a finite number")
    if nonnegative and value < 0:
        raise ValueError(f"{path} must be non-negative")
    return float(value)


def _partition(value, group_count: int, path: str) -> tuple:
    if not isinstance(value, list) or len(value) != group_count:
        raise ValueError(f"{path} must contain exactly group_count groups")
    seen: set = set()
    groups = []
    for g, raw in enumerate(value):
        gp = f"{path}[{g}]"
        if not isinstance(raw, list) or not raw:
            raise ValueError(f"{gp} must be a non-empty integer list")
        if any(type(d) is not int or d < 0 or d >= HEAD_DIM for d in raw):
            raise ValueError(f"{gp} must contain integer dimensions in 0..63")
        if raw != sorted(raw) or len(set(raw)) != len(raw):
            raise ValueError(f"{gp} must be strictly sorted and unique")
        overlap = seen & set(raw)
        if overlap:
            raise ValueError(f"{path} partition has duplicate dimensions: {sorted(overlap)!r}")
        seen.update(raw)
        groups.append(tuple(raw))
    if seen != set(range(HEAD_DIM)):
        missing = sorted(set(range(HEAD_DIM)) - seen)
        raise ValueError(f"{path} partition must cover dimensions 0..63 exactly; missing={missing!r}")
    return tuple(groups)


def _head(raw, *, layer_id: int, head_id: int, stored_gmax: int, path: str) -> GroupHeadRecord:
    _require_keys(raw, _HEAD_REQUIRED, _HEAD_OPTIONAL, path)
    gc = raw["group_count"]
    if type(gc) is not int or gc not in GROUP_COUNT_RANGE:
        raise ValueError(f"{path}.group_count must be an integer group count in 2..5")
    if gc > stored_gmax:
        raise ValueError(f"{path}.group_count must not exceed layer max_groups")
    groups = _partition(raw["groups"], gc, f"{path}.groups")
    stored_len = active_packed_length(stored_gmax)
    packed = raw["packed_lower_triangular"]
    if not isinstance(packed, list) or len(packed) != stored_len:
        raise ValueError(f"{path}.packed_lower_triangular must have the layer-padded length {stored_len}")
    stored = tuple(_finite(x, f"{path}.packed_lower_triangular[{i}]") for i, x in enumerate(packed))
    active = stored[:active_packed_length(gc)]
    expected = np.zeros((stored_gmax + 1, stored_gmax + 1))
    expected[:gc + 1, :gc + 1] = expand_packed_lower_triangular(active, gc + 1)
    mat = raw["expanded_quadratic_matrix"]
    side = stored_gmax + 1
    if not isinstance(mat, list) or len(mat) != side or any(not isinstance(r, list) or len(r) != side for r in mat):
        raise ValueError(f"{path}.expanded_quadratic_matrix must be a {side}x{side} matrix")
    matrix = np.asarray([[_finite(x, f"{path}.expanded_quadratic_matrix[{i}][{j}]") for j, x in enumerate(r)]
                         for i, r in enumerate(mat)], dtype=np.float64)
    if not np.allclose(matrix, expected, rtol=MATRIX_TOLERANCE, atol=MATRIX_TOLERANCE):
        raise ValueError(f"{path}.expanded_quadratic_matrix does not reconstruct from the stored factor")
    if "special_dims" in raw:
        flat = [d for grp in groups[1:] for d in grp]
        if raw["special_dims"] != flat:
            raise ValueError(f"{path}.special_dims must equal the nonzero groups in order")
    mse = _finite(raw["validation_output_mse"], f"{path}.validation_output_mse", nonnegative=True)
    return GroupHeadRecord(layer_id, head_id, gc, stored_gmax, groups, active, matrix, mse)


def load_oal_group_asset(source, *, num_query_heads: int = QUERY_HEADS) -> OALGroupAsset:
    """Validate and load an asset from a path, a JSON string's parsed dict, or a dict.

    Raises ValueError naming the offending field, as the reference loader does
    (legacy_group_assets.py:39-236).
    """
    if isinstance(source, (str, os.PathLike)):
        with open(source) as fh:
            data = json.load(fh)
    else:
        data = source
    _require_keys(data, _ROOT_REQUIRED, _ROOT_OPTIONAL, "group asset")
    if data["head_dim"] != HEAD_DIM or type(data["head_dim"]) is not int:
        raise ValueError(f"group asset head_dim must be exactly {HEAD_DIM}")
    eps = _finite(data["epsilon"], "group asset epsilon")
    if eps <= 0:
        raise ValueError("group asset epsilon must be positive")
    layer_ids = data["layer_ids_zero_based"]
    if (not isinstance(layer_ids, list) or not layer_ids or any(type(x) is not int or x < 0 for x in layer_ids)
            or len(set(layer_ids)) != len(layer_ids)):
        raise ValueError("group asset layer_ids_zero_based must be a list of distinct non-negative integers")
    layers = data["layers"]
    if not isinstance(layers, Mapping) or set(layers) != {str(x) for x in layer_ids}:
        raise ValueError("group asset layers must hold exactly the layer_ids_zero_based entries")
    heads = {}
    for layer_id in layer_ids:
        lpath = f"group asset layers[{layer_id}]"
        layer = layers[str(layer_id)]
        _require_keys(layer, {"max_groups", "heads"}, set(), lpath)
        gmax = layer["max_groups"]
        if type(gmax) is not int or gmax not in GROUP_COUNT_RANGE:
            raise ValueError(f"{lpath}.max_groups must be an integer in 2..5")
        if not isinstance(layer["heads"], Mapping) or set(layer["heads"]) != {str(h) for h in range(num_query_heads)}:
            raise ValueError(f"{lpath}.heads must contain exactly zero-based indices 0..{num_query_heads - 1}")
        for head_id in range(num_query_heads):
            heads[layer_id, head_id] = _head(layer["heads"][str(head_id)], layer_id=layer_id, head_id=head_id,
                                             stored_gmax=gmax, path=f"{lpath}.heads[{head_id}]")
    return OALGroupAsset(
        model_name=str(data["model_name"]),
        layer_ids_zero_based=tuple(layer_ids),
        head_dim=HEAD_DIM,
        epsilon=eps,
        seq_len=int(data["seq_len"]),
        heads=heads,
        num_query_heads=num_query_heads,
    )


__all__ = ("OALGroupAsset", "GroupHeadRecord", "load_oal_group_asset", "active_packed_length",
           "expand_packed_lower_triangular", "FACTOR_SIZE")
