"""Reference-quality execution sessions and the N=128 alignment check of the grouped layers.

Mirrors the quality-evaluation helpers of the reference adapter module
(qwen_lora_experiment/attention/grouped.py:261-450):

* ``grouped_quadratic_reference_session(model, expected_layer_ids=...)``
  (grouped.py:261-313) switches the listed OAL layers from the fast execution
  ("triton") to the reference-quality execution ("reference") for the duration
  of a ``with`` block and always switches them back, rejecting a layer set that
  does not match the model's OAL layers or an adapter that is not in the fast
  mode when the session starts;
* ``grouped_quadratic_reference_quality_session`` (:316-324), its alias;
* ``grouped_quadratic_reference_alignment(parameter_bank=..., layer_id=...,
  device=..., seed=...)`` (:327-425): a no-grad guard that runs one layer's
  groups and factor on seeded N=128 bf16 q, k, v in both executions and
  requires ``allclose(atol=0.03, rtol=0.03)``, returning the evidence record
  ``grouped_reference_alignment_v1``;
* ``grouped_quadratic_reference_quality_alignment`` (:428-441), the alias that
  relabels the record ``grouped_piqa_reference_alignment_v1``.

In the reference the "reference" execution is a pure-torch restatement of the
operator and "triton" the CUDA kernels. Here both run in liboal_amd.so on the
device: "triton" is the bf16 matrix-core path (precision ``bf16_tensorcore``)
and "reference" the fp32 kernels (precision ``fp32_ieee``, which hold rel-L2
1e-5 against an fp64/fp32 CPU evaluation of grouped_reference.py). There is no
torch or CPU formula of the operator in this package; without the built
library both executions raise.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from typing import Iterator, Sequence

import torch
from torch import nn

from .hd_block_gemm_adapters import prepare_grouped_hd_block_gemm, run_prepared_grouped_hd_block_gemm

ALIGNMENT_SEQUENCE_LENGTH = 128
ALIGNMENT_ATOL = 0.03
ALIGNMENT_RTOL = 0.03


class GroupedQuadraticAttentionError(RuntimeError):
    """Raised when a grouped OAL layer or session rejects a call (grouped.py:29-30)."""


def _context(layer_id: int) -> str:
    return f"grouped quadratic operator layer={layer_id}"


@dataclass(frozen=True)
class ModelGeometry:
    """The head geometry the alignment draws its q, k, v with."""

    num_query_heads: int
    num_kv_heads: int
    head_dim: int


class OALParameterBank:
    """Per-layer dim groups, packed factors and kernel epsilon of a model or asset.

    The read interface of the reference's KernelParameterBank used by the
    alignment (kernel_parameters.py:52-258): ``geometry``,
    ``dim_groups_for_layer``, ``packed_grouped_factor_for_layer`` and
    ``grouped_kernel_epsilon_for_runtime``.
    """

    def __init__(self, geometry: ModelGeometry, groups: dict, factors: dict, epsilon: float):
        self.geometry = geometry
        self._groups = groups
        self._factors = factors
        self._epsilon = float(epsilon)

    @classmethod
    def from_model(cls, model: nn.Module) -> "OALParameterBank":
        """The live groups and factors of every OAL layer of a QwenOALModel."""
        cfg = model.cfg
        layers = _layers(model)
        adapters = {i: a for i, a in ((i, _adapter(layer)) for i, layer in enumerate(layers)) if a is not None}
        eps = {float(a.kernel_eps) for a in adapters.values()}
        if len(eps) != 1:
            raise ValueError("the model's OAL layers do not share one kernel epsilon")
        return cls(ModelGeometry(cfg.num_heads, cfg.num_kv_heads, cfg.head_dim),
                   {i: a.dim_groups for i, a in adapters.items()},
                   {i: a.factor for i, a in adapters.items()}, eps.pop())

    @classmethod
    def from_asset(cls, asset, *, num_kv_heads: int = 2) -> "OALParameterBank":
        """The groups and factors of an :class:`oal_amd.group_assets.OALGroupAsset`."""
        layers = asset.layer_ids_zero_based
        return cls(ModelGeometry(asset.num_query_heads, num_kv_heads, asset.head_dim),
                   {i: asset.dim_groups_for_layer(i) for i in layers},
                   {i: asset.packed_grouped_factor_for_layer(i) for i in layers}, asset.epsilon)

    def active_kernel_layer_ids(self) -> tuple:
        return tuple(sorted(self._groups))

    def dim_groups_for_layer(self, layer_id: int) -> torch.Tensor:
        self._require(layer_id)
        return self._groups[layer_id].detach()

    def packed_grouped_factor_for_layer(self, layer_id: int) -> torch.Tensor:
        self._require(layer_id)
        return self._factors[layer_id].detach()

    def grouped_kernel_epsilon_for_runtime(self) -> float:
        return self._epsilon

    def _require(self, layer_id: int) -> None:
        if layer_id not in self._groups:
            raise KeyError(f"layer {layer_id} has no OAL parameters (layers {list(self.active_kernel_layer_ids())})")


def _layers(model: nn.Module):
    layers = getattr(model, "layers", None)
    if not isinstance(layers, nn.ModuleList):
        layers = getattr(getattr(model, "model", None), "layers", None)
    return layers


def _adapter(layer: nn.Module):
    from .qwen_oal import OALAttention

    for name in ("attn", "self_attn"):
        a = getattr(layer, name, None)
        if isinstance(a, OALAttention):
            return a
    return None


@contextmanager
def grouped_quadratic_reference_session(model: nn.Module, *, expected_layer_ids: Sequence[int]) -> Iterator[None]:
    """Run the model's OAL layers on the reference-quality (fp32) kernels inside the block.

    ``expected_layer_ids`` must be the sorted, unique ids of exactly the layers
    holding an OAL attention; every one of them must be in the fast execution
    when the session starts, and all are restored to it when the block returns
    or raises (grouped.py:261-313).
    """
    if not isinstance(model, nn.Module):
        raise TypeError("grouped reference session requires an nn.Module model")
    if isinstance(expected_layer_ids, (str, bytes)):
        raise TypeError("grouped reference layer IDs must be a sequence of integers")
    layer_ids = tuple(expected_layer_ids)
    if (not layer_ids or any(type(i) is not int or i < 0 for i in layer_ids)
            or layer_ids != tuple(sorted(set(layer_ids)))):
        raise ValueError("grouped reference layer IDs must be sorted unique non-negative integers")
    layers = _layers(model)
    if not isinstance(layers, nn.ModuleList):
        raise GroupedQuadraticAttentionError("grouped reference session cannot inspect Qwen layers")
    actual = tuple(i for i, layer in enumerate(layers) if _adapter(layer) is not None)
    if actual != layer_ids:
        raise GroupedQuadraticAttentionError(
            "grouped reference session adapters do not match the frozen replacement layers")
    adapters = tuple(_adapter(layers[i]) for i in layer_ids)
    if any(a._grouped_execution != "triton" for a in adapters):
        raise GroupedQuadraticAttentionError("grouped reference session requires adapters to begin in Triton mode")
    for a in adapters:
        a._grouped_execution = "reference"
    try:
        yield
    finally:
        for a in adapters:
            a._grouped_execution = "triton"


@contextmanager
def grouped_quadratic_reference_quality_session(model: nn.Module, *,
                                                expected_layer_ids: Sequence[int]) -> Iterator[None]:
    """Alias of :func:`grouped_quadratic_reference_session` (grouped.py:316-324)."""
    with grouped_quadratic_reference_session(model, expected_layer_ids=expected_layer_ids):
        yield


def _layer_attention(q, k, v, bank, layer_id: int, precision: str) -> torch.Tensor:
    groups = bank.dim_groups_for_layer(layer_id).to(device=q.device, dtype=torch.int32)
    factor = bank.packed_grouped_factor_for_layer(layer_id).to(device=q.device, dtype=torch.float32)
    prepared = prepare_grouped_hd_block_gemm(
        q, k, v, groups, factor, scale=q.shape[-1] ** -0.5,
        kernel_eps=bank.grouped_kernel_epsilon_for_runtime(), precision=precision,
    )
    out, _, _ = run_prepared_grouped_hd_block_gemm(prepared, q, k, v, factor)
    return out


def grouped_quadratic_reference_alignment(*, parameter_bank, layer_id: int, device, seed: int) -> dict:
    """Check one layer's fast execution against its reference-quality execution at N=128.

    q ~ N(0, 1) [1, Hq, 128, 64], then k and v [1, Hkv, 128, 64], drawn in that
    order from a generator on ``device`` seeded with ``seed`` and rounded to
    bf16 (grouped.py:327-392). Both executions run without autograd; the record
    reports the max and mean absolute difference of the outputs. Raises
    GroupedQuadraticAttentionError on a non-finite output or when
    ``allclose(atol=0.03, rtol=0.03)`` fails.
    """
    if type(seed) is not int:
        raise TypeError("grouped reference alignment seed must be an integer")
    target = torch.device(device)
    geo = parameter_bank.geometry
    n = ALIGNMENT_SEQUENCE_LENGTH
    gen = torch.Generator(device=target)
    gen.manual_seed(seed)

    def draw(heads):
        return torch.randn((1, heads, n, geo.head_dim), device=target, dtype=torch.float32,
                           generator=gen).to(torch.bfloat16).contiguous()

    q = draw(geo.num_query_heads)
    k = draw(geo.num_kv_heads)
    v = draw(geo.num_kv_heads)
    with torch.inference_mode():
        reference = _layer_attention(q, k, v, parameter_bank, layer_id, "fp32_ieee")
        fast = _layer_attention(q, k, v, parameter_bank, layer_id, "bf16_tensorcore")
    if not bool(torch.isfinite(reference).all()) or not bool(torch.isfinite(fast).all()):
        raise GroupedQuadraticAttentionError(_context(layer_id) + ": grouped reference alignment produced non-finite output")
    difference = (reference.float() - fast.float()).abs()
    maximum = float(difference.max().item()) if difference.numel() else 0.0
    mean = float(difference.mean().item()) if difference.numel() else 0.0
    within = bool(torch.allclose(reference.float(), fast.float(), atol=ALIGNMENT_ATOL, rtol=ALIGNMENT_RTOL))
    if not within:
        raise GroupedQuadraticAttentionError(
            _context(layer_id) + ": grouped N=128 reference-to-Triton alignment exceeded tolerance")
    return {
        "schema": "grouped_reference_alignment_v1",
        "sequence_length": n,
        "layer_id": layer_id,
        "seed": seed,
        "atol": ALIGNMENT_ATOL,
        "rtol": ALIGNMENT_RTOL,
        "max_abs_error": maximum,
        "mean_abs_error": mean,
        "within_tolerance": within,
    }


def grouped_quadratic_reference_quality_alignment(*, parameter_bank, layer_id: int, device, seed: int) -> dict:
    """Alias of :func:`grouped_quadratic_reference_alignment` with the record relabelled
    ``grouped_piqa_reference_alignment_v1`` (grouped.py:428-441)."""
    evidence = grouped_quadratic_reference_alignment(parameter_bank=parameter_bank, layer_id=layer_id,
                                                     device=device, seed=seed)
    evidence["schema"] = "grouped_piqa_reference_alignment_v1"
    return evidence


__all__ = (
    "GroupedQuadraticAttentionError", "ModelGeometry", "OALParameterBank",
    "grouped_quadratic_reference_session", "grouped_quadratic_reference_quality_session",
    "grouped_quadratic_reference_alignment", "grouped_quadratic_reference_quality_alignment",
)
