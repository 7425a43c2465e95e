"""OAL grouped coefficients for the causal HD attention API.

Same surface as ``oal_attention/hd_block_gemm_adapters.py:120-415``:
``prepare_grouped_hd_block_gemm`` freezes geometry, groups and plan once;
``run_prepared_grouped_hd_block_gemm`` expands the live factor per call (in
torch, so autograd reaches the factor) and runs the HIP operator;
``grouped_causal_attention`` does both. Callers (e.g. the reference's
``qwen_lora_experiment/attention/hd_runtime.py:200-224``) can resolve these
names unchanged.

Difference from the reference: the reference routes the factor through the
logical per-pair coefficients (a, b, c) and its cuBLAS feature GEMMs; here the
prepared run keeps the grouped form (c0, lam, Gam, labels), which the HIP
intra-chunk term evaluates in O(D + G^2) per token pair. Gradients reach the
factor through the same expansion.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from numbers import Real

import torch

from .grouped_quadratic import (
    _canonicalize_dim_groups,
    _expand_factor_coefficients,
    _resolve_working_dtype,
    _validate_factor,
    _validate_kernel_eps,
    _validate_qkv,
)
from .hd_block_gemm import HDParallelBlockPlan, build_hd_block_gemm_plan, canonical_pair_layout
from .hd_block_gemm_autograd import _require_positive_denominator, grouped_oal

_POSITIVE_FP32_FLOOR = torch.finfo(torch.float32).tiny * torch.finfo(torch.float32).eps


def _requested_gradient_mask(q, k, v, *, coefficient_source_requires_grad: bool):
    """hd_block_gemm_adapters.py:27-43."""
    live = torch.is_grad_enabled()
    coef = live and coefficient_source_requires_grad
    return (live and q.requires_grad, live and k.requires_grad, live and v.requires_grad, coef, coef, coef)


def _resolve_scale(scale: float | None, head_dimension: int) -> float:
    if scale is None:
        return head_dimension**-0.5
    if isinstance(scale, bool) or not isinstance(scale, Real):
        raise TypeError("scale must be a finite real scalar or None")
    resolved = float(scale)
    if not math.isfinite(resolved):
        raise ValueError("scale must be finite")
    return resolved


def kernel_precision(plan_precision: str) -> str:
    """Planner precision -> kernel arithmetic.

    ``bf16_tensorcore`` (bf16 operands, fp32 accumulation on the matrix cores;
    reference ``hd_block_gemm.py:132-153``) runs the gfx950 MFMA kernels;
    ``fp32_ieee`` runs the fp32 kernels.
    """
    return "bf16" if plan_precision == "bf16_tensorcore" else "fp32"


def _expand_factor_coefficients_tensorcore(factor, *, query_heads: int, gmax: int, kernel_eps: float):
    """FP32 pointwise PSD expansion (hd_block_gemm_adapters.py:57-95)."""
    return _expand_factor_coefficients(
        factor, query_heads=query_heads, gmax=gmax, kernel_eps=kernel_eps, working_dtype=torch.float32
    )


@dataclass(frozen=True)
class _PreparedGroupedHdBlockGemm:
    """Immutable structural state for repeated grouped invocations."""

    plan: HDParallelBlockPlan
    groups: torch.Tensor
    gmax: int
    scale: float
    kernel_eps: float
    normalization_floor: float


def prepare_grouped_hd_block_gemm(
    q, k, v, dim_groups, factor, *, scale=None, kernel_eps=1e-6, token_block=128, feature_wave_blocks=None,
    memory_budget_bytes=None, model_residency_bytes=0, precision="fp32_ieee",
    require_positive_denominator=True, **options,
) -> _PreparedGroupedHdBlockGemm:
    """Freeze grouped geometry once (hd_block_gemm_adapters.py:120-238).

    Extra selector keywords of the reference (key_feature_impl, backward_schedule,
    ...) are accepted and recorded on the plan.
    """
    q, k, v = _validate_qkv(q, k, v)
    factor, gmax = _validate_factor(factor, query_heads=q.shape[1], q_device=q.device)
    working = _resolve_working_dtype(q.dtype, factor.dtype)
    if working != torch.float32:
        raise TypeError("private grouped candidate currently requires FP32 working precision")
    eps = _validate_kernel_eps(kernel_eps, working_dtype=working)
    groups = _canonicalize_dim_groups(
        dim_groups, query_heads=q.shape[1], head_dimension=q.shape[-1], gmax=gmax, q_device=q.device
    )
    mask = _requested_gradient_mask(q, k, v, coefficient_source_requires_grad=factor.requires_grad)
    plan = build_hd_block_gemm_plan(
        q, k, v, token_block=token_block, feature_wave_blocks=feature_wave_blocks, precision=precision,
        requested_gradient_mask=mask, memory_budget_bytes=memory_budget_bytes,
        model_residency_bytes=model_residency_bytes,
        require_positive_denominator=require_positive_denominator, **options,
    )
    full = (groups.unsqueeze(0).expand(q.shape[1], -1) if groups.ndim == 1 else groups).detach().clone()
    return _PreparedGroupedHdBlockGemm(
        plan=plan,
        groups=full,
        gmax=gmax,
        scale=_resolve_scale(scale, q.shape[-1]),
        kernel_eps=eps,
        normalization_floor=_POSITIVE_FP32_FLOOR,
    )


def run_prepared_grouped_hd_block_gemm(prepared, q, k, v, factor):
    """One live invocation against a preparation (hd_block_gemm_adapters.py:241-312)."""
    if not isinstance(prepared, _PreparedGroupedHdBlockGemm):
        raise TypeError("prepared must be an explicit grouped HD Block-GEMM preparation")
    q, k, v = _validate_qkv(q, k, v)
    factor, gmax = _validate_factor(factor, query_heads=q.shape[1], q_device=q.device)
    if gmax != prepared.gmax:
        raise ValueError("factor group geometry does not match the preparation")
    if _resolve_working_dtype(q.dtype, factor.dtype) != torch.float32:
        raise TypeError("private grouped candidate currently requires FP32 working precision")
    mask = _requested_gradient_mask(q, k, v, coefficient_source_requires_grad=factor.requires_grad)
    if mask != prepared.plan.requested_gradient_mask:
        raise ValueError("live gradient mode does not match the preparation")
    plan = prepared.plan
    if (q.shape[0], q.shape[1], k.shape[1], q.shape[2], q.shape[3], v.shape[3]) != plan.geometry:
        raise ValueError("q, k, v geometry does not match the preparation")
    a, lam, gam = _expand_factor_coefficients_tensorcore(
        factor, query_heads=plan.query_heads, gmax=prepared.gmax, kernel_eps=prepared.kernel_eps
    )
    out, num, den = grouped_oal(
        q, k, v, prepared.groups, a, lam, gam, scale=prepared.scale, floor=prepared.normalization_floor,
        precision=kernel_precision(plan.precision),
    )
    if plan.require_positive_denominator:
        _require_positive_denominator(den)
    return out, num, den


def grouped_causal_attention(q, k, v, dim_groups, factor, **kwargs):
    """Prepare and run one grouped causal invocation (hd_block_gemm_adapters.py:347-415)."""
    prepared = prepare_grouped_hd_block_gemm(q, k, v, dim_groups, factor, **kwargs)
    return run_prepared_grouped_hd_block_gemm(prepared, q, k, v, factor)


_grouped_hd_block_gemm_forward = grouped_causal_attention
_prepare_grouped_hd_block_gemm = prepare_grouped_hd_block_gemm
_run_prepared_grouped_hd_block_gemm = run_prepared_grouped_hd_block_gemm

__all__ = (
    "grouped_causal_attention",
    "prepare_grouped_hd_block_gemm",
    "run_prepared_grouped_hd_block_gemm",
)
