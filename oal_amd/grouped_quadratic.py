"""Public grouped quadratic attention API (``oal_attention``) on MI355X.

Mirrors the reference surface ``oal_attention/grouped_quadratic.py:277-397``:
the same arguments, validation rules and error types, the same factor ->
(c0, lam, Gam) expansion (kept in torch so autograd reaches the factor), the
same return conventions. ``execution="triton"`` and ``"auto"`` run the
hand-written gfx950 HIP kernels (there is no Triton here). ``"reference"`` -- in
the original a pure-torch evaluation in the working dtype on any device
(grouped_quadratic.py:332-355), which the caller's quality sessions use on GPU
tensors (qwen_lora_experiment/attention/grouped.py:125-152, 244-247) -- runs the
fp32 HIP kernels on q, k, v cast to float32 (the 1e-5 fp32 parity route). This
package ships no CPU compute path: CPU tensors raise under every execution.
"""

from __future__ import annotations

import math
from typing import Literal

import torch

from .hd_block_gemm_autograd import grouped_oal, grouped_oal_f64

_SUPPORTED_FLOATING_DTYPES = frozenset({torch.float16, torch.bfloat16, torch.float32, torch.float64})
_SUPPORTED_FACTOR_DTYPES = frozenset({torch.float32, torch.float64})
_SUPPORTED_OUTPUT_DTYPES = _SUPPORTED_FLOATING_DTYPES
_HIP_INPUT_DTYPES = frozenset({torch.float16, torch.bfloat16, torch.float32})


def _resolve_working_dtype(q_dtype: torch.dtype, factor_dtype: torch.dtype) -> torch.dtype:
    """grouped_quadratic.py:24-29."""
    promoted = torch.promote_types(q_dtype, factor_dtype)
    return torch.float64 if promoted == torch.float64 else torch.float32


def _validate_kernel_eps(kernel_eps: object, *, working_dtype: torch.dtype) -> float:
    """grouped_quadratic.py:32-51."""
    if isinstance(kernel_eps, bool) or not isinstance(kernel_eps, (int, float)):
        raise TypeError("kernel_eps must be a positive finite Python scalar")
    try:
        resolved = float(kernel_eps)
    except OverflowError:
        raise ValueError("kernel_eps must be finite") from None
    if not math.isfinite(resolved) or resolved <= 0.0:
        raise ValueError("kernel_eps must be finite and positive")
    info = torch.finfo(working_dtype)
    if resolved < info.tiny * info.eps or resolved > info.max:
        raise ValueError("kernel_eps must remain finite and positive in the computation dtype")
    return resolved


def _validate_output_dtype(output_dtype: object) -> None:
    if output_dtype is not None and (
        not isinstance(output_dtype, torch.dtype) or output_dtype not in _SUPPORTED_OUTPUT_DTYPES
    ):
        raise TypeError("output_dtype must be a supported floating torch.dtype")


def _infer_gmax(parameter_count: int) -> int:
    """grouped_quadratic.py:62-73: (G+1)(G+2)/2 -> G."""
    discriminant = 1 + 8 * parameter_count
    root = math.isqrt(discriminant)
    if root * root != discriminant or (root - 1) % 2 != 0:
        raise ValueError("factor last dimension must be a valid packed lower-triangular size")
    gmax = (root - 1) // 2 - 1
    if gmax < 1:
        raise ValueError("factor must reserve at least one dimension group")
    return gmax


def _validate_qkv(q: object, k: object, v: object):
    """grouped_quadratic.py:76-111."""
    if not all(isinstance(t, torch.Tensor) for t in (q, k, v)):
        raise TypeError("q, k, and v must be torch.Tensor objects")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must be rank-4 head-first tensors")
    if any(t.dtype not in _SUPPORTED_FLOATING_DTYPES for t in (q, k, v)):
        raise TypeError("q, k, and v must have floating-point dtypes")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, and v must have the same dtype")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k, and v must be on the same device")
    if q.shape[-1] != k.shape[-1]:
        raise ValueError("q and k must have the same feature dimension")
    if q.shape[0] != k.shape[0] or q.shape[0] != v.shape[0]:
        raise ValueError("q, k, and v must have the same batch size")
    if q.shape[2] != k.shape[2] or q.shape[2] != v.shape[2]:
        raise ValueError("q, k, and v must have the same sequence length")
    if k.shape[1] != v.shape[1]:
        raise ValueError("k and v must have the same KV head count")
    if q.shape[1] <= 0 or k.shape[1] <= 0:
        raise ValueError("q and k must have positive head counts")
    if any(dim <= 0 for dim in tuple(q.shape) + tuple(v.shape[-1:])):
        raise ValueError("q, k, and v dimensions must be positive")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError("query head count must be divisible by KV head count")
    return q, k, v


def _validate_factor(factor: object, *, query_heads: int, q_device: torch.device):
    """grouped_quadratic.py:114-133."""
    if not isinstance(factor, torch.Tensor):
        raise TypeError("factor must be a torch.Tensor")
    if factor.ndim not in (1, 2):
        raise ValueError("factor must have shape [P] or [Hq, P]")
    if factor.dtype not in _SUPPORTED_FACTOR_DTYPES:
        raise TypeError("factor must be a floating Tensor with dtype FP32 or FP64")
    if factor.device != q_device:
        raise ValueError("factor must be on the same device as q")
    if factor.shape[-1] <= 0:
        raise ValueError("factor must contain packed lower-triangular parameters")
    gmax = _infer_gmax(factor.shape[-1])
    if factor.ndim == 2 and factor.shape[0] != query_heads:
        raise ValueError("per-query-head factor first dimension must equal Hq")
    return factor, gmax


def _canonicalize_dim_groups(
    dim_groups: object, *, query_heads: int, head_dimension: int, gmax: int, q_device: torch.device
) -> torch.Tensor:
    """grouped_quadratic.py:136-181: ids in [0, Gmax) forming a continuous prefix per head."""
    if not isinstance(dim_groups, torch.Tensor):
        raise TypeError("dim_groups must be a torch.Tensor")
    if dim_groups.dtype not in {torch.int32, torch.int64}:
        raise TypeError("dim_groups must use torch.int32 or torch.int64")
    if dim_groups.device != q_device:
        raise ValueError("dim_groups must be on the same device as q")
    if dim_groups.ndim == 1:
        if dim_groups.shape[0] != head_dimension:
            raise ValueError("dim_groups last dimension must equal D")
        heads = dim_groups.unsqueeze(0).expand(query_heads, -1)
    elif dim_groups.ndim == 2:
        if dim_groups.shape[0] != query_heads:
            raise ValueError("dim_groups first dimension must equal query-head count Hq")
        if dim_groups.shape[1] != head_dimension:
            raise ValueError("dim_groups last dimension must equal D")
        heads = dim_groups
    else:
        raise ValueError("dim_groups must have shape [D] or [Hq, D]")
    if not bool(((heads >= 0) & (heads < gmax)).all()):
        raise ValueError("dim_groups IDs must satisfy 0 <= id < Gmax")
    host = heads.detach().to("cpu", torch.int64)
    for row in host:
        used = torch.unique(row, sorted=True)
        if used.numel() == 0 or not torch.equal(used, torch.arange(used.numel(), dtype=used.dtype)):
            raise ValueError("dim_groups IDs for every query head must form a continuous prefix")
    return dim_groups.to(torch.int32).contiguous()


def _expand_factor_coefficients(
    factor: torch.Tensor, *, query_heads: int, gmax: int, kernel_eps: float, working_dtype: torch.dtype
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Packed L -> (c0 = M00 + eps, lam = 2 M[0, 1:], Gam = M[1:, 1:]), M = L L^T.

    Same expansion as grouped_quadratic.py:184-218. M is formed as an
    elementwise product-sum, so M[i][j] and M[j][i] are the same floating-point
    sum and Gam is exactly symmetric (the HIP intra-chunk term relies on it).
    """
    fac = factor.unsqueeze(0) if factor.ndim == 1 else factor
    fac = fac.to(dtype=working_dtype)
    if fac.shape[0] == 1:
        fac = fac.expand(query_heads, -1)
    side = gmax + 1
    rows, cols = torch.tril_indices(side, side, device=factor.device)
    flat = torch.zeros((query_heads, side * side), dtype=working_dtype, device=factor.device)
    flat = flat.scatter(1, (rows * side + cols).unsqueeze(0).expand(query_heads, -1), fac)
    lower = flat.reshape(query_heads, side, side)
    matrix = (lower.unsqueeze(2) * lower.unsqueeze(1)).sum(dim=-1)
    constant = matrix[:, 0, 0] + torch.as_tensor(kernel_eps, dtype=working_dtype, device=factor.device)
    linear = 2.0 * matrix[:, 0, 1:]
    quadratic = matrix[:, 1:, 1:].contiguous()
    return constant, linear, quadratic


def _validate_public_options(*, causal, execution, output_dtype, return_unnormalized):
    """grouped_quadratic.py:221-243 (plus "hip" as an explicit execution name)."""
    if not isinstance(causal, bool):
        raise TypeError("causal must be a bool")
    if not causal:
        raise ValueError("grouped quadratic attention is causal-only; causal=False is no longer supported")
    if not isinstance(execution, str) or execution not in {"reference", "triton", "auto", "hip"}:
        raise ValueError("execution must be one of: reference, triton, auto, hip")
    _validate_output_dtype(output_dtype)
    if not isinstance(return_unnormalized, bool):
        raise TypeError("return_unnormalized must be a bool")
    return causal, execution


def oal_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dim_groups: torch.Tensor,
    factor: torch.Tensor,
    *,
    scale: float | None = None,
    kernel_eps: float = 1e-6,
    causal: bool = True,
    execution: Literal["reference", "triton", "auto", "hip"] = "auto",
    output_dtype: torch.dtype | None = None,
    return_unnormalized: bool = False,
):
    """Evaluate OAL's grouped PSD quadratic attention kernel on the HIP path.

    q [B, Hq, N, D], k/v [B, Hkv, N, D | DV] (D, DV <= 64), dim_groups [D] or
    [Hq, D] int32/int64, factor [P] or [Hq, P] packed lower-triangular (float32
    for the HIP executions; float32 or float64 for "reference", which evaluates
    in the working dtype). Returns out (v.dtype or output_dtype), or (out, num,
    den) with num [B, Hq, N, DV] and den [B, Hq, N, 1] in float32 (float64 for
    the float64 "reference" execution).
    """
    q, k, v = _validate_qkv(q, k, v)
    causal, execution = _validate_public_options(
        causal=causal, execution=execution, output_dtype=output_dtype, return_unnormalized=return_unnormalized
    )
    factor, gmax = _validate_factor(factor, query_heads=q.shape[1], q_device=q.device)
    working_dtype = _resolve_working_dtype(q.dtype, factor.dtype)
    resolved_eps = _validate_kernel_eps(kernel_eps, working_dtype=working_dtype)
    dim_groups = _canonicalize_dim_groups(
        dim_groups, query_heads=q.shape[1], head_dimension=q.shape[-1], gmax=gmax, q_device=q.device
    )
    if scale is None:
        resolved_scale = q.shape[-1] ** -0.5
    elif isinstance(scale, bool) or not isinstance(scale, (int, float)):
        raise TypeError("scale must be a finite Python scalar")
    else:
        try:
            resolved_scale = float(scale)
        except OverflowError:
            raise ValueError("scale must be finite") from None
        if not math.isfinite(resolved_scale):
            raise ValueError("scale must be finite")

    if q.device.type != "cuda" or torch.version.hip is None:
        if execution == "reference":
            raise RuntimeError(
                "execution='reference' runs the fp32 HIP kernels and requires ROCm device input; oal_amd "
                "ships no CPU compute path (the pure-torch formula is test infrastructure only)"
            )
        raise RuntimeError("grouped quadratic HIP execution requires ROCm device input")
    if execution == "reference":
        # the reference evaluates in the working dtype (:332-355): the fp32 HIP
        # kernels for FP32, the FP64 route (oal_f64.hip) for FP64
        if q.shape[-1] > 64 or v.shape[-1] > 64:
            raise ValueError("grouped quadratic HIP execution supports D<=64")
        q_work, k_work, v_work = (t.to(dtype=working_dtype) for t in (q, k, v))
        constant, linear, quadratic = _expand_factor_coefficients(
            factor, query_heads=q.shape[1], gmax=gmax, kernel_eps=resolved_eps, working_dtype=working_dtype
        )
        if working_dtype == torch.float64:
            output, numerator, denominator = grouped_oal_f64(
                q_work, k_work, v_work, dim_groups, constant, linear, quadratic, scale=resolved_scale
            )
        else:
            output, numerator, denominator = grouped_oal(
                q_work, k_work, v_work, dim_groups, constant, linear, quadratic, scale=resolved_scale, floor=0.0,
                precision="fp32",
            )
    else:
        if q.dtype not in _HIP_INPUT_DTYPES:
            raise TypeError("grouped quadratic HIP execution supports float16, bfloat16 and float32")
        if factor.dtype != torch.float32:
            raise TypeError("grouped quadratic HIP factor must use FP32")
        if q.shape[-1] > 64 or v.shape[-1] > 64:
            raise ValueError("grouped quadratic HIP execution supports D<=64")
        constant, linear, quadratic = _expand_factor_coefficients(
            factor, query_heads=q.shape[1], gmax=gmax, kernel_eps=resolved_eps, working_dtype=torch.float32
        )
        output, numerator, denominator = grouped_oal(
            q, k, v, dim_groups, constant, linear, quadratic, scale=resolved_scale, floor=0.0
        )

    if not (bool(torch.isfinite(numerator).all()) and bool(torch.isfinite(denominator).all())):
        raise RuntimeError("Grouped Quadratic result must be finite")
    if not bool((denominator > 0).all()):
        raise RuntimeError("Grouped Quadratic denominator must be finite and strictly positive")
    target = v.dtype if output_dtype is None else output_dtype
    if torch.finfo(target).bits > torch.finfo(output.dtype).bits:
        # a wider output than the kernel's storage dtype: normalize the fp32 num/den
        output = numerator / denominator
    output = output.to(dtype=target)
    if not bool(torch.isfinite(output).all()):
        raise RuntimeError("Grouped Quadratic normalized output must be finite")
    if return_unnormalized:
        return output, numerator, denominator
    return output


__all__ = ["oal_attention"]
