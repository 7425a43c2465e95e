"""Autograd boundary of the HIP operator.

Two ``torch.autograd.Function`` classes share the same HIP forward/VJP:

* :class:`_GroupedOALFunction` takes the grouped coefficients (c0, lam, Gam and
  dimension labels) that ``oal_attention`` and the HD adapters derive from the
  packed factor. Its gradients are (dq, dk, dv, dc0, dlam, dGam). Gam is a
  symmetric matrix parameter: dGam is the gradient of sum_{g,h} Gam_gh s_g s_h,
  i.e. the reference routing (pair (r, c), r >= c, to Gam[g(r), g(c)];
  ``grouped_reference.py:89-93``) with each off-diagonal gradient split evenly
  between [g][h] and [h][g]. Gradients that reach a factor L (Gam = L L^T) are
  identical under both conventions.
* :class:`_HDParallelBlockGemmFunction` keeps the reference contract of
  ``oal_attention/hd_block_gemm_autograd.py:85-204``:
  forward(q, k, v, a, b, c, scale, eps, layout, plan) -> (out, num, den) with
  logical per-dimension b [Hq, D] and per-pair c [Hq, D(D+1)/2]; backward
  returns 6 gradients + 4 ``None``, no double backward, gradients cast to the
  input dtypes (:333-347). It runs the same library with one group per
  dimension (labels = d, lam = b, Gam = symmetric fill of c, G = 64) in the
  plan's precision: ``bf16_tensorcore`` takes the matrix-core path, whose
  intra-chunk local score is then formed in feature form (phi_Q . phi_K^T on
  the matrix cores, as ``hd_block_gemm_runtime.py:530-540``); ``fp32_ieee``
  (or no plan) the fp32 kernels.

Both pad D and DV up to 64 with zeros (padding contributes nothing) and slice
the results back. :class:`_GroupedOALF64Function` is the grouped Function's
float64 counterpart (the FP64 route, ``oal_f64.hip``).
"""

from __future__ import annotations

from typing import Any

import torch

from . import _native

HEAD_DIM = _native.HEAD_DIM


def _pad_last(x: torch.Tensor, size: int = HEAD_DIM) -> torch.Tensor:
    if x.shape[-1] == size:
        return x.contiguous()
    if x.shape[-1] > size:
        raise ValueError(f"the HIP kernels support head and value dimensions up to {size}")
    return torch.nn.functional.pad(x, (0, size - x.shape[-1])).contiguous()


def _kernel_dtype(dtype: torch.dtype) -> torch.dtype:
    if dtype in (torch.float32, torch.bfloat16):
        return dtype
    if dtype == torch.float16:
        return torch.float32
    raise TypeError("HIP execution supports float16, bfloat16 and float32 q, k, v")


def pad_labels(labels: torch.Tensor, query_heads: int) -> torch.Tensor:
    """[D] or [Hq, D] integer labels -> contiguous int32 [Hq, 64] (pad dims -> group 0)."""
    lab = labels if labels.ndim == 2 else labels.unsqueeze(0).expand(query_heads, -1)
    lab = lab.to(torch.int32)
    if lab.shape[-1] < HEAD_DIM:
        lab = torch.nn.functional.pad(lab, (0, HEAD_DIM - lab.shape[-1]))
    return lab.contiguous()


class _GroupedOALFunction(torch.autograd.Function):
    """(q, k, v, c0, lam, gam, labels, scale, floor) -> (out, num, den).

    q, k, v must already be [B, H, N, 64] contiguous float32 or bfloat16 on one
    ROCm device; c0 [Hq], lam [Hq, G], gam [Hq, G, G] float32, gam symmetric.
    """

    @staticmethod
    def forward(ctx: Any, q, k, v, c0, lam, gam, labels, scale: float, floor: float, precision: str = "fp32"):
        ctx.set_materialize_grads(False)
        c0c, lamc, gamc = (t.detach().to(torch.float32).contiguous() for t in (c0, lam, gam))
        out, num, den, saved = _native.forward(
            q, k, v, labels, c0c, lamc, gamc, scale=scale, floor=floor, precision=precision
        )
        ctx.save_for_backward(q, k, v, c0c, lamc, gamc, labels, num, den, saved)
        ctx.scale = float(scale)
        ctx.floor = float(floor)
        ctx.precision = precision
        ctx.coef_dtypes = (c0.dtype, lam.dtype, gam.dtype)
        return out, num, den

    @staticmethod
    def backward(ctx: Any, dout, dnum, dden):
        if torch.is_grad_enabled():
            raise RuntimeError("the OAL HIP operator does not support double backward")
        q, k, v, c0, lam, gam, labels, num, den, saved = ctx.saved_tensors
        needs = ctx.needs_input_grad
        if dout is None and dnum is None and dden is None:
            return (None,) * 10
        dq, dk, dv, dc0, dlam, dgam = _native.backward(
            q, k, v, labels, c0, lam, gam, num, den, saved, dout, dnum, dden,
            scale=ctx.scale, floor=ctx.floor, precision=ctx.precision,
            need_q=needs[0], need_k=needs[1], need_v=needs[2], need_coef=any(needs[3:6]),
        )
        cd = ctx.coef_dtypes
        return (
            dq,
            dk,
            dv,
            dc0.to(cd[0]) if needs[3] else None,
            dlam.to(cd[1]) if needs[4] else None,
            dgam.to(cd[2]) if needs[5] else None,
            None,
            None,
            None,
            None,
        )


def grouped_oal(q, k, v, labels, c0, lam, gam, *, scale: float, floor: float, precision: str = "fp32"):
    """Differentiable grouped operator on [B, H, N, D<=64] tensors of any float dtype.

    ``precision`` "fp32" runs fp32 arithmetic throughout; "bf16" runs bf16
    operands with fp32 accumulation on the matrix cores (reference HD
    ``bf16_tensorcore``). Returns (out, num, den) with out in q's dtype,
    num [B, Hq, N, DV] and den [B, Hq, N, 1] in float32.
    """
    dv_orig = v.shape[-1]
    kd = _kernel_dtype(q.dtype)
    qp, kp, vp = (_pad_last(t.to(kd)) for t in (q, k, v))
    lab = pad_labels(labels, q.shape[1])
    out, num, den = _GroupedOALFunction.apply(
        qp, kp, vp, c0, lam, gam, lab, float(scale), float(floor), precision
    )
    if dv_orig != HEAD_DIM:
        out = out[..., :dv_orig]
        num = num[..., :dv_orig]
    return out.to(q.dtype), num, den


class _GroupedOALF64Function(torch.autograd.Function):
    """(q, k, v, c0, lam, gam, labels, scale) -> (out, num, den), all float64.

    The FP64 route (``oal_forward_f64`` / ``oal_backward_f64``): the working
    dtype of ``oal_attention(execution="reference")`` for float64 inputs, as the
    reference evaluates that execution in the working dtype
    (``oal_attention/grouped_quadratic.py:332-355``). q, k, v [B, H, N, 64]
    contiguous float64 on one ROCm device; labels int32 [Hq, 64]. dGam in the
    symmetric convention of :class:`_GroupedOALFunction`.
    """

    @staticmethod
    def forward(ctx: Any, q, k, v, c0, lam, gam, labels, scale: float):
        ctx.set_materialize_grads(False)
        c0c, lamc, gamc = (t.detach().to(torch.float64).contiguous() for t in (c0, lam, gam))
        out, num, den = _native.forward_f64(q, k, v, labels, c0c, lamc, gamc, scale=scale)
        ctx.save_for_backward(q, k, v, c0c, lamc, gamc, labels, num, den)
        ctx.scale = float(scale)
        ctx.coef_dtypes = (c0.dtype, lam.dtype, gam.dtype)
        return out, num, den

    @staticmethod
    def backward(ctx: Any, dout, dnum, dden):
        if torch.is_grad_enabled():
            raise RuntimeError("the OAL HIP operator does not support double backward")
        q, k, v, c0, lam, gam, labels, num, den = ctx.saved_tensors
        needs = ctx.needs_input_grad
        if dout is None and dnum is None and dden is None:
            return (None,) * 8
        dq, dk, dv, dc0, dlam, dgam = _native.backward_f64(
            q, k, v, labels, c0, lam, gam, num, den, dout, dnum, dden, scale=ctx.scale,
            need_q=needs[0], need_kv=needs[1] or needs[2], need_coef=any(needs[3:6]),
        )
        cd = ctx.coef_dtypes
        return (
            dq,
            dk if needs[1] else None,
            dv if needs[2] else None,
            dc0.to(cd[0]) if needs[3] else None,
            dlam.to(cd[1]) if needs[4] else None,
            dgam.to(cd[2]) if needs[5] else None,
            None,
            None,
        )


def grouped_oal_f64(q, k, v, labels, c0, lam, gam, *, scale: float):
    """The grouped operator in float64 throughout (the FP64 route): [B, H, N, D<=64]
    q, k, v, labels [D] or [Hq, D], grouped coefficients. Returns (out, num, den)
    in float64, num [B, Hq, N, DV], den [B, Hq, N, 1]."""
    dv_orig = v.shape[-1]
    qp, kp, vp = (_pad_last(t.to(torch.float64)) for t in (q, k, v))
    lab = pad_labels(labels, q.shape[1])
    out, num, den = _GroupedOALF64Function.apply(qp, kp, vp, c0, lam, gam, lab, float(scale))
    if dv_orig != HEAD_DIM:
        out = out[..., :dv_orig]
        num = num[..., :dv_orig]
    return out, num, den


def _pair_rows_cols(d: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    rows, cols = torch.tril_indices(d, d, device=device)
    return rows, cols


def logical_to_grouped(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, head_dim: int):
    """Logical (a [Hq], b [Hq, D], c [Hq, D(D+1)/2]) -> one group per dimension.

    labels = d, lam = b, Gam[r][c] = Gam[c][r] = c_p(r, c) (D padded to 64).
    """
    hq = a.shape[0]
    dev = a.device
    rows, cols = _pair_rows_cols(head_dim, dev)
    gam = torch.zeros((hq, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=dev)
    cf = c.to(torch.float32)
    gam[:, rows, cols] = cf
    gam[:, cols, rows] = cf
    lam = torch.zeros((hq, HEAD_DIM), dtype=torch.float32, device=dev)
    lam[:, :head_dim] = b.to(torch.float32)
    labels = torch.arange(HEAD_DIM, dtype=torch.int32, device=dev).unsqueeze(0).expand(hq, -1).contiguous()
    return a.to(torch.float32).contiguous(), lam.contiguous(), gam.contiguous(), labels


class _HDParallelBlockGemmFunction(torch.autograd.Function):
    """Reference-contract Function over logical coefficients (see module doc)."""

    @staticmethod
    def forward(ctx: Any, q, k, v, a, b, c, scale: float, eps: float, layout, plan):
        gradient_mask = tuple(bool(x) for x in ctx.needs_input_grad[:6])
        if (
            plan is not None
            and torch.is_grad_enabled()
            and tuple(plan.requested_gradient_mask) != gradient_mask
        ):
            raise ValueError("plan gradient mask must exactly match the six tensor inputs")
        ctx.set_materialize_grads(False)
        d, dv = q.shape[-1], v.shape[-1]
        kd = _kernel_dtype(q.dtype)
        qp, kp, vp = (_pad_last(t.detach().to(kd)) for t in (q, k, v))
        c0g, lam, gam, labels = logical_to_grouped(a.detach(), b.detach(), c.detach(), d)
        precision = _plan_kernel_precision(plan)
        out, num, den, saved = _native.forward(qp, kp, vp, labels, c0g, lam, gam, scale=scale, floor=eps,
                                               precision=precision)
        if plan is not None and getattr(plan, "require_positive_denominator", True):
            _require_positive_denominator(den)
        ctx.save_for_backward(qp, kp, vp, c0g, lam, gam, labels, num, den, saved)
        ctx.meta = (float(scale), float(eps), d, dv, gradient_mask, precision)
        ctx.input_dtypes = tuple(t.dtype for t in (q, k, v, a, b, c))
        out = out[..., :dv].to(q.dtype)
        return out, num[..., :dv], den

    @staticmethod
    def backward(ctx: Any, dout, dnum, dden):
        if torch.is_grad_enabled():
            raise RuntimeError("HD Block-GEMM does not support double backward")
        qp, kp, vp, c0g, lam, gam, labels, num, den, saved = ctx.saved_tensors
        scale, eps, d, dv, mask, precision = ctx.meta
        if dout is None and dnum is None and dden is None:
            return (None,) * 10
        if dout is not None:
            dout = _pad_last(dout)
        if dnum is not None:
            dnum = _pad_last(dnum.to(torch.float32))
        need_q, need_k, need_v, need_a, need_b, need_c = mask
        dq, dk, dvv, dc0, dlam, dgam = _native.backward(
            qp, kp, vp, labels, c0g, lam, gam, num, den, saved, dout, dnum, dden,
            scale=scale, floor=eps, need_q=need_q, need_k=need_k, need_v=need_v,
            need_coef=need_a or need_b or need_c, precision=precision,
        )
        rows, cols = _pair_rows_cols(d, qp.device)
        grads = [
            dq[..., :d] if need_q else None,
            dk[..., :d] if need_k else None,
            dvv[..., :dv] if need_v else None,
            dc0 if need_a else None,
            dlam[:, :d] if need_b else None,
            torch.where(rows == cols, dgam[:, rows, cols], dgam[:, rows, cols] + dgam[:, cols, rows])
            if need_c
            else None,
        ]
        out = [g.to(dt) if g is not None else None for g, dt in zip(grads, ctx.input_dtypes)]
        return (*out, None, None, None, None)


def _plan_kernel_precision(plan) -> str:
    """Planner precision -> kernel arithmetic ("bf16" on the matrix cores for
    ``bf16_tensorcore``, else "fp32"; no plan: "fp32")."""
    if plan is not None and getattr(plan, "precision", "fp32_ieee") == "bf16_tensorcore":
        return "bf16"
    return "fp32"


def _require_positive_denominator(den: torch.Tensor) -> None:
    """Raise unless every denominator is finite and positive (two host syncs).

    Mirrors ``hd_block_gemm_runtime.py:392-408``.
    """
    lo, hi = torch.aminmax(den.detach())
    if not (bool(torch.isfinite(lo)) and bool(torch.isfinite(hi))):
        raise RuntimeError("HD Block-GEMM denominator must be finite")
    if float(lo) <= 0.0:
        raise RuntimeError("HD Block-GEMM denominator must be strictly positive")


def _hd_parallel_block_gemm_autograd(q, k, v, a, b, c, *, scale, eps, layout, plan):
    return _HDParallelBlockGemmFunction.apply(q, k, v, a, b, c, scale, eps, layout, plan)


def _hd_parallel_block_gemm(q, k, v, a, b, c, *, scale, eps, layout, plan):
    with torch.no_grad():
        return _HDParallelBlockGemmFunction.apply(q, k, v, a, b, c, scale, eps, layout, plan)


__all__: tuple[str, ...] = ()
