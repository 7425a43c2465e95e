"""The C-ABI entry points as registered torch operators.

The reference registers its native GEMM as a schema'd torch operator
(``hd_cublas_compat::bmm_fp32``, ``oal_attention/csrc/hd_cublas_compat.cpp:243-251``).
The HIP library's forward and VJP are registered here the same way, so that
code above the binding can be traced (fake tensors, ``make_fx``,
``torch.compile``) and checked with ``torch.library.opcheck``:

* ``oal_amd::forward(q, k, v, labels, c0, lam, gam, scale, floor, precision)
  -> (out, num, den, saved)``: ``oal_forward`` (``include/oal_amd.h``); saved is
  the opaque uint8 state the VJP reads, sized by ``oal_forward_saved_bytes`` and
  allocated zero-filled (its padding is then defined; one memset per call that
  the autograd Function path does not pay).
* ``oal_amd::backward(q, k, v, labels, c0, lam, gam, num, den, saved, dout?,
  dnum?, dden?, scale, floor, need_q, need_k, need_v, need_coef, precision)
  -> (dq, dk, dv, dc0, dlam, dgam)``: ``oal_backward``. A gradient that is not
  requested comes back as an empty (zero-element) tensor, since an operator's
  outputs are tensors; ``grouped_oal_op`` turns those into ``None``.

Both run on the HIP device only (``device_types="cuda"``, the ROCm device
type); their fake kernels give the output metadata without touching a device.
Autograd is registered on ``oal_amd::forward`` (its VJP calls
``oal_amd::backward``), with the autograd Function's conventions: no double
backward, coefficient gradients cast to the coefficients' dtypes by the
caller. ``grouped_oal_op`` is :func:`oal_amd.hd_block_gemm_autograd.grouped_oal`
through these operators.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _native

HEAD_DIM = _native.HEAD_DIM


def _saved_bytes(q: Tensor, k: Tensor, lam: Tensor, precision: str) -> int:
    b, hq, n, _ = q.shape
    lib = _native.load_library()
    nbytes = lib.oal_forward_saved_bytes(b, hq, k.shape[1], n, lam.shape[1], _native._dtype_code(q.dtype),
                                         _native._precision_code(precision))
    if nbytes == 0:
        raise RuntimeError("oal_forward_saved_bytes: " + lib.oal_last_error().decode("utf-8", "replace"))
    return int(nbytes)


@torch.library.custom_op("oal_amd::forward", mutates_args=(), device_types="cuda")
def oal_forward(q: Tensor, k: Tensor, v: Tensor, labels: Tensor, c0: Tensor, lam: Tensor, gam: Tensor,
                scale: float, floor: float, precision: str) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    # the saved state zero-filled: the kernels leave its alignment gaps and
    # padding tails unwritten, and an operator's outputs must be fully defined
    # (tracing compares them bytewise). The autograd Function path skips this fill.
    out, num, den, saved = _native.forward(q, k, v, labels, c0, lam, gam, scale=scale, floor=floor,
                                           precision=precision, zero_saved=True)
    return out, num, den, saved


@oal_forward.register_fake
def _oal_forward_fake(q, k, v, labels, c0, lam, gam, scale, floor, precision):
    _native.check_forward_args(q, k, v, labels, c0, lam, gam)
    b, hq, n, d = q.shape
    return (
        q.new_empty((b, hq, n, d)),
        q.new_empty((b, hq, n, d), dtype=torch.float32),
        q.new_empty((b, hq, n, 1), dtype=torch.float32),
        q.new_empty((_saved_bytes(q, k, lam, precision),), dtype=torch.uint8),
    )


@torch.library.custom_op("oal_amd::backward", mutates_args=(), device_types="cuda")
def oal_backward(q: Tensor, k: Tensor, v: Tensor, labels: Tensor, c0: Tensor, lam: Tensor, gam: Tensor,
                 num: Tensor, den: Tensor, saved: Tensor, dout: Optional[Tensor], dnum: Optional[Tensor],
                 dden: Optional[Tensor], scale: float, floor: float, need_q: bool, need_k: bool, need_v: bool,
                 need_coef: bool, precision: str) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    grads = _native.backward(q, k, v, labels, c0, lam, gam, num, den, saved, dout, dnum, dden, scale=scale,
                             floor=floor, need_q=need_q, need_k=need_k, need_v=need_v, need_coef=need_coef,
                             precision=precision)
    like = (q, k, v, c0, lam, gam)
    return tuple(g if g is not None else t.new_empty((0,)) for g, t in zip(grads, like))


@oal_backward.register_fake
def _oal_backward_fake(q, k, v, labels, c0, lam, gam, num, den, saved, dout, dnum, dden, scale, floor, need_q,
                       need_k, need_v, need_coef, precision):
    _native.check_forward_args(q, k, v, labels, c0, lam, gam)
    wants = (need_q, need_k, need_v, need_coef, need_coef, need_coef)
    like = (q, k, v, c0, lam, gam)
    return tuple(t.new_empty(t.shape) if want else t.new_empty((0,)) for t, want in zip(like, wants))


def _forward_setup_context(ctx, inputs, output):
    q, k, v, labels, c0, lam, gam, scale, floor, precision = inputs
    _, num, den, saved = output
    ctx.save_for_backward(q, k, v, labels, c0, lam, gam, num, den, saved)
    ctx.scale, ctx.floor, ctx.precision = float(scale), float(floor), precision
    ctx.set_materialize_grads(False)


def _forward_backward(ctx, dout, dnum, dden, dsaved):
    q, k, v, labels, c0, lam, gam, num, den, saved = ctx.saved_tensors
    needs = ctx.needs_input_grad
    if dout is None and dnum is None and dden is None:
        return (None,) * 10
    need_coef = any(needs[4:7])
    dq, dk, dv, dc0, dlam, dgam = oal_backward(
        q, k, v, labels, c0, lam, gam, num, den, saved, dout, dnum, dden, ctx.scale, ctx.floor,
        bool(needs[0]), bool(needs[1] or needs[2]), bool(needs[1] or needs[2]), need_coef, ctx.precision)
    return (dq if needs[0] else None, dk if needs[1] else None, dv if needs[2] else None, None,
            dc0 if needs[4] else None, dlam if needs[5] else None, dgam if needs[6] else None, None, None, None)


oal_forward.register_autograd(_forward_backward, setup_context=_forward_setup_context)


def grouped_oal_op(q, k, v, labels, c0, lam, gam, *, scale: float, floor: float, precision: str = "fp32"):
    """:func:`oal_amd.hd_block_gemm_autograd.grouped_oal` through the registered
    operators: [B, H, N, D<=64] q, k, v of any float dtype, labels [D] or
    [Hq, D], grouped coefficients (c0, lam, gam). Returns (out, num, den)."""
    from .hd_block_gemm_autograd import _kernel_dtype, _pad_last, pad_labels

    dv_orig = v.shape[-1]
    kd = _kernel_dtype(q.dtype)
    qp, kp, vp = (_pad_last(t.to(kd)) for t in (q, k, v))
    lab = pad_labels(labels, q.shape[1])
    c0c, lamc, gamc = (t.to(torch.float32).contiguous() for t in (c0, lam, gam))
    out, num, den, _ = oal_forward(qp, kp, vp, lab, c0c, lamc, gamc, float(scale), float(floor), precision)
    if dv_orig != HEAD_DIM:
        out = out[..., :dv_orig]
        num = num[..., :dv_orig]
    return out.to(q.dtype), num, den
