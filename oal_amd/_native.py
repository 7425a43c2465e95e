"""ctypes binding of liboal_amd.so (the C ABI declared in include/oal_amd.h).

PyTorch supplies device memory and the current HIP stream; every byte of the
operator's arithmetic runs in the HIP kernels behind this library. There is no
fallback: if the library is missing or the tensors are not on a ROCm device,
the call raises.

Each call sits in a ``torch.profiler.record_function`` range
("oal_amd::forward", "oal_amd::backward"), and the library brackets its own
launches with roctx ranges, as the reference brackets its stages
(``oal_attention/hd_block_gemm_profiling.py:195-226``).
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_NAME = "liboal_amd.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)
_LOCK = threading.Lock()
_LIB = None

DTYPE_F32 = 0
DTYPE_BF16 = 1
PRECISION_FP32 = 0
PRECISION_BF16 = 1
HEAD_DIM = 64

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

_SIGNATURES = {
    "oal_abi_version": ([], _i),
    "oal_last_error": ([], ctypes.c_char_p),
    "oal_profile_enable": ([_i], _i),
    "oal_profile_collect": ([ctypes.c_char_p, _sz], _i),
    "oal_feature_count": ([], _i),
    "oal_feature_stride": ([], _i),
    "oal_chunk_size": ([], _i),
    "oal_forward_saved_bytes": ([_i, _i, _i, _i, _i, _i, _i], _sz),
    "oal_backward_workspace_bytes": ([_i, _i, _i, _i, _i, _i, _i], _sz),
    "oal_forward": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _f, _vp, _vp, _vp, _vp, _vp],
        _i,
    ),
    "oal_backward": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _f, _vp, _vp, _vp, _vp, _vp, _vp,
         _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
        _i,
    ),
    "oal_backward_noalloc": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _f, _vp, _vp, _vp, _vp, _vp, _vp,
         _vp, _vp, _vp, _vp, _vp, _vp, _vp],
        _i,
    ),
    "oal_selftest": ([_vp, _vp], _i),
    "oal_forward_f64": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_double, _vp, _vp, _vp, _vp],
        _i,
    ),
    "oal_backward_f64_workspace_bytes": ([_i, _i, _i, _i, _i], _sz),
    "oal_backward_f64": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_double, _vp, _vp, _vp, _vp, _vp, _vp,
         _vp, _vp, _vp, _vp, _vp, _vp, _vp],
        _i,
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def library_path() -> str:
    return _LIB_PATH


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load liboal_amd.so once; raise if it has not been built."""
    global _LIB
    with _LOCK:
        if _LIB is not None and path is None:
            return _LIB
        target = path or _LIB_PATH
        if not os.path.exists(target):
            raise RuntimeError(
                f"{_LIB_NAME} is not built ({target}); run __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950) before using oal_amd"
            )
        lib = ctypes.CDLL(target)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.oal_abi_version() != 2:
            raise RuntimeError("liboal_amd.so ABI version mismatch")
        if path is None:
            _LIB = lib
        return lib


def load_hd_cublas_compat(manifest_path=None, runtime_probe_path=None, device=None, *, identity_policy=None):
    """Setup hook with the signature of the reference's bf16 loader
    (``oal_attention/hd_cublas_compat.py:688-799``): loads liboal_amd.so and
    checks that ``device`` is a ROCm device. The manifest and probe paths of
    the cuBLAS artifact have no meaning here and are ignored.
    """
    lib = load_library()
    if device is not None:
        dev = torch.device(device)
        if dev.type != "cuda" or torch.version.hip is None:
            raise RuntimeError("oal_amd runs only on a ROCm (HIP) device; got " + str(dev))
    return lib


def _check(rc: int, lib: ctypes.CDLL, what: str) -> None:
    if rc != 0:
        msg = lib.oal_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{what} failed: {msg}")


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _aligned(t: torch.Tensor | None) -> torch.Tensor | None:
    """t, or a fresh copy when its data pointer is not 16-byte aligned (the
    kernels move rows with 16-byte accesses; a view with an odd storage offset
    would otherwise be rejected by the library)."""
    if t is None or t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return DTYPE_F32
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    raise RuntimeError("q, k and v must be float32 or bfloat16 for the HIP kernels")


# ---------------------------------------------------------------------------
# Argument checks. Every tensor is checked for type, dtype, shape, layout and
# device before any pointer crosses the C ABI, as the reference's native op
# checks its operands (oal_attention/csrc/hd_cublas_compat.cpp:47-61, 104-148):
# the kernels trust the sizes they are given, so a short or mis-shaped buffer
# would otherwise be read or written out of bounds on the device. Failures are
# RuntimeError (the reference's TORCH_CHECK) and leave nothing enqueued.
# ---------------------------------------------------------------------------
def _check_tensor(t, name: str, *, dtype: torch.dtype, shape: tuple, device: torch.device | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a torch.Tensor")
    if t.layout != torch.strided:
        raise RuntimeError(f"{name} must be strided")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {str(dtype).replace('torch.', '')}, got {str(t.dtype).replace('torch.', '')}")
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {list(shape)}, got {list(t.shape)}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if device is not None and t.device != device:
        raise RuntimeError(f"{name} must be on the same device as q ({device}), got {t.device}")


def _check_bytes(t, name: str, nbytes: int, device: torch.device) -> None:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.uint8 or t.ndim != 1 or not t.is_contiguous():
        raise RuntimeError(f"{name} must be a contiguous 1-D uint8 tensor")
    if t.numel() < nbytes:
        raise RuntimeError(f"{name} holds {t.numel()} bytes; {nbytes} are needed")
    if t.device != device:
        raise RuntimeError(f"{name} must be on the same device as q ({device}), got {t.device}")


def _span(t: torch.Tensor) -> tuple[int, int]:
    start = t.data_ptr()
    return start, start + t.numel() * t.element_size()


def _check_no_overlap(out: torch.Tensor, name: str, others: dict) -> None:
    lo, hi = _span(out)
    for other_name, t in others.items():
        if t is None or t.device != out.device:
            continue
        a, b = _span(t)
        if a < hi and lo < b:
            raise RuntimeError(f"{name} must not overlap {other_name}")


def check_forward_args(q, k, v, labels, c0, lam, gam) -> tuple[int, int, int, int, int]:
    """Validate the forward operands; returns (B, Hq, Hkv, N, groups)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise RuntimeError(f"{name} must be a torch.Tensor")
        if t.ndim != 4:
            raise RuntimeError(f"{name} must be rank 4 [B, H, N, {HEAD_DIM}]")
    b, hq, n, d = q.shape
    hkv = k.shape[1]
    if min(b, hq, hkv, n) <= 0:
        raise RuntimeError("batch, head counts and sequence length must be positive")
    if hq % hkv != 0:
        raise RuntimeError("query head count must be divisible by KV head count")
    if d != HEAD_DIM:
        raise RuntimeError(f"q, k and v must be padded to {HEAD_DIM} features")
    _dtype_code(q.dtype)
    dev = q.device
    _check_tensor(q, "q", dtype=q.dtype, shape=(b, hq, n, HEAD_DIM))
    _check_tensor(k, "k", dtype=q.dtype, shape=(b, hkv, n, HEAD_DIM), device=dev)
    _check_tensor(v, "v", dtype=q.dtype, shape=(b, hkv, n, HEAD_DIM), device=dev)
    if not isinstance(lam, torch.Tensor) or lam.ndim != 2:
        raise RuntimeError("lam must be a [Hq, G] tensor")
    groups = lam.shape[1]
    if not 1 <= groups <= 64:
        raise RuntimeError("the group count must be in [1, 64]")
    _check_tensor(labels, "labels", dtype=torch.int32, shape=(hq, HEAD_DIM), device=dev)
    _check_tensor(c0, "c0", dtype=torch.float32, shape=(hq,), device=dev)
    _check_tensor(lam, "lam", dtype=torch.float32, shape=(hq, groups), device=dev)
    _check_tensor(gam, "gam", dtype=torch.float32, shape=(hq, groups, groups), device=dev)
    return b, hq, hkv, n, groups


def check_backward_args(q, k, v, labels, c0, lam, gam, num, den, saved, dout, dnum, dden):
    """Validate the VJP operands (dout, dnum and dden in the kernels' dtypes);
    returns (B, Hq, Hkv, N, groups)."""
    b, hq, hkv, n, groups = check_forward_args(q, k, v, labels, c0, lam, gam)
    dev = q.device
    _check_tensor(num, "num", dtype=torch.float32, shape=(b, hq, n, HEAD_DIM), device=dev)
    _check_tensor(den, "den", dtype=torch.float32, shape=(b, hq, n, 1), device=dev)
    if not isinstance(saved, torch.Tensor) or saved.dtype != torch.uint8 or saved.ndim != 1:
        raise RuntimeError("saved must be the 1-D uint8 tensor the forward returned")
    if dout is not None:
        _check_tensor(dout, "dout", dtype=q.dtype, shape=(b, hq, n, HEAD_DIM), device=dev)
    if dnum is not None:
        _check_tensor(dnum, "dnum", dtype=torch.float32, shape=(b, hq, n, HEAD_DIM), device=dev)
    if dden is not None:
        _check_tensor(dden, "dden", dtype=torch.float32, shape=(b, hq, n, 1), device=dev)
    return b, hq, hkv, n, groups


def _require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda" or torch.version.hip is None:
            raise RuntimeError("oal_amd runs only on a ROCm (HIP) device; got a tensor on " + str(t.device))


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def profile_enable(enable: bool) -> None:
    load_library().oal_profile_enable(1 if enable else 0)


def profile_collect() -> dict[str, tuple[int, float]]:
    """{kernel: (launches, total_ms)} for launches since the last collect."""
    lib = load_library()
    buf = ctypes.create_string_buffer(1 << 16)
    _check(lib.oal_profile_collect(buf, len(buf)), lib, "oal_profile_collect")
    result = {}
    for line in buf.value.decode().splitlines():
        name, count, total = line.split()
        result[name] = (int(count), float(total))
    return result


def chunk_size() -> int:
    return load_library().oal_chunk_size()


def _precision_code(precision: str) -> int:
    if precision == "fp32":
        return PRECISION_FP32
    if precision == "bf16":
        return PRECISION_BF16
    raise ValueError("precision must be 'fp32' or 'bf16'")


def selftest() -> int:
    """Run the matrix-core layout self-test on the current device; returns mismatches."""
    lib = load_library()
    dev = torch.device("cuda", torch.cuda.current_device())
    errors = torch.zeros(1, dtype=torch.int32, device=dev)
    _check(lib.oal_selftest(_ptr(errors), _stream(dev)), lib, "oal_selftest")
    return int(errors.item())


def forward(q, k, v, labels, c0, lam, gam, *, scale: float, floor: float, precision: str = "fp32",
            zero_saved: bool = False):
    """Run the HIP forward. q [B,Hq,N,64], k/v [B,Hkv,N,64] contiguous, same dtype;
    labels int32 [Hq,64]; c0 [Hq], lam [Hq,G], gam [Hq,G,G] float32.

    Returns (out [dtype], num f32, den f32 [B,Hq,N,1], saved uint8). The kernels
    leave the saved state's alignment gaps and padding tails unwritten;
    ``zero_saved`` allocates it zero-filled, so that every byte is defined (the
    registered operator's output, which tracing compares bytewise).
    """
    lib = load_library()
    b, hq, hkv, n, groups = check_forward_args(q, k, v, labels, c0, lam, gam)
    pcode = _precision_code(precision)
    _require_device(q)
    q, k, v = (_aligned(t) for t in (q, k, v))
    code = _dtype_code(q.dtype)
    dev = q.device
    with torch.cuda.device(dev), torch.profiler.record_function("oal_amd::forward"):
        nbytes = lib.oal_forward_saved_bytes(b, hq, hkv, n, groups, code, pcode)
        if nbytes == 0:
            _check(1, lib, "oal_forward_saved_bytes")
        out = torch.empty((b, hq, n, HEAD_DIM), dtype=q.dtype, device=dev)
        num = torch.empty((b, hq, n, HEAD_DIM), dtype=torch.float32, device=dev)
        den = torch.empty((b, hq, n, 1), dtype=torch.float32, device=dev)
        saved = (torch.zeros if zero_saved else torch.empty)((nbytes,), dtype=torch.uint8, device=dev)
        rc = lib.oal_forward(
            _ptr(q), _ptr(k), _ptr(v), _ptr(labels), _ptr(c0), _ptr(lam), _ptr(gam), groups,
            b, hq, hkv, n, code, pcode, float(scale), float(floor),
            _ptr(out), _ptr(num), _ptr(den), _ptr(saved), _stream(dev),
        )
        _check(rc, lib, "oal_forward")
    return out, num, den, saved


def backward(q, k, v, labels, c0, lam, gam, num, den, saved, dout, dnum, dden, *, scale: float, floor: float,
             need_q: bool, need_k: bool, need_v: bool, need_coef: bool, precision: str = "fp32",
             workspace: torch.Tensor | None = None):
    """Run the HIP VJP; returns (dq, dk, dv, dc0, dlam, dgam) with None where not requested.

    dout is cast to q's dtype and dnum, dden to float32 (the kernels' operand
    types) before the checks; every operand is then validated.
    """
    lib = load_library()
    if isinstance(q, torch.Tensor):
        if dout is not None:
            dout = dout.to(q.dtype).contiguous()
        if dnum is not None:
            dnum = dnum.to(torch.float32).contiguous()
        if dden is not None:
            dden = dden.to(torch.float32)
            dden = (dden.unsqueeze(-1) if dden.ndim == 3 else dden).contiguous()
    b, hq, hkv, n, groups = check_backward_args(q, k, v, labels, c0, lam, gam, num, den, saved, dout, dnum, dden)
    pcode = _precision_code(precision)
    _require_device(q)
    code = _dtype_code(q.dtype)
    dev = q.device
    with torch.cuda.device(dev), torch.profiler.record_function("oal_amd::backward"):
        sbytes = lib.oal_forward_saved_bytes(b, hq, hkv, n, groups, code, pcode)
        wbytes = lib.oal_backward_workspace_bytes(b, hq, hkv, n, groups, code, pcode)
        if sbytes == 0 or wbytes == 0:
            _check(1, lib, "oal_backward_workspace_bytes")
        _check_bytes(saved, "saved", sbytes, dev)
        if workspace is not None:
            _check_bytes(workspace, "workspace", wbytes, dev)
            _check_no_overlap(workspace, "workspace", {"q": q, "k": k, "v": v, "num": num, "den": den,
                                                       "saved": saved, "dout": dout, "dnum": dnum, "dden": dden})
        work = workspace if workspace is not None else torch.empty((wbytes,), dtype=torch.uint8, device=dev)
        dq = torch.empty_like(q) if need_q else None
        # the key-side kernels produce dk and dv together
        dk = torch.empty_like(k) if need_k or need_v else None
        dv = torch.empty_like(v) if need_k or need_v else None
        if need_coef:
            dc0 = torch.empty_like(c0)
            dlam = torch.empty_like(lam)
            dgam = torch.empty_like(gam)
        else:
            dc0 = dlam = dgam = None
        q, k, v, num, den, saved, dout, dnum, dden = (
            _aligned(t) for t in (q, k, v, num, den, saved, dout, dnum, dden))
        rc = lib.oal_backward(
            _ptr(q), _ptr(k), _ptr(v), _ptr(labels), _ptr(c0), _ptr(lam), _ptr(gam), groups,
            b, hq, hkv, n, code, pcode, float(scale), float(floor),
            _ptr(num), _ptr(den), _ptr(saved), _ptr(dout), _ptr(dnum), _ptr(dden),
            _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dc0), _ptr(dlam), _ptr(dgam), _ptr(work), _stream(dev),
        )
        _check(rc, lib, "oal_backward")
    return dq, dk if need_k else None, dv if need_v else None, dc0, dlam, dgam


# ---------------------------------------------------------------------------
# FP64 route (oal_forward_f64 / oal_backward_f64): every tensor float64.
# ---------------------------------------------------------------------------
def check_forward_args_f64(q, k, v, labels, c0, lam, gam) -> tuple[int, int, int, int, int]:
    """Validate the FP64 operands; returns (B, Hq, Hkv, N, groups)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise RuntimeError(f"{name} must be a torch.Tensor")
        if t.ndim != 4:
            raise RuntimeError(f"{name} must be rank 4 [B, H, N, {HEAD_DIM}]")
    b, hq, n, d = q.shape
    hkv = k.shape[1]
    if min(b, hq, hkv, n) <= 0:
        raise RuntimeError("batch, head counts and sequence length must be positive")
    if hq % hkv != 0:
        raise RuntimeError("query head count must be divisible by KV head count")
    if d != HEAD_DIM:
        raise RuntimeError(f"q, k and v must be padded to {HEAD_DIM} features")
    dev = q.device
    f64 = torch.float64
    _check_tensor(q, "q", dtype=f64, shape=(b, hq, n, HEAD_DIM))
    _check_tensor(k, "k", dtype=f64, shape=(b, hkv, n, HEAD_DIM), device=dev)
    _check_tensor(v, "v", dtype=f64, shape=(b, hkv, n, HEAD_DIM), device=dev)
    if not isinstance(lam, torch.Tensor) or lam.ndim != 2:
        raise RuntimeError("lam must be a [Hq, G] tensor")
    groups = lam.shape[1]
    if not 1 <= groups <= 64:
        raise RuntimeError("the group count must be in [1, 64]")
    _check_tensor(labels, "labels", dtype=torch.int32, shape=(hq, HEAD_DIM), device=dev)
    _check_tensor(c0, "c0", dtype=f64, shape=(hq,), device=dev)
    _check_tensor(lam, "lam", dtype=f64, shape=(hq, groups), device=dev)
    _check_tensor(gam, "gam", dtype=f64, shape=(hq, groups, groups), device=dev)
    return b, hq, hkv, n, groups


def forward_f64(q, k, v, labels, c0, lam, gam, *, scale: float):
    """FP64 forward: q [B,Hq,N,64], k/v [B,Hkv,N,64], c0/lam/gam float64, labels
    int32 [Hq,64]. Returns (out, num [B,Hq,N,64], den [B,Hq,N,1]), all float64."""
    lib = load_library()
    b, hq, hkv, n, groups = check_forward_args_f64(q, k, v, labels, c0, lam, gam)
    _require_device(q)
    q, k, v = (_aligned(t) for t in (q, k, v))
    dev = q.device
    with torch.cuda.device(dev), torch.profiler.record_function("oal_amd::forward_f64"):
        out = torch.empty((b, hq, n, HEAD_DIM), dtype=torch.float64, device=dev)
        num = torch.empty((b, hq, n, HEAD_DIM), dtype=torch.float64, device=dev)
        den = torch.empty((b, hq, n, 1), dtype=torch.float64, device=dev)
        rc = lib.oal_forward_f64(
            _ptr(q), _ptr(k), _ptr(v), _ptr(labels), _ptr(c0), _ptr(lam), _ptr(gam), groups,
            b, hq, hkv, n, float(scale), _ptr(out), _ptr(num), _ptr(den), _stream(dev),
        )
        _check(rc, lib, "oal_forward_f64")
    return out, num, den


def backward_f64(q, k, v, labels, c0, lam, gam, num, den, dout, dnum, dden, *, scale: float, need_q: bool,
                 need_kv: bool, need_coef: bool):
    """FP64 VJP; returns (dq, dk, dv, dc0, dlam, dgam) with None where not requested."""
    lib = load_library()
    f64 = torch.float64
    if dout is not None:
        dout = dout.to(f64).contiguous()
    if dnum is not None:
        dnum = dnum.to(f64).contiguous()
    if dden is not None:
        dden = dden.to(f64)
        dden = (dden.unsqueeze(-1) if dden.ndim == 3 else dden).contiguous()
    b, hq, hkv, n, groups = check_forward_args_f64(q, k, v, labels, c0, lam, gam)
    dev = q.device
    _check_tensor(num, "num", dtype=f64, shape=(b, hq, n, HEAD_DIM), device=dev)
    _check_tensor(den, "den", dtype=f64, shape=(b, hq, n, 1), device=dev)
    if dout is not None:
        _check_tensor(dout, "dout", dtype=f64, shape=(b, hq, n, HEAD_DIM), device=dev)
    if dnum is not None:
        _check_tensor(dnum, "dnum", dtype=f64, shape=(b, hq, n, HEAD_DIM), device=dev)
    if dden is not None:
        _check_tensor(dden, "dden", dtype=f64, shape=(b, hq, n, 1), device=dev)
    _require_device(q)
    with torch.cuda.device(dev), torch.profiler.record_function("oal_amd::backward_f64"):
        wbytes = lib.oal_backward_f64_workspace_bytes(b, hq, hkv, n, groups)
        if wbytes == 0:
            _check(1, lib, "oal_backward_f64_workspace_bytes")
        work = torch.empty((wbytes,), dtype=torch.uint8, device=dev)
        dq = torch.empty_like(q) if need_q else None
        dk = torch.empty_like(k) if need_kv else None
        dv = torch.empty_like(v) if need_kv else None
        if need_coef:
            dc0, dlam, dgam = torch.empty_like(c0), torch.empty_like(lam), torch.empty_like(gam)
        else:
            dc0 = dlam = dgam = None
        q, k, v, num, den, dout, dnum, dden = (_aligned(t) for t in (q, k, v, num, den, dout, dnum, dden))
        rc = lib.oal_backward_f64(
            _ptr(q), _ptr(k), _ptr(v), _ptr(labels), _ptr(c0), _ptr(lam), _ptr(gam), groups,
            b, hq, hkv, n, float(scale), _ptr(num), _ptr(den), _ptr(dout), _ptr(dnum), _ptr(dden),
            _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dc0), _ptr(dlam), _ptr(dgam), _ptr(work), _stream(dev),
        )
        _check(rc, lib, "oal_backward_f64")
    return dq, dk, dv, dc0, dlam, dgam
