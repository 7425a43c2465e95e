"""The ctypes binding validates every tensor before a pointer crosses the C ABI.

Mirrors the operand checks of the reference's native op
(oal_attention/csrc/hd_cublas_compat.cpp:47-61, 104-148): type, dtype, shape,
contiguity and device, raised as RuntimeError with nothing enqueued. One case
per rejection; valid CPU operands get as far as the ROCm-device check, which is
the last one (no kernel runs here).
"""

import pytest
import torch

from oal_amd import _native


def _valid(b=1, hq=2, hkv=1, n=5, g=3, dtype=torch.float32):
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(b, hq, n, 64, generator=gen).to(dtype)
    k = torch.randn(b, hkv, n, 64, generator=gen).to(dtype)
    v = torch.randn(b, hkv, n, 64, generator=gen).to(dtype)
    labels = (torch.arange(64, dtype=torch.int32) % g).expand(hq, 64).contiguous()
    c0 = torch.ones(hq)
    lam = torch.ones(hq, g)
    gam = torch.eye(g).expand(hq, g, g).contiguous()
    return dict(q=q, k=k, v=v, labels=labels, c0=c0, lam=lam, gam=gam)


def _fwd(a):
    return _native.forward(a["q"], a["k"], a["v"], a["labels"], a["c0"], a["lam"], a["gam"], scale=0.125,
                           floor=0.0, precision="bf16")


def test_valid_operands_reach_the_device_check():
    a = _valid()
    assert _native.check_forward_args(a["q"], a["k"], a["v"], a["labels"], a["c0"], a["lam"], a["gam"]) == (
        1, 2, 1, 5, 3)
    with pytest.raises(RuntimeError, match="ROCm"):
        _fwd(a)


FORWARD_REJECTIONS = [
    ("q not a tensor", lambda a: a.update(q=[1.0]), "q must be a torch.Tensor"),
    ("q rank", lambda a: a.update(q=a["q"][0]), "q must be rank 4"),
    ("unpadded head dim", lambda a: a.update(q=a["q"][..., :32].contiguous()), "padded to 64"),
    ("Hq % Hkv", lambda a: a.update(k=torch.cat([a["k"]] * 3, 1), v=torch.cat([a["v"]] * 3, 1)), "divisible"),
    ("float16 q", lambda a: a.update(q=a["q"].half(), k=a["k"].half(), v=a["v"].half()), "float32 or bfloat16"),
    ("k dtype", lambda a: a.update(k=a["k"].double()), "k must be float32"),
    ("k seq len", lambda a: a.update(k=a["k"][:, :, :4].contiguous()), r"k must have shape \[1, 1, 5, 64\]"),
    ("v batch", lambda a: a.update(v=torch.cat([a["v"]] * 2, 0)), r"v must have shape"),
    ("q non-contiguous", lambda a: a.update(q=a["q"].transpose(2, 3).contiguous().transpose(2, 3)),
     "q must be contiguous"),
    ("labels int64", lambda a: a.update(labels=a["labels"].long()), "labels must be int32"),
    ("labels shape", lambda a: a.update(labels=a["labels"][:1].contiguous()), r"labels must have shape \[2, 64\]"),
    ("labels non-contiguous", lambda a: a.update(labels=a["labels"].t().contiguous().t()),
     "labels must be contiguous"),
    ("c0 dtype", lambda a: a.update(c0=a["c0"].double()), "c0 must be float32"),
    ("c0 shape", lambda a: a.update(c0=a["c0"][:1]), r"c0 must have shape \[2\]"),
    ("lam rank", lambda a: a.update(lam=a["lam"][0]), r"lam must be a \[Hq, G\] tensor"),
    ("too many groups", lambda a: a.update(lam=torch.ones(2, 65)), r"group count must be in \[1, 64\]"),
    ("lam heads", lambda a: a.update(lam=a["lam"][:1].contiguous()), r"lam must have shape \[2, 3\]"),
    ("gam smaller than lam", lambda a: a.update(gam=a["gam"][:, :2, :2].contiguous()),
     r"gam must have shape \[2, 3, 3\]"),
    ("gam non-contiguous", lambda a: a.update(gam=a["gam"].transpose(1, 2)), "gam must be contiguous"),
    ("gam dtype", lambda a: a.update(gam=a["gam"].half()), "gam must be float32"),
]


@pytest.mark.parametrize("case,mutate,message", FORWARD_REJECTIONS, ids=[c[0] for c in FORWARD_REJECTIONS])
def test_forward_rejects(case, mutate, message):
    a = _valid()
    mutate(a)
    with pytest.raises(RuntimeError, match=message):
        _fwd(a)


def test_precision_is_checked_before_the_device():
    a = _valid()
    with pytest.raises(ValueError, match="precision"):
        _native.forward(a["q"], a["k"], a["v"], a["labels"], a["c0"], a["lam"], a["gam"], scale=0.1, floor=0.0,
                        precision="fp16")


def _bwd_args(b=1, hq=2, n=5):
    a = _valid(b=b, hq=hq, n=n)
    a.update(
        num=torch.zeros(b, hq, n, 64),
        den=torch.ones(b, hq, n, 1),
        saved=torch.zeros(16, dtype=torch.uint8),
        dout=torch.zeros(b, hq, n, 64),
        dnum=None,
        dden=None,
    )
    return a


def _bwd(a):
    return _native.backward(a["q"], a["k"], a["v"], a["labels"], a["c0"], a["lam"], a["gam"], a["num"], a["den"],
                            a["saved"], a["dout"], a["dnum"], a["dden"], scale=0.125, floor=0.0, need_q=True,
                            need_k=True, need_v=True, need_coef=True)


BACKWARD_REJECTIONS = [
    ("num dtype", lambda a: a.update(num=a["num"].bfloat16()), "num must be float32"),
    ("num shape", lambda a: a.update(num=a["num"][..., :32].contiguous()), r"num must have shape \[1, 2, 5, 64\]"),
    ("den shape", lambda a: a.update(den=a["den"][:, :, :4].contiguous()), r"den must have shape \[1, 2, 5, 1\]"),
    ("den non-contiguous", lambda a: a.update(den=torch.ones(1, 5, 2, 1).transpose(1, 2)), "den must be contiguous"),
    ("saved dtype", lambda a: a.update(saved=torch.zeros(4, dtype=torch.float32)), "saved must be the 1-D uint8"),
    ("dout shape", lambda a: a.update(dout=torch.zeros(1, 2, 6, 64)), r"dout must have shape \[1, 2, 5, 64\]"),
    ("dnum shape", lambda a: a.update(dnum=torch.zeros(1, 2, 5, 63)), r"dnum must have shape"),
    ("dden shape", lambda a: a.update(dden=torch.zeros(1, 1, 5)), r"dden must have shape \[1, 2, 5, 1\]"),
    ("forward operand", lambda a: a.update(gam=a["gam"][:, :2, :2].contiguous()), r"gam must have shape"),
]


@pytest.mark.parametrize("case,mutate,message", BACKWARD_REJECTIONS, ids=[c[0] for c in BACKWARD_REJECTIONS])
def test_backward_rejects(case, mutate, message):
    a = _bwd_args()
    mutate(a)
    with pytest.raises(RuntimeError, match=message):
        _bwd(a)


def test_valid_backward_operands_reach_the_device_check():
    a = _bwd_args()
    a["dden"] = torch.zeros(1, 2, 5)  # [B, Hq, N] is accepted and viewed as [B, Hq, N, 1]
    with pytest.raises(RuntimeError, match="ROCm"):
        _bwd(a)


def test_caller_workspace_is_checked(monkeypatch):
    # with the device check passed, a short or overlapping workspace is refused
    # before the library is called
    a = _bwd_args()
    monkeypatch.setattr(_native, "_require_device", lambda *t: None)

    class _NoDevice:
        def __enter__(self):
            return self

        def __exit__(self, *exc):
            return False

    monkeypatch.setattr(torch.cuda, "device", lambda dev: _NoDevice())

    class _Lib:
        def oal_forward_saved_bytes(self, *args):
            return 16

        def oal_backward_workspace_bytes(self, *args):
            return 64

        def oal_backward(self, *args):
            raise AssertionError("the library must not be called")

    monkeypatch.setattr(_native, "load_library", lambda path=None: _Lib())
    with pytest.raises(RuntimeError, match="workspace holds 32 bytes; 64 are needed"):
        _native.backward(*[a[n] for n in ("q", "k", "v", "labels", "c0", "lam", "gam", "num", "den", "saved",
                                          "dout", "dnum", "dden")], scale=0.1, floor=0.0, need_q=True, need_k=True,
                         need_v=True, need_coef=False, workspace=torch.zeros(32, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="saved holds 16 bytes; 17 are needed|saved holds"):
        _Lib.oal_forward_saved_bytes = lambda self, *args: 17
        _native.backward(*[a[n] for n in ("q", "k", "v", "labels", "c0", "lam", "gam", "num", "den", "saved",
                                          "dout", "dnum", "dden")], scale=0.1, floor=0.0, need_q=True, need_k=True,
                         need_v=True, need_coef=False)
    _Lib.oal_forward_saved_bytes = lambda self, *args: 16
    base = torch.zeros(1024, dtype=torch.uint8)
    a["saved"] = base[:16]
    with pytest.raises(RuntimeError, match="workspace must not overlap saved"):
        _native.backward(*[a[n] for n in ("q", "k", "v", "labels", "c0", "lam", "gam", "num", "den", "saved",
                                          "dout", "dnum", "dden")], scale=0.1, floor=0.0, need_q=True, need_k=True,
                         need_v=True, need_coef=False, workspace=base[8:200])


# FP64 route (oal_forward_f64 / oal_backward_f64): every tensor float64.
def _valid64(b=1, hq=2, hkv=1, n=5, g=3):
    a = _valid(b, hq, hkv, n, g)
    for key in ("q", "k", "v", "c0", "lam", "gam"):
        a[key] = a[key].double()
    return a


def _fwd64(a):
    return _native.forward_f64(a["q"], a["k"], a["v"], a["labels"], a["c0"], a["lam"], a["gam"], scale=0.125)


def test_valid_f64_operands_reach_the_device_check():
    a = _valid64()
    assert _native.check_forward_args_f64(a["q"], a["k"], a["v"], a["labels"], a["c0"], a["lam"],
                                          a["gam"]) == (1, 2, 1, 5, 3)
    with pytest.raises(RuntimeError, match="ROCm"):
        _fwd64(a)
    n = a["q"].shape[2]
    num = torch.zeros(1, 2, n, 64, dtype=torch.float64)
    den = torch.ones(1, 2, n, 1, dtype=torch.float64)
    with pytest.raises(RuntimeError, match="ROCm"):
        _native.backward_f64(a["q"], a["k"], a["v"], a["labels"], a["c0"], a["lam"], a["gam"], num, den,
                             torch.zeros_like(num), None, None, scale=0.125, need_q=True, need_kv=True,
                             need_coef=True)


F64_REJECTIONS = [
    ("float32 q", lambda a: a.update(q=a["q"].float(), k=a["k"].float(), v=a["v"].float()), "q must be float64"),
    ("v dtype", lambda a: a.update(v=a["v"].float()), "v must be float64"),
    ("unpadded head dim", lambda a: a.update(q=a["q"][..., :32].contiguous()), "padded to 64"),
    ("c0 float32", lambda a: a.update(c0=a["c0"].float()), "c0 must be float64"),
    ("gam shape", lambda a: a.update(gam=a["gam"][:, :2, :2].contiguous()), r"gam must have shape \[2, 3, 3\]"),
    ("too many groups", lambda a: a.update(lam=torch.ones(2, 65, dtype=torch.float64)),
     r"group count must be in \[1, 64\]"),
    ("labels int64", lambda a: a.update(labels=a["labels"].long()), "labels must be int32"),
]


@pytest.mark.parametrize("case,mutate,message", F64_REJECTIONS, ids=[c[0] for c in F64_REJECTIONS])
def test_f64_forward_rejects(case, mutate, message):
    a = _valid64()
    mutate(a)
    with pytest.raises(RuntimeError, match=message):
        _fwd64(a)


def test_f64_backward_checks_num_and_den():
    a = _valid64()
    n = a["q"].shape[2]
    num = torch.zeros(1, 2, n, 64, dtype=torch.float32)
    den = torch.ones(1, 2, n, 1, dtype=torch.float64)
    with pytest.raises(RuntimeError, match="num must be float64"):
        _native.backward_f64(a["q"], a["k"], a["v"], a["labels"], a["c0"], a["lam"], a["gam"], num, den, None,
                             None, None, scale=0.125, need_q=True, need_kv=False, need_coef=False)
