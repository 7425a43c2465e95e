"""The registered operators (oal_amd/ops.py) without a GPU: schemas, fake
kernels (output metadata and argument checks) and tracing of the forward into
a graph of the operator. Runs on fake ROCm tensors, so no
device is touched; the library is loaded only for its size query."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from oal_amd import _native, ops


def _lib_or_skip():
    try:
        _native.load_library()
    except RuntimeError as exc:
        pytest.skip(str(exc))


def _fake_inputs(dtype=torch.bfloat16, b=1, hq=14, hkv=2, n=300, dv=64, groups=8):
    dev = "cuda"
    q = torch.empty(b, hq, n, 64, device=dev, dtype=dtype)
    k = torch.empty(b, hkv, n, 64, device=dev, dtype=dtype)
    v = torch.empty(b, hkv, n, dv, device=dev, dtype=dtype)
    labels = torch.zeros(hq, 64, device=dev, dtype=torch.int32)
    c0 = torch.empty(hq, device=dev)
    lam = torch.empty(hq, groups, device=dev)
    gam = torch.empty(hq, groups, groups, device=dev)
    return q, k, v, labels, c0, lam, gam


def test_schemas():
    fwd = str(torch.ops.oal_amd.forward.default._schema)
    bwd = str(torch.ops.oal_amd.backward.default._schema)
    assert fwd == ("oal_amd::forward(Tensor q, Tensor k, Tensor v, Tensor labels, Tensor c0, Tensor lam, "
                   "Tensor gam, float scale, float floor, str precision) -> (Tensor, Tensor, Tensor, Tensor)")
    assert bwd.startswith("oal_amd::backward(Tensor q, Tensor k, Tensor v, Tensor labels, Tensor c0, Tensor lam, "
                          "Tensor gam, Tensor num, Tensor den, Tensor saved, Tensor? dout, Tensor? dnum, "
                          "Tensor? dden, float scale, float floor, bool need_q, bool need_k, bool need_v, "
                          "bool need_coef, str precision)")


@pytest.mark.parametrize("dtype,precision", [(torch.bfloat16, "bf16"), (torch.float32, "fp32")])
def test_fake_forward_metadata(dtype, precision):
    _lib_or_skip()
    with FakeTensorMode():
        q, k, v, labels, c0, lam, gam = _fake_inputs(dtype)
        out, num, den, saved = torch.ops.oal_amd.forward(q, k, v, labels, c0, lam, gam, 0.125, 0.0, precision)
        assert out.shape == q.shape and out.dtype == dtype and out.device == q.device
        assert num.shape == q.shape and num.dtype == torch.float32
        assert den.shape == (1, 14, 300, 1) and den.dtype == torch.float32
        assert saved.dtype == torch.uint8 and saved.ndim == 1
    lib = _native.load_library()
    want = lib.oal_forward_saved_bytes(1, 14, 2, 300, 8, _native._dtype_code(dtype), _native._precision_code(precision))
    assert saved.numel() == want


def test_fake_backward_metadata_follows_the_requests():
    _lib_or_skip()
    with FakeTensorMode():
        q, k, v, labels, c0, lam, gam = _fake_inputs()
        out, num, den, saved = torch.ops.oal_amd.forward(q, k, v, labels, c0, lam, gam, 0.125, 0.0, "bf16")
        grads = torch.ops.oal_amd.backward(q, k, v, labels, c0, lam, gam, num, den, saved, out, None, None,
                                           0.125, 0.0, True, False, False, True, "bf16")
        assert [tuple(g.shape) for g in grads] == [tuple(q.shape), (0,), (0,), (14,), (14, 8), (14, 8, 8)]


def test_fake_forward_checks_arguments():
    _lib_or_skip()
    with FakeTensorMode():
        q, k, v, labels, c0, lam, gam = _fake_inputs()
        with pytest.raises(RuntimeError, match="labels must have shape"):
            torch.ops.oal_amd.forward(q, k, v, labels[:, :32], c0, lam, gam, 0.125, 0.0, "bf16")
        with pytest.raises(RuntimeError, match="query head count must be divisible"):
            torch.ops.oal_amd.forward(q[:, :13].contiguous(), k, v, labels[:13], c0[:13], lam[:13], gam[:13],
                                      0.125, 0.0, "bf16")


def test_make_fx_traces_the_forward():
    # (the backward is traced in tests/test_gpu_ops.py: the autograd engine
    # needs a device for ROCm tensors, fake or not)
    _lib_or_skip()

    def fwd(q, k, v, labels, c0, lam, gam):
        return ops.grouped_oal_op(q, k, v, labels, c0, lam, gam, scale=0.125, floor=0.0, precision="bf16")

    with FakeTensorMode():
        gm = make_fx(fwd, tracing_mode="fake")(*_fake_inputs(dv=48))
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert "oal_amd.forward.default" in targets
