"""The allocation-free backward (oal_backward_noalloc) against oal_backward.

Called through the C ABI with ctypes. Two calls in a row on one device, the
second with a smaller input (the static scratch keeps the first call's
contents), each compared with oal_backward on the same inputs and a
caller-allocated workspace, bitwise (every reduction of both routes has a fixed
order), for 8 groups, 12 groups and per-pair coefficients (64 groups), whose
workspaces differ (the per-pair bf16 layout adds per-head dk partials and local
slot partials; more than 8 groups run the fp32 route's scalar kernels). A geometry whose workspace
exceeds the 256 MiB scratch is refused with an error before anything runs.
"""

import ctypes

import pytest
import torch

from oal_amd import _native
from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _inputs(b, n, dtype, seed, dev, gcount=8):
    """8 groups: the configuration-1 inputs; 12 groups: random labels and a factor;
    64 groups: labels d -> d (the per-pair layout, whose bf16 workspace adds the
    per-head dk partials and the local slot partials)."""
    if gcount == 8:
        inp = go.config_inputs(1, batch=b, seq_len=n, seed=seed)
        q, k, v = (inp[x].to(dtype).to(dev).contiguous() for x in ("q", "k", "v"))
        labels, c0, lam, gam = (inp[x].to(dev).contiguous() for x in ("groups", "c0", "lam", "gam"))
        scale = inp["scale"]
    else:
        gen = torch.Generator().manual_seed(seed)
        q = (torch.randn((b, 14, n, 64), generator=gen) * 0.6).to(dtype).to(dev)
        k = (torch.randn((b, 2, n, 64), generator=gen) * 0.6).to(dtype).to(dev)
        v = torch.randn((b, 2, n, 64), generator=gen).to(dtype).to(dev)
        if gcount == 64:
            labels = torch.arange(64, dtype=torch.int32).unsqueeze(0).expand(14, -1).contiguous()
        else:
            labels = torch.randint(0, gcount, (14, 64), generator=gen, dtype=torch.int32)
            labels[:, :gcount] = torch.arange(gcount, dtype=torch.int32)
        side = gcount + 1
        factor = torch.randn((14, side * (side + 1) // 2), generator=gen, dtype=torch.float64)
        factor *= 0.05 if gcount == 64 else 0.3
        c0, lam, gam = (t.float().to(dev).contiguous()
                        for t in go.expand_factor(factor, query_heads=14, kernel_eps=0.05))
        labels = labels.to(dev)
        scale = 0.125
    gen = torch.Generator().manual_seed(seed + 1)
    dout = torch.randn(q.shape, generator=gen).to(dtype).to(dev)
    dden = torch.randn(q.shape[:3] + (1,), generator=gen).to(dev)
    return q, k, v, labels, c0, lam, gam, scale, dout, dden


def _noalloc(lib, q, k, v, labels, c0, lam, gam, num, den, saved, dout, dden, scale, precision):
    b, hq, n, _ = q.shape
    hkv = k.shape[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dc0, dlam, dgam = torch.empty_like(c0), torch.empty_like(lam), torch.empty_like(gam)
    p = _native._ptr
    rc = lib.oal_backward_noalloc(
        p(q), p(k), p(v), p(labels), p(c0), p(lam), p(gam), lam.shape[1], b, hq, hkv, n,
        _native._dtype_code(q.dtype), _native._precision_code(precision), float(scale), 0.0,
        p(num), p(den), p(saved), p(dout), None, p(dden), p(dq), p(dk), p(dv), p(dc0), p(dlam), p(dgam),
        _native._stream(q.device))
    assert rc == 0, lib.oal_last_error()
    return dq, dk, dv, dc0, dlam, dgam


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


@pytest.mark.parametrize("precision,dtype,gcount", [
    ("bf16", torch.bfloat16, 8), ("fp32", torch.float32, 8), ("bf16", torch.bfloat16, 12),
    ("fp32", torch.float32, 12), ("bf16", torch.bfloat16, 64), ("fp32", torch.float32, 64)])
def test_noalloc_backward_matches_the_workspace_entry_point(precision, dtype, gcount):
    dev = _dev()
    lib = _native.load_library()
    shapes = ((1, 1024, 3), (1, 200, 4)) if gcount <= 12 else ((1, 640, 3), (1, 130, 4))
    for call, (b, n, seed) in enumerate(shapes):
        print(f"noalloc call {call}: precision={precision} groups={gcount} B={b} N={n}", flush=True)
        q, k, v, labels, c0, lam, gam, scale, dout, dden = _inputs(b, n, dtype, seed, dev, gcount)
        _, num, den, saved = _native.forward(q, k, v, labels, c0, lam, gam, scale=scale, floor=0.0,
                                             precision=precision)
        want = _native.backward(q, k, v, labels, c0, lam, gam, num, den, saved, dout, None, dden, scale=scale,
                                floor=0.0, need_q=True, need_k=True, need_v=True, need_coef=True,
                                precision=precision)
        got = _noalloc(lib, q, k, v, labels, c0, lam, gam, num, den, saved, dout, dden, scale, precision)
        torch.cuda.synchronize()
        for name, g, w in zip(("dq", "dk", "dv", "dc0", "dlam", "dgam"), got, want):
            assert torch.isfinite(g.float()).all(), name
            # every reduction of both routes has a fixed order: bitwise
            assert torch.equal(g, w), (call, name, _rel(g, w))


def test_noalloc_refuses_a_geometry_beyond_the_scratch():
    _dev()
    lib = _native.load_library()
    need = lib.oal_backward_workspace_bytes(4, 14, 2, 4096, 8, 1, 1)
    assert need > (256 << 20)
    rc = lib.oal_backward_noalloc(
        *([ctypes.c_void_p(1 << 20)] * 7), 8, 4, 14, 2, 4096, 1, 1, ctypes.c_float(0.125), ctypes.c_float(0.0),
        *([ctypes.c_void_p(1 << 20)] * 3), None, None, None, *([None] * 6), None)
    assert rc != 0 and b"static scratch holds" in lib.oal_last_error()
