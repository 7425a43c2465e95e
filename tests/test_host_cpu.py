"""CPU-side checks: the C ABI library loads and exports every declared symbol,
and the host mirror of the reference interface validates like the reference
(no kernel is launched; there is no GPU here)."""

import ctypes
import os
import re

import pytest
import torch

from oal_amd import _native
from oal_amd import grouped_quadratic as gq
from oal_amd.hd_block_gemm import build_hd_block_gemm_plan, canonical_pair_layout

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "oal_amd.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(oal_[a-z_0-9]+)\(", text, re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    if not os.path.exists(_native.library_path()):
        pytest.skip("liboal_amd.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_native.library_path())
    declared = _declared_symbols()
    assert len(declared) >= 9
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.EXPORTED_SYMBOLS)
    loaded = _native.load_library()
    assert loaded.oal_feature_count() == 2145
    assert loaded.oal_feature_stride() % 64 == 0
    assert loaded.oal_chunk_size() > 0
    # the plan reports the token block the kernels run
    from oal_amd.hd_block_gemm import KERNEL_TOKEN_BLOCK

    assert loaded.oal_chunk_size() == KERNEL_TOKEN_BLOCK


def test_size_queries_and_argument_errors_without_a_gpu():
    if not os.path.exists(_native.library_path()):
        pytest.skip("liboal_amd.so not built")
    lib = _native.load_library()
    fp32 = lib.oal_forward_saved_bytes(1, 14, 2, 4096, 8, 1, 0)
    mfma = lib.oal_forward_saved_bytes(1, 14, 2, 4096, 8, 1, 1)
    assert fp32 > 0 and mfma > 0 and mfma != fp32
    # more than 8 groups stays on the matrix cores (feature-form local score,
    # same saved layout); more than 8 query heads per KV head runs the fp32 kernels
    assert lib.oal_forward_saved_bytes(1, 14, 2, 4096, 64, 1, 1) == mfma
    assert lib.oal_forward_saved_bytes(1, 18, 2, 4096, 8, 1, 1) == lib.oal_forward_saved_bytes(1, 18, 2, 4096, 8, 1, 0)
    # the per-pair path's workspace holds its local buffers too
    assert lib.oal_backward_workspace_bytes(1, 14, 2, 4096, 64, 1, 1) > lib.oal_backward_workspace_bytes(
        1, 14, 2, 4096, 8, 1, 1)
    assert lib.oal_backward_workspace_bytes(4, 14, 2, 4096, 8, 1, 1) > 0
    assert lib.oal_forward_saved_bytes(1, 14, 3, 4096, 8, 1, 0) == 0  # Hq % Hkv != 0
    assert b"divisible" in lib.oal_last_error()
    assert lib.oal_forward_saved_bytes(1, 14, 2, 4096, 8, 1, 5) == 0
    assert b"precision" in lib.oal_last_error()
    rc = lib.oal_forward(None, None, None, None, None, None, None, 8, 1, 1, 1, 64, 0, 0, 0.1, 0.0,
                         None, None, None, None, None)
    assert rc != 0 and b"null" in lib.oal_last_error()
    rc = lib.oal_forward(None, None, None, None, None, None, None, 8, 1, 1, 1, 64, 7, 0, 0.1, 0.0,
                         None, None, None, None, None)
    assert rc != 0 and b"dtype" in lib.oal_last_error()
    # misaligned tensor pointers are rejected before anything is enqueued (the
    # pointers are never dereferenced on this path)
    ok, odd = ctypes.c_void_p(1 << 20), ctypes.c_void_p((1 << 20) + 8)
    small = (ctypes.c_float * 64)()
    rc = lib.oal_forward(odd, ok, ok, small, small, small, small, 8, 1, 1, 1, 64, 0, 0, ctypes.c_float(0.1),
                         ctypes.c_float(0.0), ok, ok, ok, ok, None)
    assert rc != 0 and b"16-byte" in lib.oal_last_error()


def _case(dtype=torch.float32):
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(1, 2, 5, 4, generator=gen, dtype=dtype)
    k = torch.randn(1, 1, 5, 4, generator=gen, dtype=dtype)
    v = torch.randn(1, 1, 5, 3, generator=gen, dtype=dtype)
    return q, k, v


def test_invalid_dim_groups_are_rejected_like_the_reference():
    q, k, v = _case()
    factor = torch.tensor((1.1, 0.5, 0.9, 0.4, 0.8, 0.7))
    for bad in (
        torch.tensor((0.0, 0.0, 1.0, 1.0)),
        torch.tensor((-1, 0, 1, 1)),
        torch.tensor((0, 2, 2, 2)),
        torch.tensor((1, 1, 2, 2)),
        torch.tensor((0, 0, 2, 2)),
    ):
        with pytest.raises((TypeError, ValueError), match="dim_groups|group"):
            gq.oal_attention(q, k, v, bad, factor)


def test_invalid_factor_eps_and_options_are_rejected():
    q, k, v = _case()
    groups = torch.tensor((0, 0, 1, 1), dtype=torch.int32)
    with pytest.raises(ValueError, match="triangular|factor"):
        gq.oal_attention(q, k, v, groups, torch.ones(5))
    with pytest.raises(TypeError, match="floating"):
        gq.oal_attention(q, k, v, groups, torch.ones(6, dtype=torch.int64))
    for eps in (0.0, -1.0, float("inf"), 1e-50):
        with pytest.raises((TypeError, ValueError), match="kernel_eps"):
            gq.oal_attention(q, k, v, groups, torch.ones(6), kernel_eps=eps)
    with pytest.raises(ValueError, match="execution"):
        gq.oal_attention(q, k, v, groups, torch.ones(6), execution="torch")
    with pytest.raises(ValueError, match="causal"):
        gq.oal_attention(q, k, v, groups, torch.ones(6), causal=False)


def test_cpu_tensors_fail_loudly_instead_of_falling_back():
    q, k, v = _case()
    groups = torch.tensor((0, 0, 1, 1), dtype=torch.int32)
    factor = torch.tensor((1.1, 0.5, 0.9, 0.4, 0.8, 0.7))
    with pytest.raises(RuntimeError, match="ROCm|HIP"):
        gq.oal_attention(q, k, v, groups, factor)
    with pytest.raises(RuntimeError, match="reference"):
        gq.oal_attention(q, k, v, groups, factor, execution="reference")
    qp, kp, vp = (torch.nn.functional.pad(t, (0, 64 - t.shape[-1])).contiguous() for t in (q, k, v))
    labels = torch.nn.functional.pad(groups, (0, 60)).expand(2, 64).contiguous()
    with pytest.raises(RuntimeError, match="ROCm|HIP"):
        _native.forward(qp, kp, vp, labels, torch.ones(2), torch.ones(2, 2), torch.ones(2, 2, 2), scale=0.5,
                        floor=0.0)


def test_factor_expansion_is_exactly_symmetric_and_matches_known_answer():
    factor = torch.tensor((1.1, 0.5, 0.9, 0.4, 0.8, 0.7), dtype=torch.float64)
    c0, lam, gam = gq._expand_factor_coefficients(
        factor, query_heads=1, gmax=2, kernel_eps=0.07, working_dtype=torch.float64
    )
    lower = torch.tensor(((1.1, 0.0, 0.0), (0.5, 0.9, 0.0), (0.4, 0.8, 0.7)), dtype=torch.float64)
    m = lower @ lower.T
    torch.testing.assert_close(c0, m[0, 0].view(1) + 0.07)
    torch.testing.assert_close(lam, 2 * m[0, 1:].view(1, 2))
    torch.testing.assert_close(gam, m[1:, 1:].view(1, 2, 2))
    rnd = torch.randn(14, 45, generator=torch.Generator().manual_seed(4))
    _, _, g = gq._expand_factor_coefficients(rnd, query_heads=14, gmax=8, kernel_eps=1e-6,
                                             working_dtype=torch.float32)
    assert torch.equal(g, g.transpose(-1, -2))


def test_plan_records_caller_options_and_pair_layout():
    q, k, v = _case()
    plan = build_hd_block_gemm_plan(
        q, k, v, token_block=64, precision="bf16_tensorcore", requested_gradient_mask=(True,) * 6,
        key_feature_impl="triton_materialized", backward_schedule="shared_wave",
    )
    assert plan.key_feature_impl == "triton_materialized"
    assert plan.backward_schedule == "shared_wave"
    assert plan.number_blocks == 1 and plan.gqa_ratio == 2 and plan.pair_count == 10
    with pytest.raises(ValueError, match="precision"):
        build_hd_block_gemm_plan(q, k, v, precision="tf32", requested_gradient_mask=(False,) * 6)
    # a request of 128 (the reference planner's default) is recorded; the plan
    # reports the kernels' token block and its block count
    q2 = torch.zeros((1, 2, 300, 4))
    k2 = torch.zeros((1, 1, 300, 4))
    plan128 = build_hd_block_gemm_plan(q2, k2, k2, token_block=128, feature_wave_blocks=3,
                                       requested_gradient_mask=(True,) * 6)
    assert plan128.requested_token_block == 128
    assert plan128.token_block == 64 and plan128.number_blocks == 5
    assert plan128.feature_wave_blocks == 3
    layout = canonical_pair_layout(64)
    assert layout.pair_count == 2080
    assert layout.rows[:4] == (0, 1, 1, 2) and layout.columns[:4] == (0, 0, 1, 0)
