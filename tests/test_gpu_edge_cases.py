"""Edge shapes of the bf16 matrix-core path against the fp32 oracle (GPU).

* sequence lengths at chunk boundaries: N = 1 (one token, one chunk, one scan
  segment), 63, 64, 65 (a one-token last chunk);
* heads per KV head R = 1 (Hq = Hkv), R = 8 (the largest the matrix-core kernels
  hold) and R = 9 (routed to the fp32 kernels);
* one group (every dimension in group 0) and eight groups of which three are
  empty for some heads.

Tolerance: rel-L2 <= 2e-2 (bf16 mode) on num, den and every gradient, against
the oracle evaluated on the same bf16-rounded q, k, v. dO is kept on the
well-conditioned tokens (denominator not a near-cancelling sum), as in
tests/test_gpu_parity.py.
"""

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    n = b.norm()
    return float((a - b).norm() / n) if n > 0 else float((a - b).norm())


def _case(b, hq, hkv, n, labels, seed):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn((b, hq, n, 64), generator=gen) * 0.6).to(torch.bfloat16).float()
    k = (torch.randn((b, hkv, n, 64), generator=gen) * 0.6).to(torch.bfloat16).float()
    v = torch.randn((b, hkv, n, 64), generator=gen).to(torch.bfloat16).float()
    g = int(labels.max()) + 1
    c0 = torch.ones(hq)
    lam = 0.5 + torch.rand((hq, g), generator=gen)
    upper = torch.triu(0.5 * torch.rand((hq, g, g), generator=gen))
    gam = 0.5 * (upper + upper.transpose(-1, -2))
    return q, k, v, c0, lam, gam


def _run(b, hq, hkv, n, labels, seed=0):
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    dev = _dev()
    q, k, v, c0, lam, gam = _case(b, hq, hkv, n, labels, seed)
    qb, kb, vb = (t.to(torch.bfloat16).to(dev).requires_grad_() for t in (q, k, v))
    c0d, lamd, gamd = (t.to(dev).requires_grad_() for t in (c0, lam, gam))
    out, num, den = grouped_oal(qb, kb, vb, labels.to(dev), c0d, lamd, gamd, scale=0.125, floor=0.0,
                                precision="bf16")
    wq = go.feature_coefficients(labels, c0, lam, gam, scale=0.125, head_dim=64)
    _, num_r, den_r = go.chunked_forward(q, k, v, wq, chunk=64)
    _, _, den_abs = go.chunked_forward(q.abs(), k.abs(), v, wq.abs(), chunk=64)
    mask = ((den_r.abs() > 0.5) & (den_abs <= 20 * den_r.abs())).float()
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 1)) * mask
    (out.float() * dout.to(dev)).sum().backward()
    dq_r, dk_r, dv_r, dwq_r = go.chunked_backward(q, k, v, wq, num_r, den_r, dout, None, None)
    g = lam.shape[1]
    dc0_r, dlam_r, dgam_r = go.coefficient_gradients_from_wq(dwq_r, labels, g, scale=0.125, head_dim=64)
    dgam_r = go.symmetrize_gamma_gradient(dgam_r)
    errs = {"num": rel(num, num_r), "den": rel(den, den_r)}
    for name, got, want in (("dq", qb.grad, dq_r), ("dk", kb.grad, dk_r), ("dv", vb.grad, dv_r),
                            ("dc0", c0d.grad, dc0_r), ("dlam", lamd.grad, dlam_r), ("dgam", gamd.grad, dgam_r)):
        errs[name] = rel(got, want)
    print(f"B={b} Hq={hq} Hkv={hkv} N={n} G={g}: " + " ".join(f"{k_}={e:.1e}" for k_, e in errs.items()), flush=True)
    if n == 1:
        # one token: out = v exactly, so every gradient but dv is zero (the oracle's
        # are rounding noise); here ds = g.v + gz cancels to bf16 rounding of G and
        # v, so they must stay within the bf16 tolerance of the scale of dv
        scale = float(vb.grad.abs().max())
        for name, got in (("dq", qb.grad), ("dk", kb.grad), ("dc0", c0d.grad), ("dlam", lamd.grad),
                          ("dgam", gamd.grad)):
            assert float(got.abs().max()) <= BF16_TOL * scale, (name, float(got.abs().max()), scale)
        errs = {k_: errs[k_] for k_ in ("num", "den", "dv")}
    assert all(e <= BF16_TOL for e in errs.values()), errs


def _labels(hq, g, seed=0):
    gen = torch.Generator().manual_seed(seed)
    lab = torch.randint(0, g, (hq, 64), generator=gen, dtype=torch.int32)
    lab[:, :g] = torch.arange(g, dtype=torch.int32)
    return lab


@pytest.mark.parametrize("n", [1, 63, 64, 65])
def test_sequence_lengths_at_chunk_boundaries(n):
    _run(2, 14, 2, n, _labels(14, 8), seed=n)


@pytest.mark.parametrize("hq,hkv", [(2, 2), (6, 2), (4, 1), (10, 2), (12, 2), (16, 2), (18, 2)])
def test_heads_per_kv_head(hq, hkv):
    """1 to 9 query heads per KV head: the shared-copy readout for 1 to 7 (one
    readout wave per head plus the copy wave), per-head readout blocks for 8, the
    fp32 kernels for 9."""
    _run(1, hq, hkv, 130, _labels(hq, 4), seed=hq)


def test_single_group_and_empty_groups():
    _run(1, 14, 2, 100, torch.zeros((14, 64), dtype=torch.int32), seed=5)
    lab = _labels(14, 5, seed=6)  # groups 5, 6, 7 of an eight-group factor stay empty
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    dev = _dev()
    q, k, v, c0, lam, gam = _case(1, 14, 2, 100, torch.full((1,), 7), 7)
    wq = go.feature_coefficients(lab, c0, lam, gam, scale=0.125, head_dim=64)
    _, num_r, den_r = go.chunked_forward(q, k, v, wq, chunk=64)
    args = [t.to(torch.bfloat16).to(dev) for t in (q, k, v)] + [t.to(dev) for t in (lab, c0, lam, gam)]
    _, num, den = grouped_oal(*args, scale=0.125, floor=0.0, precision="bf16")
    assert rel(num, num_r) <= BF16_TOL and rel(den, den_r) <= BF16_TOL


@pytest.mark.parametrize("grads", ["q", "k", "v", "kv", "coef"])
def test_partial_gradient_requests(grads):
    """Only some inputs require gradients: the others get None, the requested
    ones match the run where every input requires one."""
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    dev = _dev()
    lab = _labels(14, 8)
    q, k, v, c0, lam, gam = _case(1, 14, 2, 96, lab, 21)

    def run(req):
        ins = [t.to(torch.bfloat16).to(dev) for t in (q, k, v)] + [t.to(dev) for t in (c0, lam, gam)]
        for name, t in zip(("q", "k", "v", "c0", "lam", "gam"), ins):
            t.requires_grad_(name in req)
        out, num, den = grouped_oal(ins[0], ins[1], ins[2], lab.to(dev), ins[3], ins[4], ins[5], scale=0.125,
                                    floor=0.0, precision="bf16")
        g = torch.randn(out.shape, generator=torch.Generator().manual_seed(3)).to(dev)
        (out.float() * g).sum().backward()
        return [t.grad for t in ins]

    full = run({"q", "k", "v", "c0", "lam", "gam"})
    want = {"q": {"q"}, "k": {"k"}, "v": {"v"}, "kv": {"k", "v"}, "coef": {"c0", "lam", "gam"}}[grads]
    part = run(want)
    for name, gf, gp in zip(("q", "k", "v", "c0", "lam", "gam"), full, part):
        if name in want:
            assert gp is not None and torch.equal(gp, gf), name
        else:
            assert gp is None, name


@pytest.mark.parametrize("b,hq,hkv,n", [(3, 6, 3, 1000), (1, 7, 1, 777), (5, 4, 2, 200), (1, 2, 1, 4165)])
def test_irregular_shapes(b, hq, hkv, n):
    """Unit counts B * Hkv = 9, 1, 10 (the XCD-ordered block mappings fall back to
    plain order when the block count is not a multiple of 8), N not a multiple of
    the 64-token chunk, 2 to 7 query heads per KV head, and scan plans whose
    segments do not divide the chunk count. N = 4165 is 66 chunks: the
    denominator prefix scans take a full 64-chunk tile, then a tile of two."""
    _run(b, hq, hkv, n, _labels(hq, 6, seed=n), seed=b + n)


def test_misaligned_views_match_aligned_tensors():
    """q, k, v whose data pointers are 2 bytes past a 16-byte boundary (views
    into a larger buffer) give bit-identical outputs and gradients: the binding
    copies them to aligned memory before the library's 16-byte row accesses."""
    from oal_amd.hd_block_gemm_autograd import grouped_oal

    dev = _dev()
    labels = torch.arange(64).remainder(4).repeat(2, 1).to(torch.int32)
    q, k, v, c0, lam, gam = _case(1, 2, 1, 130, labels, seed=5)

    def run(shift):
        outs = []
        leaves = []
        for t in (q, k, v):
            buf = torch.zeros(t.numel() + shift, dtype=torch.bfloat16, device=dev)
            x = buf[shift:].view(t.shape)
            x.copy_(t.to(torch.bfloat16))
            leaves.append(x.requires_grad_())
        out, num, den = grouped_oal(*leaves, labels.to(dev), c0.to(dev), lam.to(dev), gam.to(dev), scale=0.125,
                                    floor=0.0, precision="bf16")
        (num.float().sum() + den.float().sum()).backward()
        torch.cuda.synchronize()
        return [out, num, den] + [x.grad for x in leaves], leaves

    base, leaves0 = run(0)
    mis, leaves1 = run(1)
    assert leaves0[0].data_ptr() % 16 == 0 and leaves1[0].data_ptr() % 16 == 2
    for a, b in zip(base, mis):
        assert torch.equal(a, b)
