"""Torch-CPU restatement of OAL grouped quadratic attention (test oracle).

TEST INFRASTRUCTURE ONLY -- never imported by the ``oal_amd`` package.

Kernel (reference ``oal_attention/grouped_reference.py:102-178``)::

    s_g(i, j)  = sum_{d : group(d) = g} sigma * q_{i,d} * k_{j,d}
    kappa(i,j) = c0 + sum_g lam_g s_g + sum_{r >= c} m_rc Gam[g(r), g(c)] x_r x_c
    num_i = sum_{j <= i} kappa(i, j) v_j ,  den_i = sum_{j <= i} kappa(i, j)

with x = sigma * q_i * k_j (elementwise), pairs (r, c) in
``torch.tril_indices`` order and multiplicity m_rc = 1 on the diagonal, 2 off
it.  For a symmetric Gam the pair sum equals sum_{g,h} Gam_gh s_g s_h.

Feature form used by the chunked path: kappa = phi_Q(q) . phi_K(k) with
``phi_K(k) = [1, k_d, k_r k_c]`` and ``phi_Q(q) = wq * [1, q_d, q_r q_c]``,
where the per-head feature coefficients are
``wq = [c0, sigma * lam[g(d)], m_rc * sigma^2 * Gam[g(r), g(c)]]``
(reference ``hd_block_gemm_feature_forward.py:259-389`` folds the same
coefficients into its query features).
"""

from __future__ import annotations

import math

import torch

# --------------------------------------------------------------------------
# Layout helpers
# --------------------------------------------------------------------------


def pair_indices(head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed lower-triangular pair order p(r, c) = r(r+1)/2 + c, r >= c.

    Follows ``grouped_reference.py:8-15`` (``torch.tril_indices``).
    """
    rows, cols = torch.tril_indices(head_dim, head_dim)
    return rows, cols


def infer_gmax(parameter_count: int) -> int:
    """Gmax from a packed (Gmax+1)(Gmax+2)/2 factor length.

    Follows ``grouped_quadratic.py:62-73``.
    """
    disc = 1 + 8 * parameter_count
    root = math.isqrt(disc)
    if root * root != disc or (root - 1) % 2 != 0:
        raise ValueError("factor last dimension must be a valid packed lower-triangular size")
    side = (root - 1) // 2
    return side - 1


def unpack_lower(factor: torch.Tensor, query_heads: int, gmax: int) -> torch.Tensor:
    """Packed row-major lower-triangular factor -> ``[Hq, G+1, G+1]``."""
    fac = factor.unsqueeze(0) if factor.ndim == 1 else factor
    if fac.shape[0] == 1:
        fac = fac.expand(query_heads, -1)
    side = gmax + 1
    rows, cols = torch.tril_indices(side, side)
    lower = torch.zeros((query_heads, side, side), dtype=fac.dtype)
    lower = lower.index_put((torch.arange(query_heads)[:, None], rows[None, :], cols[None, :]), fac)
    return lower


def expand_factor(
    factor: torch.Tensor, *, query_heads: int, kernel_eps: float
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Factor L -> (c0, lam, Gam) with M = L L^T.

    Follows ``grouped_quadratic.py:184-218``: c0 = M00 + eps,
    lam = 2 M[0, 1:], Gam = M[1:, 1:].
    """
    gmax = infer_gmax(factor.shape[-1])
    lower = unpack_lower(factor, query_heads, gmax)
    m = lower @ lower.transpose(-1, -2)
    c0 = m[:, 0, 0] + kernel_eps
    lam = 2.0 * m[:, 0, 1:]
    gam = m[:, 1:, 1:].contiguous()
    return c0, lam, gam


def _head_groups(dim_groups: torch.Tensor, query_heads: int) -> torch.Tensor:
    g = dim_groups if dim_groups.ndim == 2 else dim_groups.unsqueeze(0).expand(query_heads, -1)
    return g.to(torch.int64)


def feature_coefficients(
    dim_groups: torch.Tensor,
    c0: torch.Tensor,
    lam: torch.Tensor,
    gam: torch.Tensor,
    *,
    scale: float,
    head_dim: int,
) -> torch.Tensor:
    """Per-head feature coefficients ``wq [Hq, 1 + D + D(D+1)/2]``.

    Same selection as ``grouped_reference.py:61-99`` (lam gathered per
    dimension, Gam gathered per pair, multiplicity 1/2) with sigma folded in.
    Differentiable with respect to c0, lam and gam.
    """
    hq = c0.shape[0]
    groups = _head_groups(dim_groups, hq)
    rows, cols = pair_indices(head_dim)
    lin = lam.gather(1, groups) * scale
    heads = torch.arange(hq)[:, None]
    quad = gam[heads, groups[:, rows], groups[:, cols]]
    mult = torch.where(rows == cols, 1.0, 2.0).to(quad.dtype)
    quad = quad * mult[None, :] * (scale * scale)
    return torch.cat((c0[:, None], lin, quad), dim=1)


def raw_features(x: torch.Tensor) -> torch.Tensor:
    """``[..., D] -> [..., 1 + D + D(D+1)/2]`` = [1, x_d, x_r x_c]."""
    rows, cols = pair_indices(x.shape[-1])
    ones = torch.ones(x.shape[:-1] + (1,), dtype=x.dtype)
    return torch.cat((ones, x, x[..., rows] * x[..., cols]), dim=-1)


def fold_feature_gradient(dr: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """Adjoint of :func:`raw_features`: d/dx of sum(dr * raw_features(x)).

    Restates ``hd_block_gemm_key_ops.py:29-50`` (diagonal counted twice).
    """
    d = x.shape[-1]
    rows, cols = pair_indices(d)
    dp = dr[..., 1 + d :]
    out = dr[..., 1 : 1 + d].clone()
    out.index_add_(-1, rows, dp * x[..., cols])
    out.index_add_(-1, cols, dp * x[..., rows])
    return out


# --------------------------------------------------------------------------
# Materialized H0/H1/H2 restatement (grouped_reference.py:18-178)
# --------------------------------------------------------------------------


def materialized_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dim_groups: torch.Tensor,
    c0: torch.Tensor,
    lam: torch.Tensor,
    gam: torch.Tensor,
    *,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Causal num/den from token-cumulative KV states (small shapes only)."""
    b, hq, n, d = q.shape
    hkv = k.shape[1]
    dv = v.shape[-1]
    rows, cols = pair_indices(d)
    u = torch.cat((v, torch.ones((b, hkv, n, 1), dtype=v.dtype)), dim=-1)
    h0 = u.cumsum(2)
    h1 = (k.unsqueeze(-1) * u.unsqueeze(-2)).cumsum(2)
    h2 = ((k[..., rows] * k[..., cols]).unsqueeze(-1) * u.unsqueeze(-2)).cumsum(2)
    kv_of = torch.arange(hq) // (hq // hkv)
    h0, h1, h2 = (t.index_select(1, kv_of) for t in (h0, h1, h2))
    groups = _head_groups(dim_groups, hq)
    lin = lam.gather(1, groups)
    heads = torch.arange(hq)[:, None]
    quad = gam[heads, groups[:, rows], groups[:, cols]]
    mult = torch.where(rows == cols, 1.0, 2.0).to(quad.dtype)
    qs = q * scale
    qp = qs[..., rows] * qs[..., cols]
    y = (
        c0[None, :, None, None] * h0
        + (qs.unsqueeze(-1) * h1 * lin[None, :, None, :, None]).sum(-2)
        + (qp.unsqueeze(-1) * h2 * (quad * mult)[None, :, None, :, None]).sum(-2)
    )
    return y[..., :dv], y[..., dv:]


# --------------------------------------------------------------------------
# Dense N^2 factor-form oracle (tests/operators/test_grouped_quadratic.py:31-84)
# --------------------------------------------------------------------------


def dense_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dim_groups: torch.Tensor,
    factor: torch.Tensor,
    *,
    scale: float,
    kernel_eps: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Token-pair oracle: kappa = ||[1, z] L||^2 + eps, z = group sums."""
    b, hq, n, d = q.shape
    hkv = k.shape[1]
    gmax = infer_gmax(factor.shape[-1])
    lower = unpack_lower(factor, hq, gmax).to(q.dtype)
    groups = _head_groups(dim_groups, hq)
    kv_of = torch.arange(hq) // (hq // hkv)
    km = k.index_select(1, kv_of)
    vm = v.index_select(1, kv_of)
    contrib = (q * scale)[:, :, :, None, :] * km[:, :, None, :, :]  # [B,H,i,j,D]
    onehot = torch.nn.functional.one_hot(groups, gmax).to(q.dtype)  # [H,D,G]
    z = torch.einsum("bhijd,hdg->bhijg", contrib, onehot)
    feats = torch.cat((torch.ones_like(z[..., :1]), z), dim=-1)
    proj = torch.einsum("bhijc,hcs->bhijs", feats, lower)
    w = proj.square().sum(-1) + kernel_eps
    mask = torch.ones((n, n), dtype=torch.bool).tril()
    w = w.masked_fill(~mask, 0.0)
    num = torch.einsum("bhij,bhjv->bhiv", w, vm)
    den = w.sum(-1, keepdim=True)
    return num / den, num, den


def dense_forward_coefficients(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dim_groups: torch.Tensor,
    c0: torch.Tensor,
    lam: torch.Tensor,
    gam: torch.Tensor,
    *,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Token-pair oracle in the explicit pair-sum form (any Gam, symmetric or not)."""
    b, hq, n, d = q.shape
    hkv = k.shape[1]
    groups = _head_groups(dim_groups, hq)
    rows, cols = pair_indices(d)
    kv_of = torch.arange(hq) // (hq // hkv)
    km = k.index_select(1, kv_of)
    vm = v.index_select(1, kv_of)
    x = (q * scale)[:, :, :, None, :] * km[:, :, None, :, :]
    lin = lam.gather(1, groups)
    heads = torch.arange(hq)[:, None]
    quad = gam[heads, groups[:, rows], groups[:, cols]]
    mult = torch.where(rows == cols, 1.0, 2.0).to(q.dtype)
    w = (
        c0[None, :, None, None]
        + (x * lin[None, :, None, None, :]).sum(-1)
        + (x[..., rows] * x[..., cols] * (quad * mult)[None, :, None, None, :]).sum(-1)
    )
    mask = torch.ones((n, n), dtype=torch.bool).tril()
    w = w.masked_fill(~mask, 0.0)
    return torch.einsum("bhij,bhjv->bhiv", w, vm), w.sum(-1, keepdim=True)


# --------------------------------------------------------------------------
# Chunked feature form with closed-form backward
# --------------------------------------------------------------------------


def _chunks(n: int, chunk: int):
    for start in range(0, n, chunk):
        yield start, min(start + chunk, n)


@torch.no_grad()
def chunked_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    wq: torch.Tensor,
    *,
    chunk: int = 64,
    floor: float = 0.0,
    return_carry: bool = False,
):
    """Chunked causal forward in feature form.

    ``T_c = phi_K(K_c)^T [V_c, 1]``; ``P_c = sum_{c' < c} T_c'``;
    ``Y_i = phi_Q(q_i) P_c + sum_{j in c, j <= i} kappa(i, j) [v_j, 1]``;
    ``out = num / max(den, floor)``.  Mirrors the reference HD runtime
    (``hd_block_gemm_runtime.py:617-805``: block totals, exclusive cumsum,
    query wave contraction, normalize).  Returns (out, num, den[, carry]).
    """
    b, hq, n, d = q.shape
    hkv = k.shape[1]
    r = hq // hkv
    dv = v.shape[-1]
    dt = q.dtype
    state = torch.zeros((b, hkv, wq.shape[1], dv + 1), dtype=dt)
    y = torch.empty((b, hq, n, dv + 1), dtype=dt)
    carries = []
    for s, e in _chunks(n, chunk):
        fk = raw_features(k[:, :, s:e])  # [B,Hkv,C,F]
        u = torch.cat((v[:, :, s:e], torch.ones((b, hkv, e - s, 1), dtype=dt)), -1)
        fq = raw_features(q[:, :, s:e]) * wq[None, :, None, :]  # [B,Hq,C,F]
        fq5 = fq.view(b, hkv, r, e - s, -1)
        carry = state.clone()
        if return_carry:
            carries.append(carry)
        y_state = torch.einsum("bkrcf,bkfe->bkrce", fq5, carry)
        score = torch.einsum("bkrif,bkjf->bkrij", fq5, fk)
        score = torch.tril(score)
        y_loc = torch.einsum("bkrij,bkje->bkrie", score, u)
        y[:, :, s:e] = (y_state + y_loc).reshape(b, hq, e - s, dv + 1)
        state += torch.einsum("bkjf,bkje->bkfe", fk, u)
    num = y[..., :dv].contiguous()
    den = y[..., dv:].contiguous()
    out = num / torch.clamp(den, min=floor) if floor > 0 else num / den
    if return_carry:
        return out, num, den, carries
    return out, num, den


@torch.no_grad()
def normalization_vjp(dout, dnum, dden, num, den, *, floor: float = 0.0):
    """G = [dO/den' + dnum, -(dO . num)/den'^2 [den >= floor] + dden].

    Restates ``hd_block_gemm_normalization_ops.py:32-71``; den' = max(den, floor).
    """
    denp = torch.clamp(den, min=floor) if floor > 0 else den
    g = torch.zeros(num.shape[:-1] + (num.shape[-1] + 1,), dtype=num.dtype)
    if dout is not None:
        g[..., :-1] += dout / denp
        gz = -(dout * num).sum(-1, keepdim=True) / (denp * denp)
        if floor > 0:
            gz = gz * (den >= floor).to(gz.dtype)
        g[..., -1:] += gz
    if dnum is not None:
        g[..., :-1] += dnum
    if dden is not None:
        g[..., -1:] += dden
    return g


@torch.no_grad()
def chunked_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    wq: torch.Tensor,
    num: torch.Tensor,
    den: torch.Tensor,
    dout,
    dnum=None,
    dden=None,
    *,
    chunk: int = 64,
    floor: float = 0.0,
):
    """Closed-form VJP of :func:`chunked_forward`.

    Returns (dq, dk, dv, dwq) with dwq the gradient of the per-head feature
    coefficients (summed over batch and tokens).  The steps follow
    ``hd_block_gemm_backward.py``: normalization VJP (:191-308), dCarry per
    block and exclusive right scan (:764-908), query side
    dphi_Q = G P^T + ds phi_K (:473-761), KV side
    dphi_K = U dT^T + ds^T phi_Q and dU = phi_K dT + S^T G (:911-1452), and
    the feature folds (``hd_block_gemm_feature_backward.py:59-491``).
    """
    b, hq, n, d = q.shape
    hkv = k.shape[1]
    r = hq // hkv
    dv = v.shape[-1]
    dt = q.dtype
    f = wq.shape[1]
    g = normalization_vjp(dout, dnum, dden, num, den, floor=floor)  # [B,Hq,N,DV+1]
    spans = list(_chunks(n, chunk))

    # Forward carries (recomputed) and per-chunk dCarry.
    state = torch.zeros((b, hkv, f, dv + 1), dtype=dt)
    carries = []
    dcarry = []
    for s, e in spans:
        fk = raw_features(k[:, :, s:e])
        u = torch.cat((v[:, :, s:e], torch.ones((b, hkv, e - s, 1), dtype=dt)), -1)
        carries.append(state.clone())
        state += torch.einsum("bkjf,bkje->bkfe", fk, u)
        fq5 = (raw_features(q[:, :, s:e]) * wq[None, :, None, :]).view(b, hkv, r, e - s, f)
        g5 = g[:, :, s:e].reshape(b, hkv, r, e - s, dv + 1)
        dcarry.append(torch.einsum("bkrif,bkrie->bkfe", fq5, g5))
    # Exclusive right scan: dT_c = sum_{c' > c} dCarry_c'.
    dts = [None] * len(spans)
    acc = torch.zeros((b, hkv, f, dv + 1), dtype=dt)
    for idx in range(len(spans) - 1, -1, -1):
        dts[idx] = acc.clone()
        acc += dcarry[idx]

    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dvv = torch.zeros_like(v)
    dwq = torch.zeros_like(wq)
    for idx, (s, e) in enumerate(spans):
        c = e - s
        rq = raw_features(q[:, :, s:e])  # [B,Hq,C,F]
        fq = rq * wq[None, :, None, :]
        fq5 = fq.view(b, hkv, r, c, f)
        fk = raw_features(k[:, :, s:e])  # [B,Hkv,C,F]
        u = torch.cat((v[:, :, s:e], torch.ones((b, hkv, c, 1), dtype=dt)), -1)
        g5 = g[:, :, s:e].reshape(b, hkv, r, c, dv + 1)
        mask = torch.ones((c, c), dtype=torch.bool).tril()
        score = torch.einsum("bkrif,bkjf->bkrij", fq5, fk).masked_fill(~mask, 0.0)
        ds = torch.einsum("bkrie,bkje->bkrij", g5, u).masked_fill(~mask, 0.0)
        # Query side.
        dphi_q = torch.einsum("bkrie,bkfe->bkrif", g5, carries[idx]) + torch.einsum(
            "bkrij,bkjf->bkrif", ds, fk
        )
        dphi_q = dphi_q.reshape(b, hq, c, f)
        dwq += (dphi_q * rq).sum(dim=(0, 2))
        dq[:, :, s:e] = fold_feature_gradient(dphi_q * wq[None, :, None, :], q[:, :, s:e])
        # KV side.
        dphi_k = torch.einsum("bkje,bkfe->bkjf", u, dts[idx]) + torch.einsum(
            "bkrij,bkrif->bkjf", ds, fq5
        )
        dk[:, :, s:e] = fold_feature_gradient(dphi_k, k[:, :, s:e])
        du = torch.einsum("bkjf,bkfe->bkje", fk, dts[idx]) + torch.einsum(
            "bkrij,bkrie->bkje", score, g5
        )
        dvv[:, :, s:e] = du[..., :dv]
    return dq, dk, dvv, dwq


def coefficient_gradients_from_wq(
    dwq: torch.Tensor,
    dim_groups: torch.Tensor,
    gmax: int,
    *,
    scale: float,
    head_dim: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Map feature-coefficient gradients back to (dc0, dlam, dGam).

    Adjoint of :func:`feature_coefficients`: dGam[g(r), g(c)] accumulates
    pair (r, c) with r >= c exactly as the reference gather
    (``grouped_reference.py:89-93``) routes it.
    """
    hq = dwq.shape[0]
    groups = _head_groups(dim_groups, hq)
    rows, cols = pair_indices(head_dim)
    d = head_dim
    dc0 = dwq[:, 0].clone()
    dlam = torch.zeros((hq, gmax), dtype=dwq.dtype)
    dlam.scatter_add_(1, groups, dwq[:, 1 : 1 + d] * scale)
    mult = torch.where(rows == cols, 1.0, 2.0).to(dwq.dtype)
    dquad = dwq[:, 1 + d :] * mult[None, :] * (scale * scale)
    flat = groups[:, rows] * gmax + groups[:, cols]
    dgam = torch.zeros((hq, gmax * gmax), dtype=dwq.dtype)
    dgam.scatter_add_(1, flat, dquad)
    return dc0, dlam, dgam.view(hq, gmax, gmax)


def symmetrize_gamma_gradient(dgam: torch.Tensor) -> torch.Tensor:
    """Symmetric-Gam convention: off-diagonal [g][h] and [h][g] carry their mean.

    This is the gradient of sum_{g,h} Gam_gh s_g s_h with Gam a symmetric
    parameter; the reference routing and this one give identical gradients for
    any symmetric parameterization of Gam (e.g. the factor L L^T).
    """
    return 0.5 * (dgam + dgam.transpose(-1, -2))


# --------------------------------------------------------------------------
# Synthetic inputs of the benchmark configurations
# --------------------------------------------------------------------------

UNEVEN_GROUP_SIZES = (2, 4, 6, 8, 10, 10, 12, 12)


def seeded_groups(head_dim: int, sizes, generator: torch.Generator) -> torch.Tensor:
    """Labels ``[D]`` from a seeded permutation split into the given sizes."""
    perm = torch.randperm(head_dim, generator=generator)
    labels = torch.empty(head_dim, dtype=torch.int32)
    start = 0
    for gid, size in enumerate(sizes):
        labels[perm[start : start + size]] = gid
        start += size
    assert start == head_dim
    return labels


def seeded_coefficients(query_heads: int, gcount: int, generator: torch.Generator):
    """c0 = 1, lam_g ~ U(0.5, 1.5), b_gh ~ U(0, 0.5) for g <= h.

    The upper-triangle form sum_{g<=h} b_gh s_g s_h maps to a symmetric Gam
    with Gam_gg = b_gg and Gam_gh = Gam_hg = b_gh / 2.
    """
    c0 = torch.ones(query_heads, dtype=torch.float64)
    lam = 0.5 + torch.rand((query_heads, gcount), generator=generator, dtype=torch.float64)
    bmat = 0.5 * torch.rand((query_heads, gcount, gcount), generator=generator, dtype=torch.float64)
    upper = torch.triu(bmat)
    gam = 0.5 * (upper + upper.transpose(-1, -2))
    return c0, lam, gam


def config_inputs(
    config: int,
    *,
    batch: int | None = None,
    seq_len: int | None = None,
    dtype: torch.dtype = torch.float32,
    seed: int = 0,
):
    """Synthetic inputs of the benchmark configurations 0-3 (CPU tensors).

    config 0: B=1, H=1, N=256, D=64, q,k,v ~ N(0,1)/sqrt(8), 4 groups of 16.
    configs 1-3: Hq=14, Hkv=2, D=64, q,k,v ~ N(0,1) with 2 seeded outlier dims
    per head scaled x8; 8 uneven groups; coefficients as config 0.
    Returns dict(q, k, v, groups[Hq, D], c0, lam, gam, scale).
    """
    gen = torch.Generator().manual_seed(seed)
    d = 64
    if config == 0:
        b, hq, hkv, n = 1, 1, 1, 256
        sizes = (16, 16, 16, 16)
    else:
        b = {1: 1, 2: 4, 3: 1}[config]
        hq, hkv = 14, 2
        n = {1: 4096, 2: 4096, 3: 32768}[config]
        sizes = UNEVEN_GROUP_SIZES
    if batch is not None:
        b = batch
    if seq_len is not None:
        n = seq_len
    q = torch.randn((b, hq, n, d), generator=gen)
    k = torch.randn((b, hkv, n, d), generator=gen)
    v = torch.randn((b, hkv, n, d), generator=gen)
    if config == 0:
        q, k, v = (t / math.sqrt(8.0) for t in (q, k, v))
    else:
        for t, heads in ((q, hq), (k, hkv), (v, hkv)):
            for h in range(heads):
                dims = torch.randperm(d, generator=gen)[:2]
                t[:, h, :, dims] *= 8.0
    labels = seeded_groups(d, sizes, gen)
    groups = labels.unsqueeze(0).expand(hq, -1).contiguous()
    c0, lam, gam = seeded_coefficients(hq, len(sizes), gen)
    return dict(
        q=q.to(dtype),
        k=k.to(dtype),
        v=v.to(dtype),
        groups=groups,
        c0=c0.to(torch.float32),
        lam=lam.to(torch.float32),
        gam=gam.to(torch.float32),
        scale=d**-0.5,
    )
