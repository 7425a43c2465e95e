// FP64 evaluation of the grouped quadratic operator for gfx950: the HIP route
// of oal_attention(execution="reference") when the working dtype is float64.
//
// The reference evaluates that execution in the working dtype
// (oal_attention/grouped_quadratic.py:332-355, grouped_reference.py:102-211),
// and its gradients come from torch autograd of that evaluation. Here the
// operator is evaluated over token pairs, every operand and every sum in fp64:
//   p_d(i,j) = scale q_i[d] k_j[d]              (d < 64)
//   kappa    = c0 + sum_d a_d p_d + sum_{d,e} A_de p_d p_e
//   a_d      = lam[g(d)],  A_de = gam[g(d)][g(e)]
// which is the reference's kappa (s_g = sum_{d in g} p_d). Per pair, with
// inner_d = sum_e A_de p_e:
//   kappa = c0 + sum_d p_d (a_d + inner_d),   d kappa / d p_d = a_d + 2 inner_d.
// num_i = sum_{j<=i} kappa_ij v_j, den_i = sum_{j<=i} kappa_ij, out = num / den.
// VJP (normalization as hd_block_gemm_normalization_ops.py:32-71 without a floor):
//   G_i = dout_i / den_i + dnum_i,  Gz_i = -(dout_i . num_i) / den_i^2 + dden_i
//   ds_ij = G_i . v_j + Gz_i
//   dq_i[d] += ds_ij scale k_j[d] (a_d + 2 inner_d),  dk_j[d] likewise with q_i[d]
//   dv_j += kappa_ij G_i
//   dW[f] = sum ds_ij p_r p_c over the feature (r, c) table (p_64 = 1), routed to
//   dc0 = dW[0], dlam[g] = sum_{d in g} dW[1 + d],
//   dgam[g][h] = sum_{d in g, e in h} dW[pair(max(d,e), min(d,e))]
// (dgam is d/dgam of sum_{g,h} gam_gh s_g s_h, the convention of the fp32 and
// bf16 routes; a factor's gradient is the same under the reference's gather).
//
// The cost is O(N^2 (64 + 64 * 64 / 4)) per head in the forward: this route is
// for validation in double precision (gradcheck, quality sessions in float64),
// not for speed. Tiles of 32 queries x 32 keys; a block's 128 threads are 32
// tokens x 4 quarters, each quarter owning 16 of the 64 dimensions.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oal_common.hpp"
#include "oal_internal.hpp"

namespace oal {

static __constant__ FeatureTable kTab64 = make_feature_table();

namespace {

constexpr int kT = 32;         // tokens per tile
constexpr int kS = kD + 2;     // LDS row stride in doubles (16-byte aligned rows)
constexpr int kNT = 4 * kT;    // threads per block
constexpr int kCoefThreads = 256;
constexpr int kCoefSlots = (kFeat + kCoefThreads - 1) / kCoefThreads;  // features per thread

// Rows [tok0, tok0 + kT) of a [N][64] fp64 matrix into LDS; rows past N are zero.
__device__ __forceinline__ void stage_tile(double (*dst)[kS], const double* __restrict__ src, int tok0, int N) {
  for (int idx = threadIdx.x; idx < kT * (kD / 2); idx += blockDim.x) {
    const int r = idx / (kD / 2), c2 = idx % (kD / 2), tok = tok0 + r;
    double2 x = make_double2(0.0, 0.0);
    if (tok < N) x = reinterpret_cast<const double2*>(src + (size_t)tok * kD)[c2];
    reinterpret_cast<double2*>(&dst[r][0])[c2] = x;
  }
}

// G and Gz rows of a query tile: [G_i (64), Gz_i] per row; rows past N are zero.
__device__ __forceinline__ void stage_grad_tile(double (*dst)[kS], const double* __restrict__ Gv,
                                                const double* __restrict__ Gz, int tok0, int N) {
  stage_tile(dst, Gv, tok0, N);
  for (int r = threadIdx.x; r < kT; r += blockDim.x) dst[r][kD] = tok0 + r < N ? Gz[tok0 + r] : 0.0;
}

// Per-dimension coefficients of head h: A[d][e] = gam[g(d)][g(e)], A[d][64] =
// lam[g(d)]. Labels are clamped into [0, G) (the host validates them).
__device__ void stage_coefficients(double (*A)[kS], int* lab, const int32_t* __restrict__ labels,
                                   const double* __restrict__ lam, const double* __restrict__ gam, int G, int h) {
  __syncthreads();
  if (threadIdx.x < kD) {
    const int g = labels[h * kD + threadIdx.x];
    lab[threadIdx.x] = g < 0 ? 0 : (g >= G ? G - 1 : g);
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < kD * (kD + 1); idx += blockDim.x) {
    const int d = idx / (kD + 1), e = idx % (kD + 1);
    A[d][e] = e < kD ? gam[((size_t)h * G + lab[d]) * G + lab[e]] : lam[(size_t)h * G + lab[d]];
  }
  __syncthreads();
}

// Sum over the four quarters of a token (lanes 4 t .. 4 t + 3).
__device__ __forceinline__ double quarter_sum(double x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  return x;
}

// The quarter's part of a pair's p vector: pm[m] = scale x[d] y[d] for
// d = 16 cq + m, also written to the token's LDS row prow (the four quarters of
// a token are lanes of one wave, whose LDS accesses complete in program order,
// so the row is whole when the quarters read it back).
__device__ __forceinline__ void quarter_products(const double* x, const double* y, double scale, int cq,
                                                 double* prow, double (&pm)[16]) {
#pragma unroll
  for (int m = 0; m < 16; m += 2) {
    const int d = 16 * cq + m;
    const double2 a = *reinterpret_cast<const double2*>(x + d);
    const double2 b = *reinterpret_cast<const double2*>(y + d);
    pm[m] = scale * a.x * b.x;
    pm[m + 1] = scale * a.y * b.y;
    *reinterpret_cast<double2*>(prow + d) = make_double2(pm[m], pm[m + 1]);
  }
}

// inner_d = sum_e A[d][e] p[e] for the quarter's 16 dimensions d = 16 cq + m,
// p read back from the token's LDS row.
__device__ __forceinline__ void quarter_inner(const double (*A)[kS], int cq, const double* prow,
                                              double (&inner)[16]) {
#pragma unroll
  for (int m = 0; m < 16; ++m) inner[m] = 0.0;
#pragma unroll 2
  for (int e = 0; e < kD; e += 2) {
    const double2 pe = *reinterpret_cast<const double2*>(prow + e);
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const double2 w = *reinterpret_cast<const double2*>(&A[16 * cq + m][e]);
      inner[m] = fma(w.y, pe.y, fma(w.x, pe.x, inner[m]));
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Forward: one block per (query tile, batch x query head).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kNT) void k64_fwd(const double* __restrict__ q, const double* __restrict__ k,
                                               const double* __restrict__ v, const int32_t* __restrict__ labels,
                                               const double* __restrict__ c0, const double* __restrict__ lam,
                                               const double* __restrict__ gam, int G, int Hq, int Hkv, int N,
                                               double scale, double* __restrict__ out, double* __restrict__ num,
                                               double* __restrict__ den) {
  __shared__ __attribute__((aligned(16))) double A[kD][kS];
  __shared__ __attribute__((aligned(16))) double qs[kT][kS];
  __shared__ __attribute__((aligned(16))) double ks[kT][kS];
  __shared__ __attribute__((aligned(16))) double vs[kT][kS];
  __shared__ __attribute__((aligned(16))) double ps[kT][kS];  // p of each token's current pair
  __shared__ int lab[kD];
  const int it = blockIdx.x, bh = blockIdx.y;
  const int b = bh / Hq, h = bh % Hq, u = b * Hkv + h / (Hq / Hkv);
  const int t = threadIdx.x, i = t >> 2, cq = t & 3;
  const int tq = it * kT + i;
  stage_coefficients(A, lab, labels, lam, gam, G, h);
  stage_tile(qs, q + (size_t)bh * N * kD, it * kT, N);
  const double cc = c0[h];
  double acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) acc[m] = 0.0;
  double accz = 0.0;
  for (int jt = 0; jt <= it; ++jt) {
    __syncthreads();
    stage_tile(ks, k + (size_t)u * N * kD, jt * kT, N);
    stage_tile(vs, v + (size_t)u * N * kD, jt * kT, N);
    __syncthreads();
    for (int j = 0; j < kT; ++j) {
      double pm[16], inner[16];
      quarter_products(qs[i], ks[j], scale, cq, ps[i], pm);
      quarter_inner(A, cq, ps[i], inner);
      double part = 0.0;
#pragma unroll
      for (int m = 0; m < 16; ++m) part = fma(pm[m], A[16 * cq + m][kD] + inner[m], part);
      part = quarter_sum(part);
      const int tk = jt * kT + j;
      const double kap = (tk <= tq && tk < N) ? cc + part : 0.0;
#pragma unroll
      for (int m = 0; m < 16; ++m) acc[m] = fma(kap, vs[j][16 * cq + m], acc[m]);
      accz += kap;
    }
  }
  if (tq < N) {
    const size_t o = ((size_t)bh * N + tq) * kD + 16 * cq;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      num[o + m] = acc[m];
      out[o + m] = acc[m] / accz;
    }
    if (cq == 0) den[(size_t)bh * N + tq] = accz;
  }
}

// ---------------------------------------------------------------------------
// Normalization VJP, one wave per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k64_gvec(const double* __restrict__ dout, const double* __restrict__ dnum,
                                                const double* __restrict__ dden, const double* __restrict__ num,
                                                const double* __restrict__ den, long rows, double* __restrict__ Gv,
                                                double* __restrict__ Gz) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const double dd = den[row];
  const double dO = dout ? dout[row * kD + lane] : 0.0;
  double g = dO / dd;
  if (dnum) g += dnum[row * kD + lane];
  Gv[row * kD + lane] = g;
  double dot = dO * num[row * kD + lane];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
  if (lane == 0) {
    double gz = -dot / (dd * dd);
    if (dden) gz += dden[row];
    Gz[row] = gz;
  }
}

// ---------------------------------------------------------------------------
// Query-side VJP: one block per (query tile, batch x query head).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kNT) void k64_dq(const double* __restrict__ q, const double* __restrict__ k,
                                              const double* __restrict__ v, const int32_t* __restrict__ labels,
                                              const double* __restrict__ lam, const double* __restrict__ gam, int G,
                                              int Hq, int Hkv, int N, double scale, const double* __restrict__ Gv,
                                              const double* __restrict__ Gz, double* __restrict__ dq) {
  __shared__ __attribute__((aligned(16))) double A[kD][kS];
  __shared__ __attribute__((aligned(16))) double qs[kT][kS];
  __shared__ __attribute__((aligned(16))) double gs[kT][kS];
  __shared__ __attribute__((aligned(16))) double ks[kT][kS];
  __shared__ __attribute__((aligned(16))) double vs[kT][kS];
  __shared__ __attribute__((aligned(16))) double ps[kT][kS];  // p of each token's current pair
  __shared__ int lab[kD];
  const int it = blockIdx.x, bh = blockIdx.y;
  const int b = bh / Hq, h = bh % Hq, u = b * Hkv + h / (Hq / Hkv);
  const int t = threadIdx.x, i = t >> 2, cq = t & 3;
  const int tq = it * kT + i;
  stage_coefficients(A, lab, labels, lam, gam, G, h);
  stage_tile(qs, q + (size_t)bh * N * kD, it * kT, N);
  stage_grad_tile(gs, Gv + (size_t)bh * N * kD, Gz + (size_t)bh * N, it * kT, N);
  double acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) acc[m] = 0.0;
  for (int jt = 0; jt <= it; ++jt) {
    __syncthreads();
    stage_tile(ks, k + (size_t)u * N * kD, jt * kT, N);
    stage_tile(vs, v + (size_t)u * N * kD, jt * kT, N);
    __syncthreads();
    for (int j = 0; j < kT; ++j) {
      double ds = 0.0;
#pragma unroll
      for (int m = 0; m < 16; ++m) ds = fma(gs[i][16 * cq + m], vs[j][16 * cq + m], ds);
      ds = quarter_sum(ds) + gs[i][kD];
      const int tk = jt * kT + j;
      if (!(tk <= tq && tk < N)) ds = 0.0;
      double pm[16], inner[16];
      quarter_products(qs[i], ks[j], scale, cq, ps[i], pm);
      quarter_inner(A, cq, ps[i], inner);
      const double sds = ds * scale;
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const int d = 16 * cq + m;
        acc[m] = fma(sds * ks[j][d], A[d][kD] + 2.0 * inner[m], acc[m]);
      }
    }
  }
  if (tq < N) {
    const size_t o = ((size_t)bh * N + tq) * kD + 16 * cq;
#pragma unroll
    for (int m = 0; m < 16; ++m) dq[o + m] = acc[m];
  }
}

// ---------------------------------------------------------------------------
// Key/value-side VJP: one block per (key tile, unit = batch x KV head), summed
// over the unit's query heads in head order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kNT) void k64_dkv(const double* __restrict__ q, const double* __restrict__ k,
                                               const double* __restrict__ v, const int32_t* __restrict__ labels,
                                               const double* __restrict__ c0, const double* __restrict__ lam,
                                               const double* __restrict__ gam, int G, int Hq, int Hkv, int N,
                                               double scale, const double* __restrict__ Gv,
                                               const double* __restrict__ Gz, double* __restrict__ dk,
                                               double* __restrict__ dv) {
  __shared__ __attribute__((aligned(16))) double A[kD][kS];
  __shared__ __attribute__((aligned(16))) double qs[kT][kS];
  __shared__ __attribute__((aligned(16))) double gs[kT][kS];
  __shared__ __attribute__((aligned(16))) double ks[kT][kS];
  __shared__ __attribute__((aligned(16))) double vs[kT][kS];
  __shared__ __attribute__((aligned(16))) double ps[kT][kS];  // p of each token's current pair
  __shared__ int lab[kD];
  const int jt = blockIdx.x, u = blockIdx.y;
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int NT = (N + kT - 1) / kT;
  const int t = threadIdx.x, j = t >> 2, cq = t & 3;
  const int tk = jt * kT + j;
  stage_tile(ks, k + (size_t)u * N * kD, jt * kT, N);
  stage_tile(vs, v + (size_t)u * N * kD, jt * kT, N);
  double dka[16], dva[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) dka[m] = dva[m] = 0.0;
  for (int hh = 0; hh < R; ++hh) {
    const int h = kh * R + hh, bh = b * Hq + h;
    stage_coefficients(A, lab, labels, lam, gam, G, h);
    const double cc = c0[h];
    for (int it = jt; it < NT; ++it) {
      __syncthreads();
      stage_tile(qs, q + (size_t)bh * N * kD, it * kT, N);
      stage_grad_tile(gs, Gv + (size_t)bh * N * kD, Gz + (size_t)bh * N, it * kT, N);
      __syncthreads();
      for (int i = 0; i < kT; ++i) {
        const int tq = it * kT + i;
        const bool ok = tk <= tq && tq < N && tk < N;
        double pm[16], inner[16];
        quarter_products(qs[i], ks[j], scale, cq, ps[j], pm);
        quarter_inner(A, cq, ps[j], inner);
        double part = 0.0, ds = 0.0;
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          const int d = 16 * cq + m;
          part = fma(pm[m], A[d][kD] + inner[m], part);
          ds = fma(gs[i][d], vs[j][d], ds);
        }
        part = quarter_sum(part);
        ds = quarter_sum(ds) + gs[i][kD];
        const double kap = ok ? cc + part : 0.0;
        const double sds = ok ? ds * scale : 0.0;
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          const int d = 16 * cq + m;
          dva[m] = fma(kap, gs[i][d], dva[m]);
          dka[m] = fma(sds * qs[i][d], A[d][kD] + 2.0 * inner[m], dka[m]);
        }
      }
    }
  }
  if (tk < N) {
    const size_t o = ((size_t)u * N + tk) * kD + 16 * cq;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      if (dk) dk[o + m] = dka[m];
      if (dv) dv[o + m] = dva[m];
    }
  }
}

// ---------------------------------------------------------------------------
// Coefficient partials: one block per (query tile, batch x query head);
// part[bh][it][f] = sum over the tile's pairs of ds p_r p_c for feature f =
// (r, c) of the feature table (p_64 = 1, padding features 0). Each thread owns
// features f = t + 256 m; a query row's 32 pairs are staged at a time.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kCoefThreads) void k64_coef_part(const double* __restrict__ q,
                                                              const double* __restrict__ k,
                                                              const double* __restrict__ v, int Hq, int Hkv, int N,
                                                              double scale, const double* __restrict__ Gv,
                                                              const double* __restrict__ Gz,
                                                              double* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) double qs[kT][kS];
  __shared__ __attribute__((aligned(16))) double gs[kT][kS];
  __shared__ __attribute__((aligned(16))) double ks[kT][kS];
  __shared__ __attribute__((aligned(16))) double vs[kT][kS];
  __shared__ __attribute__((aligned(16))) double pr[kT][kS];  // p of one query row: [key][64 dims, 1, 0]
  __shared__ double dsr[kT];
  const int it = blockIdx.x, bh = blockIdx.y;
  const int NT = (N + kT - 1) / kT;
  const int b = bh / Hq, h = bh % Hq, u = b * Hkv + h / (Hq / Hkv);
  const int t = threadIdx.x;
  int fr[kCoefSlots], fc[kCoefSlots];
  double acc[kCoefSlots];
#pragma unroll
  for (int m = 0; m < kCoefSlots; ++m) {
    const int f = t + kCoefThreads * m;
    fr[m] = f < kFeat ? kTab64.r[f] : kD + 1;
    fc[m] = f < kFeat ? kTab64.c[f] : kD + 1;
    acc[m] = 0.0;
  }
  stage_tile(qs, q + (size_t)bh * N * kD, it * kT, N);
  stage_grad_tile(gs, Gv + (size_t)bh * N * kD, Gz + (size_t)bh * N, it * kT, N);
  for (int r = t; r < kT; r += blockDim.x) {
    pr[r][kD] = 1.0;
    pr[r][kD + 1] = 0.0;
  }
  for (int jt = 0; jt <= it; ++jt) {
    __syncthreads();
    stage_tile(ks, k + (size_t)u * N * kD, jt * kT, N);
    stage_tile(vs, v + (size_t)u * N * kD, jt * kT, N);
    for (int i = 0; i < kT; ++i) {
      __syncthreads();
      const int tq = it * kT + i;
      for (int idx = t; idx < kT * kD; idx += blockDim.x) {
        const int jj = idx / kD, d = idx % kD;
        pr[jj][d] = scale * qs[i][d] * ks[jj][d];
      }
      if (t < kT) {
        const int tk = jt * kT + t;
        double ds = gs[i][kD];
        for (int c = 0; c < kD; ++c) ds = fma(gs[i][c], vs[t][c], ds);
        dsr[t] = (tk <= tq && tk < N && tq < N) ? ds : 0.0;
      }
      __syncthreads();
      for (int jj = 0; jj < kT; ++jj) {
        const double ds = dsr[jj];
#pragma unroll
        for (int m = 0; m < kCoefSlots; ++m) acc[m] = fma(ds * pr[jj][fr[m]], pr[jj][fc[m]], acc[m]);
      }
    }
  }
  double* dst = part + ((size_t)bh * NT + it) * kFP;
#pragma unroll
  for (int m = 0; m < kCoefSlots; ++m) {
    const int f = t + kCoefThreads * m;
    if (f < kFP) dst[f] = f < kFeat ? acc[m] : 0.0;
  }
  for (int f = t + kCoefThreads * kCoefSlots; f < kFP; f += kCoefThreads) dst[f] = 0.0;
}

// ---------------------------------------------------------------------------
// dc0, dlam, dgam of head h: the partials summed over (batch, query tile) in a
// fixed order, then routed through the labels in ascending dimension order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k64_coef_grad(const double* __restrict__ part, int B, int Hq, int NT,
                                                     const int32_t* __restrict__ labels, int G,
                                                     double* __restrict__ dc0, double* __restrict__ dlam,
                                                     double* __restrict__ dgam) {
  __shared__ double w[kFP];
  __shared__ int lab[kD];
  __shared__ uint8_t mem[kD][kD];  // mem[g][0 .. cnt[g]): the dimensions of group g, ascending
  __shared__ int cnt[kD];
  const int h = blockIdx.x, t = threadIdx.x;
  if (t < kD) {
    const int g = labels[h * kD + t];
    lab[t] = g < 0 ? 0 : (g >= G ? G - 1 : g);
  }
  for (int f = t; f < kFP; f += blockDim.x) {
    double acc = 0.0;
    for (int b = 0; b < B; ++b) {
      const double* src = part + ((size_t)(b * Hq + h) * NT) * kFP + f;
      for (int it = 0; it < NT; ++it) acc += src[(size_t)it * kFP];
    }
    w[f] = acc;
  }
  for (int g = t; g < G; g += blockDim.x) {
    int n = 0;
    for (int d = 0; d < kD; ++d)
      if (lab[d] == g) mem[g][n++] = (uint8_t)d;
    cnt[g] = n;
  }
  __syncthreads();
  if (t == 0) dc0[h] = w[0];
  for (int g = t; g < G; g += blockDim.x) {
    double acc = 0.0;
    for (int i = 0; i < cnt[g]; ++i) acc += w[1 + mem[g][i]];
    dlam[(size_t)h * G + g] = acc;
  }
  // every (g, h) entry walks only its two groups' members: 64 x 64 terms per
  // head in all, whatever the group count
  for (int e = t; e < G * G; e += blockDim.x) {
    const int gr = e / G, gc = e % G;
    double acc = 0.0;
    for (int i = 0; i < cnt[gr]; ++i) {
      const int d = mem[gr][i];
      for (int j = 0; j < cnt[gc]; ++j) {
        const int c = mem[gc][j];
        const int r0 = d > c ? d : c, c0i = d > c ? c : d;
        acc += w[1 + kD + r0 * (r0 + 1) / 2 + c0i];
      }
    }
    dgam[(size_t)h * G * G + e] = acc;
  }
}

// ---------------------------------------------------------------------------
// Host launches.
// ---------------------------------------------------------------------------
size_t f64_workspace_bytes(int B, int Hq, int N) {
  const size_t rows = (size_t)B * Hq * N;
  const size_t NT = (size_t)(N + kT - 1) / kT;
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  return al(sizeof(double) * rows * kD) + al(sizeof(double) * rows) + al(sizeof(double) * B * Hq * NT * kFP);
}

void launch_f64_forward(const F64Geom& g, const double* q, const double* k, const double* v, const int32_t* labels,
                        const double* c0, const double* lam, const double* gam, int G, double scale, double* out,
                        double* num, double* den, hipStream_t st, const Timer& timed) {
  const int NT = (g.N + kT - 1) / kT;
  timed("k64_fwd", st, [&] {
    hipLaunchKernelGGL(k64_fwd, dim3(NT, g.B * g.Hq), dim3(kNT), 0, st, q, k, v, labels, c0, lam, gam, G, g.Hq,
                       g.Hkv, g.N, scale, out, num, den);
  });
}

void launch_f64_backward(const F64Geom& g, const double* q, const double* k, const double* v,
                         const int32_t* labels, const double* c0, const double* lam, const double* gam, int G,
                         double scale, const double* num, const double* den, const double* dout,
                         const double* dnum, const double* dden, double* dq, double* dk, double* dv, double* dc0,
                         double* dlam, double* dgam, void* workspace, hipStream_t st, const Timer& timed) {
  const int NT = (g.N + kT - 1) / kT;
  const size_t rows = (size_t)g.B * g.Hq * g.N;
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  char* p = static_cast<char*>(workspace);
  double* Gv = reinterpret_cast<double*>(p);
  p += al(sizeof(double) * rows * kD);
  double* Gz = reinterpret_cast<double*>(p);
  p += al(sizeof(double) * rows);
  double* part = reinterpret_cast<double*>(p);
  timed("k64_gvec", st, [&] {
    hipLaunchKernelGGL(k64_gvec, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, dout, dnum, dden, num, den,
                       (long)rows, Gv, Gz);
  });
  if (dq) {
    timed("k64_dq", st, [&] {
      hipLaunchKernelGGL(k64_dq, dim3(NT, g.B * g.Hq), dim3(kNT), 0, st, q, k, v, labels, lam, gam, G, g.Hq, g.Hkv,
                         g.N, scale, Gv, Gz, dq);
    });
  }
  if (dk || dv) {
    timed("k64_dkv", st, [&] {
      hipLaunchKernelGGL(k64_dkv, dim3(NT, g.B * g.Hkv), dim3(kNT), 0, st, q, k, v, labels, c0, lam, gam, G, g.Hq,
                         g.Hkv, g.N, scale, Gv, Gz, dk, dv);
    });
  }
  if (dc0) {
    timed("k64_coef_part", st, [&] {
      hipLaunchKernelGGL(k64_coef_part, dim3(NT, g.B * g.Hq), dim3(kCoefThreads), 0, st, q, k, v, g.Hq, g.Hkv, g.N,
                         scale, Gv, Gz, part);
    });
    timed("k64_coef_grad", st, [&] {
      hipLaunchKernelGGL(k64_coef_grad, dim3(g.Hq), dim3(256), 0, st, part, g.B, g.Hq, NT, labels, G, dc0, dlam,
                         dgam);
    });
  }
}

}  // namespace oal
