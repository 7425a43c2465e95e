// OAL grouped quadratic attention for gfx950: causal chunked forward and its
// first-order VJP, plus the C ABI declared in include/oal_amd.h.
//
// Algorithm (chunked feature form of the reference HD Block-GEMM core,
// oal_attention/hd_block_gemm_runtime.py:617-805 and hd_block_gemm_backward.py):
//   phi_K(k) = [1, k_d, k_r k_c],  phi_Q(q) = wq * [1, q_d, q_r q_c]
//   T_c = sum_{j in c} phi_K(k_j) [v_j, 1]^T,  P_c = sum_{c' < c} T_c'
//   y_i = phi_Q(q_i) P_c + sum_{j in c, j <= i} kappa(i, j) [v_j, 1]
// The intra-chunk kappa uses the group-sum form (O(D + G^2) per pair); the
// state terms use the 2145-wide feature space.
//
// Unit u = (b, kv head). Buffers (f32 unless noted):
//   wq     [Hq][kFP]              feature coefficients (saved)
//   carry  [U][NB][kFP][64], carry_z [U][NB][kFP]   exclusive prefix states (saved)
//   G      [B][Hq][N][64], Gz [B][Hq][N]            normalization VJP
//   dT     [U][NB][kFP][64], dTz [U][NB][kFP]       exclusive suffix of dCarry
//   dwq_part [B][Hq][NB][kFP], dwq [Hq][kFP]         feature-coefficient gradients

#include <hip/hip_runtime.h>
#include <rocprofiler-sdk-roctx/roctx.h>
#include <stdint.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "oal_amd.h"
#include "oal_common.hpp"
#include "oal_internal.hpp"

namespace oal {

__constant__ FeatureTable kTab = make_feature_table();

// ---------------------------------------------------------------------------
// Feature coefficients wq[h][f] (reference hd_block_gemm_feature_forward.py:259-389
// folds the same a / b / c coefficients into its query features).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_feature_coefficients(const int32_t* __restrict__ labels,
                                                              const float* __restrict__ c0,
                                                              const float* __restrict__ lam,
                                                              const float* __restrict__ gam, int G,
                                                              float scale, float* __restrict__ wq) {
  const int h = blockIdx.x;
  auto label = [&](int d) {
    int g = labels[h * kD + d];
    return g < 0 ? 0 : (g >= G ? G - 1 : g);
  };
  for (int f = threadIdx.x; f < kFP; f += blockDim.x) {
    const int r = kTab.r[f], c = kTab.c[f];
    float w;
    if (f == 0) {
      w = c0[h];
    } else if (f <= kD) {
      w = scale * lam[(size_t)h * G + label(r)];
    } else if (f < kFeat) {
      const float m = (r == c) ? 1.f : 2.f;
      w = m * scale * scale * gam[((size_t)h * G + label(r)) * G + label(c)];
    } else {
      w = 0.f;
    }
    wq[(size_t)h * kFP + f] = w;
  }
}

// Stages one chunk of a [.., N, 64] tensor into LDS rows [x, 1, 0]; rows past
// N are zero (including the constant slot).
template <typename T>
__device__ __forceinline__ void stage_rows(float (*dst)[kRow], const T* __restrict__ src, size_t base,
                                           int tok0, int N) {
  const int t = threadIdx.x;
  for (int idx = t; idx < kC * kD; idx += blockDim.x) {
    const int j = idx >> 6, d = idx & 63, tok = tok0 + j;
    dst[j][d] = tok < N ? to_f(src[base + (size_t)tok * kD + d]) : 0.f;
  }
  for (int j = t; j < kC; j += blockDim.x) {
    dst[j][kD] = (tok0 + j < N) ? 1.f : 0.f;
    dst[j][kD + 1] = 0.f;
  }
}

template <typename T>
__device__ __forceinline__ void stage_plain(float (*dst)[kD], const T* __restrict__ src, size_t base,
                                            int tok0, int N) {
  for (int idx = threadIdx.x; idx < kC * kD; idx += blockDim.x) {
    const int j = idx >> 6, d = idx & 63, tok = tok0 + j;
    dst[j][d] = tok < N ? to_f(src[base + (size_t)tok * kD + d]) : 0.f;
  }
}

// Stages a [kTile][64] (+ z column) feature tile of a per-chunk state.
__device__ __forceinline__ void stage_state_tile(float (*dst)[kD + 1], const float* __restrict__ s,
                                                 const float* __restrict__ sz, size_t row0) {
  const int t = threadIdx.x;
  for (int idx = t; idx < kTile * 16; idx += blockDim.x) {
    const int fr = idx >> 4, c4 = idx & 15;
    const float4 val = *reinterpret_cast<const float4*>(s + (row0 + fr) * kD + c4 * 4);
    dst[fr][c4 * 4 + 0] = val.x;
    dst[fr][c4 * 4 + 1] = val.y;
    dst[fr][c4 * 4 + 2] = val.z;
    dst[fr][c4 * 4 + 3] = val.w;
  }
  for (int fr = t; fr < kTile; fr += blockDim.x) dst[fr][kD] = sz[row0 + fr];
}

// ---------------------------------------------------------------------------
// Forward state scan: one block per (16-feature slice, unit); walks the chunks
// in order, stores the exclusive prefix P_c and accumulates
// T_c = phi_K^T [V, 1] (reference _write_block_totals_wave :271-310 plus
// _exclusive_cumsum_block_totals :313-320, fused).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_state_fwd(const T* __restrict__ k, const T* __restrict__ v, int N,
                                                   int NB, float* __restrict__ carry,
                                                   float* __restrict__ carry_z) {
  __shared__ float kx[kC][kRow];
  __shared__ float vx[kC][kD];
  const int u = blockIdx.y;
  const int t = threadIdx.x;
  const int f = blockIdx.x * 16 + (t >> 4);
  const int cg = t & 15;
  const int r = kTab.r[f], c = kTab.c[f];
  const size_t base = (size_t)u * N * kD;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float accz = 0.f;
  for (int ch = 0; ch < NB; ++ch) {
    const size_t row = ((size_t)u * NB + ch) * kFP + f;
    *reinterpret_cast<float4*>(carry + row * kD + cg * 4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    if (cg == 0) carry_z[row] = accz;
    __syncthreads();
    stage_rows(kx, k, base, ch * kC, N);
    stage_plain(vx, v, base, ch * kC, N);
    __syncthreads();
    for (int j = 0; j < kC; ++j) {
      const float phi = kx[j][r] * kx[j][c];
      const float4 vv = *reinterpret_cast<const float4*>(&vx[j][cg * 4]);
      acc[0] += phi * vv.x;
      acc[1] += phi * vv.y;
      acc[2] += phi * vv.z;
      acc[3] += phi * vv.w;
      accz += phi;
    }
  }
}

// ---------------------------------------------------------------------------
// Forward readout: one block per (query head in group, chunk, unit).
// y_i = phi_Q(q_i) P_c (state readout) + sum_{j<=i} kappa(i,j) [v_j, 1]
// (reference _contract_query_wave :411-614 and _write_and_normalize_query_wave
// :351-385). Thread t owns token i = t/4 and value columns 16*(t%4) .. +15.
// ---------------------------------------------------------------------------
template <typename T, int GMAX>
__global__ __launch_bounds__(256) void k_out_fwd(const T* __restrict__ q, const T* __restrict__ k,
                                                 const T* __restrict__ v, const float* __restrict__ wq,
                                                 const float* __restrict__ carry,
                                                 const float* __restrict__ carry_z,
                                                 const int32_t* __restrict__ labels,
                                                 const float* __restrict__ c0, const float* __restrict__ lam,
                                                 const float* __restrict__ gam, int G, int Hq, int Hkv, int N,
                                                 int NB, float scale, float floor, T* __restrict__ out,
                                                 float* __restrict__ num, float* __restrict__ den) {
  __shared__ float qx[kC][kRow];
  __shared__ float kx[kC][kRow];
  __shared__ float vx[kC][kD];
  __shared__ float kap[kC][kC + 1];
  __shared__ float pt[kTile][kD + 1];
  __shared__ HeadGroups<GMAX> hg;

  const int hh = blockIdx.x, ch = blockIdx.y, u = blockIdx.z;
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int t = threadIdx.x;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;

  stage_rows(qx, q, qbase, tok0, N);
  stage_rows(kx, k, kbase, tok0, N);
  stage_plain(vx, v, kbase, tok0, N);
  load_head_groups(hg, labels, c0, lam, gam, G, h);

  // Intra-chunk kappa(i, j), j <= i.
  for (int m = 0; m < kC / 4; ++m) {
    const int i = t >> 2, j = (t & 3) + 4 * m;
    float kv = 0.f;
    if (j <= i && tok0 + i < N) {
      float s[GMAX];
      group_sums(hg, G, qx[i], kx[j], scale, s);
      kv = kappa_of(hg, G, s);
    }
    kap[i][j] = kv;
  }

  const int i = t >> 2, cq = t & 3;
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  float accz = 0.f;
  const size_t crow0 = ((size_t)u * NB + ch) * kFP;
  const float* wqh = wq + (size_t)h * kFP;
  for (int f0 = 0; f0 < kFP; f0 += kTile) {
    __syncthreads();
    stage_state_tile(pt, carry, carry_z, crow0 + f0);
    __syncthreads();
    for (int fl = 0; fl < kTile; ++fl) {
      const int f = f0 + fl;
      const float phi = wqh[f] * qx[i][kTab.r[f]] * qx[i][kTab.c[f]];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] += phi * pt[fl][cq * 16 + e];
      accz += phi * pt[fl][kD];
    }
  }
  for (int j = 0; j <= i; ++j) {
    const float kv = kap[i][j];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] += kv * vx[j][cq * 16 + e];
    accz += kv;
  }
  const int tok = tok0 + i;
  if (tok < N) {
    const float dp = floor > 0.f ? fmaxf(accz, floor) : accz;
    const float inv = 1.f / dp;
    const size_t o = qbase + (size_t)tok * kD + cq * 16;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      num[o + e] = acc[e];
      out[o + e] = from_f<T>(acc[e] * inv);
    }
    if (cq == 0) den[(size_t)(b * Hq + h) * N + tok] = accz;
  }
}

// ---------------------------------------------------------------------------
// Normalization VJP (reference hd_block_gemm_normalization_ops.py:32-71):
// G = dO / den' + dnum,  Gz = -(dO . num) / den'^2 [den >= floor] + dden,
// den' = max(den, floor) (floor <= 0: den' = den, no mask). One wave per row.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_gvec(const T* __restrict__ dout, const float* __restrict__ dnum,
                                              const float* __restrict__ dden, const float* __restrict__ num,
                                              const float* __restrict__ den, long rows, float floor,
                                              float* __restrict__ G, float* __restrict__ Gz) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float dd = den[row];
  const float dp = floor > 0.f ? fmaxf(dd, floor) : dd;
  const float dO = dout ? to_f(dout[row * kD + lane]) : 0.f;
  float g = dO / dp;
  if (dnum) g += dnum[row * kD + lane];
  G[row * kD + lane] = g;
  const float dot = wave_sum(dO * num[row * kD + lane]);
  if (lane == 0) {
    float gz = -dot / (dp * dp);
    if (floor > 0.f && !(dd >= floor)) gz = 0.f;
    if (dden) gz += dden[row];
    Gz[row] = gz;
  }
}

// ---------------------------------------------------------------------------
// Backward state scan (reverse): dT_c = sum_{c' > c} dCarry_c',
// dCarry_c = sum_{h in unit} wq_h * (phi_raw(Q_h)^T G_h) over the chunk
// (reference _query_dcarry :764-877 and _exclusive_right_scan :880-908, fused).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_state_bwd(const T* __restrict__ q, const float* __restrict__ wq,
                                                   const float* __restrict__ Gv, const float* __restrict__ Gz,
                                                   int Hq, int Hkv, int N, int NB, float* __restrict__ dT,
                                                   float* __restrict__ dTz) {
  __shared__ float qx[kC][kRow];
  __shared__ float gs[kC][kD + 1];
  const int u = blockIdx.y;
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int t = threadIdx.x;
  const int f = blockIdx.x * 16 + (t >> 4);
  const int cg = t & 15;
  const int r = kTab.r[f], c = kTab.c[f];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float accz = 0.f;
  for (int ch = NB - 1; ch >= 0; --ch) {
    const size_t row = ((size_t)u * NB + ch) * kFP + f;
    *reinterpret_cast<float4*>(dT + row * kD + cg * 4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    if (cg == 0) dTz[row] = accz;
    const int tok0 = ch * kC;
    for (int hh = 0; hh < R; ++hh) {
      const int h = kh * R + hh;
      const size_t qbase = (size_t)(b * Hq + h) * N * kD;
      __syncthreads();
      stage_rows(qx, q, qbase, tok0, N);
      for (int idx = t; idx < kC * kD; idx += blockDim.x) {
        const int j = idx >> 6, d = idx & 63, tok = tok0 + j;
        gs[j][d] = tok < N ? Gv[qbase + (size_t)tok * kD + d] : 0.f;
      }
      for (int j = t; j < kC; j += blockDim.x) {
        const int tok = tok0 + j;
        gs[j][kD] = tok < N ? Gz[(size_t)(b * Hq + h) * N + tok] : 0.f;
      }
      __syncthreads();
      float tq[4] = {0.f, 0.f, 0.f, 0.f};
      float tz = 0.f;
      for (int i = 0; i < kC; ++i) {
        const float phi = qx[i][r] * qx[i][c];
        tq[0] += phi * gs[i][cg * 4 + 0];
        tq[1] += phi * gs[i][cg * 4 + 1];
        tq[2] += phi * gs[i][cg * 4 + 2];
        tq[3] += phi * gs[i][cg * 4 + 3];
        tz += phi * gs[i][kD];
      }
      const float w = wq[(size_t)h * kFP + f];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += w * tq[e];
      accz += w * tz;
    }
  }
}

// ---------------------------------------------------------------------------
// Query-side VJP: one block per (query head in group, chunk, unit).
// dphi_Q(i) = P_c g_i + sum_{j<=i} ds_ij phi_K(k_j), ds_ij = g_i . [v_j, 1]
// (reference _query_side_vjp :473-761), folded into dq
// (_fold_query_feature_gradient, feature_backward.py:157-422) and reduced into
// per-chunk feature-coefficient partials dwq_part (feature_backward.py:425-491).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_q_bwd(const T* __restrict__ q, const T* __restrict__ k,
                                               const T* __restrict__ v, const float* __restrict__ wq,
                                               const float* __restrict__ carry,
                                               const float* __restrict__ carry_z, const float* __restrict__ Gv,
                                               const float* __restrict__ Gz, int Hq, int Hkv, int N, int NB,
                                               T* __restrict__ dq, float* __restrict__ dwq_part) {
  __shared__ float qx[kC][kRow];
  __shared__ float kx[kC][kRow];
  __shared__ float vx[kC][kD];
  __shared__ float gs[kC][kD + 1];
  __shared__ float dsm[kC][kC + 1];
  __shared__ float pt[kTile][kD + 1];
  __shared__ float dqa[kC][kRow];
  __shared__ float dwr[4][kTile];

  const int hh = blockIdx.x, ch = blockIdx.y, u = blockIdx.z;
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int t = threadIdx.x;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;

  stage_rows(qx, q, qbase, tok0, N);
  stage_rows(kx, k, kbase, tok0, N);
  stage_plain(vx, v, kbase, tok0, N);
  for (int idx = t; idx < kC * kD; idx += blockDim.x) {
    const int j = idx >> 6, d = idx & 63, tok = tok0 + j;
    gs[j][d] = tok < N ? Gv[qbase + (size_t)tok * kD + d] : 0.f;
  }
  for (int j = t; j < kC; j += blockDim.x) {
    const int tok = tok0 + j;
    gs[j][kD] = tok < N ? Gz[(size_t)(b * Hq + h) * N + tok] : 0.f;
  }
  for (int idx = t; idx < kC * kRow; idx += blockDim.x) (&dqa[0][0])[idx] = 0.f;
  __syncthreads();

  for (int m = 0; m < kC / 4; ++m) {
    const int i = t >> 2, j = (t & 3) + 4 * m;
    float ds = 0.f;
    if (j <= i && tok0 + i < N) {
      ds = gs[i][kD];
      for (int e = 0; e < kD; ++e) ds += gs[i][e] * vx[j][e];
    }
    dsm[i][j] = ds;
  }

  const int i = t >> 2, fq = t & 3;
  const int lane = t & 63, wave = t >> 6;
  const size_t crow0 = ((size_t)u * NB + ch) * kFP;
  const float* wqh = wq + (size_t)h * kFP;
  float* dwp = dwq_part + ((size_t)(b * Hq + h) * NB + ch) * kFP;
  for (int f0 = 0; f0 < kFP; f0 += kTile) {
    __syncthreads();
    stage_state_tile(pt, carry, carry_z, crow0 + f0);
    __syncthreads();
    for (int m = 0; m < kTile / 4; ++m) {
      const int fl = fq + 4 * m, f = f0 + fl;
      const int r = kTab.r[f], c = kTab.c[f];
      float dphi = 0.f;
      for (int e = 0; e <= kD; ++e) dphi += gs[i][e] * pt[fl][e];
      for (int j = 0; j <= i; ++j) dphi += dsm[i][j] * kx[j][r] * kx[j][c];
      const float qr = qx[i][r], qc = qx[i][c];
      const float wd = wqh[f] * dphi;
      // the four lanes of token i (one wave) add their features' terms to its
      // row in turn, feature order f0 + 4 m + 0 .. 3: a fixed summation order
      // (lanes of the other tokens write other rows in the same turn)
      const float ar = wd * qc, ac = wd * qr;
#pragma unroll
      for (int turn = 0; turn < 4; ++turn) {
        if (fq == turn) {
          dqa[i][r] += ar;
          dqa[i][c] += ac;
        }
        __builtin_amdgcn_wave_barrier();
      }
      // sum over the 64 tokens: lanes sharing t % 4 within the wave, then waves
      float part = qr * qc * dphi;
      part += __shfl_xor(part, 4, 64);
      part += __shfl_xor(part, 8, 64);
      part += __shfl_xor(part, 16, 64);
      part += __shfl_xor(part, 32, 64);
      if (lane < 4) dwr[wave][fl] = part;
    }
    __syncthreads();
    if (t < kTile) dwp[f0 + t] = (dwr[0][t] + dwr[1][t]) + (dwr[2][t] + dwr[3][t]);
  }
  __syncthreads();
  if (dq) {
    for (int idx = t; idx < kC * kD; idx += blockDim.x) {
      const int j = idx >> 6, d = idx & 63, tok = tok0 + j;
      if (tok < N) dq[qbase + (size_t)tok * kD + d] = from_f<T>(dqa[j][d]);
    }
  }
}

// ---------------------------------------------------------------------------
// KV-side VJP: one block per (chunk, unit).
// state:  dphi_K(j) = dT_c [v_j, 1] -> dk (fold);  dv_j = dT_c^T phi_K(k_j)
// local:  dk_j += sum_h sum_{i>=j} ds_ij scale q_i (lam + 2 gam s)_{g(.)},
//         dv_j += sum_h sum_{i>=j} kappa_ij g_i
// (reference _kv_side_vjp :1031-1452 and _add_kv_cross_term_ :911-1028; the
// local term here uses the group-sum derivative instead of feature GEMMs).
// ---------------------------------------------------------------------------
template <typename T, int GMAX>
__global__ __launch_bounds__(256) void k_kv_bwd(const T* __restrict__ q, const T* __restrict__ k,
                                                const T* __restrict__ v, const float* __restrict__ dT,
                                                const float* __restrict__ dTz, const float* __restrict__ Gv,
                                                const float* __restrict__ Gz, const int32_t* __restrict__ labels,
                                                const float* __restrict__ c0, const float* __restrict__ lam,
                                                const float* __restrict__ gam, int G, int Hq, int Hkv, int N,
                                                int NB, float scale, T* __restrict__ dk, T* __restrict__ dv) {
  __shared__ float kx[kC][kRow];
  __shared__ float vx[kC][kD];
  __shared__ float qx[kC][kRow];
  __shared__ float gs[kC][kD + 1];
  __shared__ float dsm[kC][kC + 1];
  __shared__ float pt[kTile][kD + 1];
  __shared__ float dka[kC][kRow];
  __shared__ HeadGroups<GMAX> hg;

  const int ch = blockIdx.x, u = blockIdx.y;
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int t = threadIdx.x;
  const int tok0 = ch * kC;
  const size_t kbase = (size_t)u * N * kD;
  stage_rows(kx, k, kbase, tok0, N);
  stage_plain(vx, v, kbase, tok0, N);
  for (int idx = t; idx < kC * kRow; idx += blockDim.x) (&dka[0][0])[idx] = 0.f;

  const int j = t >> 2, xq = t & 3;
  float accv[16];
  float dkl[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    accv[e] = 0.f;
    dkl[e] = 0.f;
  }
  const size_t crow0 = ((size_t)u * NB + ch) * kFP;
  for (int f0 = 0; f0 < kFP; f0 += kTile) {
    __syncthreads();
    stage_state_tile(pt, dT, dTz, crow0 + f0);
    __syncthreads();
    for (int fl = 0; fl < kTile; ++fl) {
      const int f = f0 + fl;
      const float rk = kx[j][kTab.r[f]] * kx[j][kTab.c[f]];
#pragma unroll
      for (int e = 0; e < 16; ++e) accv[e] += rk * pt[fl][xq * 16 + e];
    }
    for (int m = 0; m < kTile / 4; ++m) {
      const int fl = xq + 4 * m, f = f0 + fl;
      const int r = kTab.r[f], c = kTab.c[f];
      float dphi = pt[fl][kD] * kx[j][kD];
      for (int e = 0; e < kD; ++e) dphi += pt[fl][e] * vx[j][e];
      // the four lanes of token j (one wave) add in turn: a fixed order
      const float ar = dphi * kx[j][c], ac = dphi * kx[j][r];
#pragma unroll
      for (int turn = 0; turn < 4; ++turn) {
        if (xq == turn) {
          dka[j][r] += ar;
          dka[j][c] += ac;
        }
        __builtin_amdgcn_wave_barrier();
      }
    }
  }

  for (int hh = 0; hh < R; ++hh) {
    const int h = kh * R + hh;
    const size_t qbase = (size_t)(b * Hq + h) * N * kD;
    __syncthreads();
    stage_rows(qx, q, qbase, tok0, N);
    for (int idx = t; idx < kC * kD; idx += blockDim.x) {
      const int jj = idx >> 6, d = idx & 63, tok = tok0 + jj;
      gs[jj][d] = tok < N ? Gv[qbase + (size_t)tok * kD + d] : 0.f;
    }
    for (int jj = t; jj < kC; jj += blockDim.x) {
      const int tok = tok0 + jj;
      gs[jj][kD] = tok < N ? Gz[(size_t)(b * Hq + h) * N + tok] : 0.f;
    }
    load_head_groups(hg, labels, c0, lam, gam, G, h);
    for (int m = 0; m < kC / 4; ++m) {
      const int ii = t >> 2, jj = (t & 3) + 4 * m;
      float ds = 0.f;
      if (jj <= ii && tok0 + ii < N) {
        ds = gs[ii][kD];
        for (int e = 0; e < kD; ++e) ds += gs[ii][e] * vx[jj][e];
      }
      dsm[ii][jj] = ds;
    }
    __syncthreads();
    if (tok0 + j < N) {
      for (int ii = j; ii < kC; ++ii) {
        if (tok0 + ii >= N) break;
        float s[GMAX];
        group_sums(hg, G, qx[ii], kx[j], scale, s);
        const float kapv = kappa_of(hg, G, s);
        const float ds = dsm[ii][j] * scale;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int x = xq * 16 + e;
          dkl[e] += ds * kappa_grad(hg, G, hg.lab[x], s) * qx[ii][x];
          accv[e] += kapv * gs[ii][x];
        }
      }
    }
  }
  __syncthreads();
  const int tok = tok0 + j;
  if (tok < N) {
    const size_t o = kbase + (size_t)tok * kD + xq * 16;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if (dk) dk[o + e] = from_f<T>(dka[j][xq * 16 + e] + dkl[e]);
      if (dv) dv[o + e] = from_f<T>(accv[e]);
    }
  }
}

// dwq[h][f] = sum_{b, chunk} dwq_part[b][h][chunk][f] in a fixed order. Block
// (64 features, head): 16 row sets, row set q sums rows q, q + 16, ... (row r =
// batch r / NB, chunk r % NB), then a fixed pairwise tree over the 16 sums.
__global__ __launch_bounds__(1024) void k_dwq_reduce(const float* __restrict__ part, int B, int Hq, int NB,
                                                     float* __restrict__ dwq) {
  __shared__ float ps[16][64];
  const int h = blockIdx.y, fl = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int f = blockIdx.x * 64 + fl;
  float acc = 0.f;
  if (f < kFP)
    for (int r = q; r < B * NB; r += 16) {
      const int b = r / NB, ch = r - b * NB;
      acc += part[((size_t)(b * Hq + h) * NB + ch) * kFP + f];
    }
  ps[q][fl] = acc;
  __syncthreads();
  for (int w = 8; w >= 1; w >>= 1) {
    if (q < w) ps[q][fl] += ps[q + w][fl];
    __syncthreads();
  }
  if (q == 0 && f < kFP) dwq[(size_t)h * kFP + f] = ps[0][fl];
}

// Adjoint of k_feature_coefficients: dc0, dlam[g], dgam[g][g'] in a fixed
// summation order. Pair (r, c), r >= c, is first routed to [g(r)][g(c)] as the
// reference gather does (grouped_reference.py:89-93); dgam is then reported in
// the symmetric-Gam convention (off-diagonal entries carry the mean of the two
// routings), the gradient of sum_{g,h} Gam_gh s_g s_h.
// loc (the matrix-core fp32 route, G <= 8): per-head local parts [Hq][73]
// (c0, lam[8], Gam[8][8] full symmetric, already in these coordinates).
__global__ __launch_bounds__(256) void k_coef_grad(const float* __restrict__ dwq,
                                                   const int32_t* __restrict__ labels, int G, float scale,
                                                   float* __restrict__ dc0, float* __restrict__ dlam,
                                                   float* __restrict__ dgam, const float* __restrict__ loc = nullptr) {
  __shared__ int lab[kD];
  __shared__ float raw[64 * 64];
  __shared__ float w[kFP];           // the head's slot gradients
  __shared__ uint8_t mem[64][kD];    // mem[g][0..cnt[g]): dims of group g, ascending
  __shared__ int cnt[64];
  const int h = blockIdx.x, t = threadIdx.x;
  if (t < kD) {
    int g = labels[h * kD + t];
    lab[t] = g < 0 ? 0 : (g >= G ? G - 1 : g);
  }
  for (int i = t; i < kFP; i += blockDim.x) w[i] = dwq[(size_t)h * kFP + i];
  __syncthreads();
  for (int g = t; g < G; g += blockDim.x) {
    int n = 0;
    for (int d = 0; d < kD; ++d)
      if (lab[d] == g) mem[g][n++] = (uint8_t)d;
    cnt[g] = n;
  }
  __syncthreads();
  const float* lc = loc ? loc + (size_t)h * 73 : nullptr;
  if (t == 0) dc0[h] = w[0] + (lc ? lc[0] : 0.f);
  // Both sums below visit dims in ascending order, the order of a plain scan over d / (r, c<=r).
  for (int g = t; g < G; g += blockDim.x) {
    float acc = 0.f;
    for (int i = 0; i < cnt[g]; ++i) acc += w[1 + mem[g][i]];
    dlam[(size_t)h * G + g] = acc * scale + (lc ? lc[1 + g] : 0.f);
  }
  const float s2 = scale * scale;
  for (int e = t; e < G * G; e += blockDim.x) {
    const int gr = e / G, gc = e % G;
    float acc = 0.f;
    for (int i = 0; i < cnt[gr]; ++i) {
      const int r = mem[gr][i];
      const float* row = w + 1 + kD + r * (r + 1) / 2;
      for (int j = 0; j < cnt[gc]; ++j) {
        const int c = mem[gc][j];
        if (c > r) break;
        acc += (r == c ? 1.f : 2.f) * row[c];
      }
    }
    raw[e] = acc * s2;
  }
  __syncthreads();
  for (int e = t; e < G * G; e += blockDim.x) {
    const int gr = e / G, gc = e % G;
    dgam[(size_t)h * G * G + e] =
        (gr == gc ? raw[e] : 0.5f * (raw[e] + raw[gc * G + gr])) + (lc ? lc[9 + 8 * gr + gc] : 0.f);
  }
}

}  // namespace oal

// ===========================================================================
// C ABI
// ===========================================================================
namespace {

thread_local std::string g_error;

int fail(const std::string& msg) {
  g_error = msg;
  return 1;
}

size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

struct Geometry {
  int B, Hq, Hkv, N, NB, U, R;
};

int check_geometry(int batch, int q_heads, int kv_heads, int seq_len, int dtype, Geometry* g) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq_len <= 0)
    return fail("batch, q_heads, kv_heads and seq_len must be positive");
  if (q_heads % kv_heads != 0) return fail("query head count must be divisible by KV head count");
  if (dtype != OAL_DTYPE_F32 && dtype != OAL_DTYPE_BF16) return fail("dtype must be OAL_DTYPE_F32 or OAL_DTYPE_BF16");
  const int NB = (seq_len + oal::kC - 1) / oal::kC;
  if ((long)batch * kv_heads > 65535 || NB > 65535) return fail("grid too large");
  *g = Geometry{batch, q_heads, kv_heads, seq_len, NB, batch * kv_heads, q_heads / kv_heads};
  return 0;
}

size_t saved_bytes(const Geometry& g) {
  const size_t wq = align_up(sizeof(float) * (size_t)g.Hq * oal::kFP);
  const size_t carry = align_up(sizeof(float) * (size_t)g.U * g.NB * oal::kFP * oal::kD);
  const size_t carry_z = align_up(sizeof(float) * (size_t)g.U * g.NB * oal::kFP);
  return wq + carry + carry_z;
}

struct SavedView {
  float* wq;
  float* carry;
  float* carry_z;
};

SavedView saved_view(const Geometry& g, void* base) {
  char* p = static_cast<char*>(base);
  SavedView s;
  s.wq = reinterpret_cast<float*>(p);
  p += align_up(sizeof(float) * (size_t)g.Hq * oal::kFP);
  s.carry = reinterpret_cast<float*>(p);
  p += align_up(sizeof(float) * (size_t)g.U * g.NB * oal::kFP * oal::kD);
  s.carry_z = reinterpret_cast<float*>(p);
  return s;
}

struct WorkView {
  float* G;
  float* Gz;
  float* dT;
  float* dTz;
  float* dwq_part;
  float* dwq;
  // matrix-core fp32 route (G <= 8): local parts and coefficient partials
  float* dql;    // [B][Hq][N][64]
  float* dkl;    // [B][Hq][N][64] per query head
  float* dvl;    // [B][Hq][N][64] per query head
  float* coefl;  // [B][Hq][NB][73]
  float* coefs;  // [Hq][73]
  float* segt;   // backward scan segment totals [U][S][kFP][64] (S > 1)
  float* segtz;  // [U][S][kFP]
  size_t bytes;
};

// The fp32 route runs on the matrix cores for up to 8 groups; more (per-pair
// coefficients) take the scalar feature-form kernels.
bool f32_mma(int groups) { return groups <= 8; }

WorkView work_view(const Geometry& g, void* base, bool mma) {
  char* p = static_cast<char*>(base);
  WorkView w;
  const size_t rows = (size_t)g.B * g.Hq * g.N;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    float* r = reinterpret_cast<float*>(p ? p + off : nullptr);
    off += align_up(bytes);
    return r;
  };
  w.G = take(sizeof(float) * rows * oal::kD);
  w.Gz = take(sizeof(float) * rows);
  w.dT = take(sizeof(float) * (size_t)g.U * g.NB * oal::kFP * oal::kD);
  w.dTz = take(sizeof(float) * (size_t)g.U * g.NB * oal::kFP);
  w.dwq_part = take(sizeof(float) * (size_t)g.B * g.Hq * g.NB * oal::kFP);
  w.dwq = take(sizeof(float) * (size_t)g.Hq * oal::kFP);
  w.dql = mma ? take(sizeof(float) * rows * oal::kD) : nullptr;
  w.dkl = mma ? take(sizeof(float) * rows * oal::kD) : nullptr;
  w.dvl = mma ? take(sizeof(float) * rows * oal::kD) : nullptr;
  w.coefl = mma ? take(sizeof(float) * (size_t)g.B * g.Hq * g.NB * 73) : nullptr;
  w.coefs = mma ? take(sizeof(float) * (size_t)g.Hq * 73) : nullptr;
  const int S = mma ? oal::f32_bwd_plan(g.U, g.NB, g.R).S : 1;
  w.segt = S > 1 ? take(sizeof(float) * (size_t)g.U * S * oal::kFP * oal::kD) : nullptr;
  w.segtz = S > 1 ? take(sizeof(float) * (size_t)g.U * S * oal::kFP) : nullptr;
  w.bytes = off;
  return w;
}

int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(std::string(what) + ": " + hipGetErrorString(err));
  return 0;
}

// Opt-in per-kernel timing: each launch is bracketed by HIP events recorded
// on its own stream; oal_profile_collect() waits for them and aggregates.
// The switch is atomic, so a launch with timing off takes no lock; the record
// list and the event pool are guarded by g_prof_mu.
struct ProfRecord {
  const char* name;
  hipEvent_t start, stop;
};
std::mutex g_prof_mu;
std::atomic<bool> g_prof_on{false};
std::vector<ProfRecord> g_prof_records;
std::vector<hipEvent_t> g_prof_pool;

hipEvent_t prof_event() {
  if (!g_prof_pool.empty()) {
    hipEvent_t e = g_prof_pool.back();
    g_prof_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Host-side stage ranges (roctx): every launch sits in a range named after its
// kernel, inside a range per entry point ("oal_forward", "oal_backward"), so a
// profiler's marker trace (rocprofv3 --marker-trace) shows the stages of a call
// next to its kernels, as the reference brackets its stages with
// record_function (oal_attention/hd_block_gemm_profiling.py:195-226). Without a
// profiler attached a range costs a call into an empty dispatch.
struct Range {
  explicit Range(const char* name) { roctxRangePushA(name); }
  ~Range() { roctxRangePop(); }
  Range(const Range&) = delete;
  Range& operator=(const Range&) = delete;
};

template <typename F>
void timed(const char* name, hipStream_t st, F&& launch) {
  Range range(name);
  if (!g_prof_on.load(std::memory_order_acquire)) {
    launch();
    return;
  }
  std::lock_guard<std::mutex> lock(g_prof_mu);
  hipEvent_t a = prof_event(), b = prof_event();
  if (a) hipEventRecord(a, st);
  launch();
  if (b) hipEventRecord(b, st);
  if (a && b) g_prof_records.push_back({name, a, b});
}

// The matrix-core kernels keep up to 8 query heads per KV head in registers;
// more run the fp32 kernels. Up to 8 groups take the group-sum intra-chunk
// kernels, more (per-pair coefficients) the feature-form ones.
bool use_mfma(int precision, int groups, const Geometry& g) {
  return precision == OAL_PRECISION_BF16 && groups <= 64 && g.R <= 8;
}

oal::LaunchGeom launch_geom(const Geometry& g) { return oal::LaunchGeom{g.B, g.Hq, g.Hkv, g.N, g.NB, g.U, g.R}; }

// Second stream and fork/join events per device, created on first use and kept
// until the process ends. An event is recorded on the signalling stream and
// waited for within the same call, a few records later at most; the ring is
// long enough that an event is recorded again only after its earlier waits
// were enqueued (a wait takes the record at the time it is enqueued).
constexpr int kAuxDevices = 64;
constexpr int kAuxEvents = 64;
struct AuxState {
  hipStream_t stream = nullptr;
  hipEvent_t events[kAuxEvents] = {};
  unsigned next = 0;
  bool failed = false;
};
std::mutex g_aux_mu;
AuxState g_aux[kAuxDevices];

}  // namespace

namespace oal {

hipStream_t aux_stream(hipStream_t st) {
  if (g_prof_on.load(std::memory_order_acquire)) return st;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kAuxDevices) return st;
  if (st) {
    int sdev = -1;
    if (hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev) return st;
  }
  std::lock_guard<std::mutex> lock(g_aux_mu);
  AuxState& a = g_aux[dev];
  if (a.failed) return st;
  if (!a.stream) {
    // the stream and its events are not created while st is being captured
    // into a graph (that call then runs on st alone)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (st && (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)) {
      (void)hipGetLastError();
      return st;
    }
    bool ok = hipStreamCreateWithFlags(&a.stream, hipStreamNonBlocking) == hipSuccess;
    for (int i = 0; ok && i < kAuxEvents; ++i)
      ok = hipEventCreateWithFlags(&a.events[i], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
      a.failed = true;
      (void)hipGetLastError();
      return st;
    }
  }
  return a.stream;
}

hipEvent_t next_event() {
  int dev = -1;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lock(g_aux_mu);
  AuxState& a = g_aux[dev];
  return a.events[a.next++ % kAuxEvents];
}

hipEvent_t record_event(hipStream_t s) {
  hipEvent_t ev = next_event();
  (void)hipEventRecord(ev, s);
  return ev;
}

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return cs != hipStreamCaptureStatusNone;
}

void wait_event(hipStream_t waiter, hipEvent_t ev) { (void)hipStreamWaitEvent(waiter, ev, 0); }

void stream_wait(hipStream_t waiter, hipStream_t signaller) { wait_event(waiter, record_event(signaller)); }

}  // namespace oal

namespace {

oal::Timer make_timer() {
  return [](const char* name, hipStream_t st, const std::function<void()>& launch) { timed(name, st, launch); };
}

template <typename T, int GMAX>
int forward_impl(const Geometry& g, const void* q, const void* k, const void* v, const int32_t* labels,
                 const float* c0, const float* lam, const float* gam, int groups, float scale, float floor,
                 void* out, float* num, float* den, void* saved, hipStream_t st, hipStream_t aux) {
  using namespace oal;
  SavedView sv = saved_view(g, saved);
  const T* qt = static_cast<const T*>(q);
  const T* kt = static_cast<const T*>(k);
  const T* vt = static_cast<const T*>(v);
  timed("k_feature_coefficients", st, [&] { hipLaunchKernelGGL(k_feature_coefficients, dim3(g.Hq), dim3(256), 0, st, labels, c0, lam, gam, groups, scale,
                     sv.wq); });
  if constexpr (GMAX <= 8) {
    // matrix-core route: state scan, intra-chunk part, then the state readout
    const oal::LaunchGeom lg = launch_geom(g);
    // the intra-chunk part on the second stream beside the state scan, whose
    // 272 blocks leave most CUs idle (measured with the backward's fork:
    // 3.944-3.953 -> 3.774-3.783 ms per config-2 step)
    if (aux != st) {
      oal::stream_wait(aux, st);
      oal::launch_f32_intra_fwd<T>(lg, qt, kt, vt, labels, c0, lam, gam, groups, scale, num, den, aux, make_timer());
      oal::launch_f32_state_fwd<T>(lg, kt, vt, sv.carry, sv.carry_z, st, make_timer());
      oal::stream_wait(st, aux);
    } else {
      oal::launch_f32_state_fwd<T>(lg, kt, vt, sv.carry, sv.carry_z, st, make_timer());
      oal::launch_f32_intra_fwd<T>(lg, qt, kt, vt, labels, c0, lam, gam, groups, scale, num, den, st, make_timer());
    }
    oal::launch_f32_readout_fwd<T>(lg, qt, sv.wq, sv.carry, sv.carry_z, floor, num, den, static_cast<T*>(out), st,
                                   make_timer());
    return launch_status("oal_forward launch");
  }
  timed("k_state_fwd", st, [&] { hipLaunchKernelGGL(k_state_fwd<T>, dim3(kFP / 16, g.U), dim3(256), 0, st, kt, vt, g.N, g.NB, sv.carry,
                     sv.carry_z); });
  timed("k_out_fwd", st, [&] { hipLaunchKernelGGL((k_out_fwd<T, GMAX>), dim3(g.R, g.NB, g.U), dim3(256), 0, st, qt, kt, vt, sv.wq, sv.carry,
                     sv.carry_z, labels, c0, lam, gam, groups, g.Hq, g.Hkv, g.N, g.NB, scale, floor,
                     static_cast<T*>(out), num, den); });
  return launch_status("oal_forward launch");
}

template <typename T, int GMAX>
int backward_impl(const Geometry& g, const void* q, const void* k, const void* v, const int32_t* labels,
                  const float* c0, const float* lam, const float* gam, int groups, float scale, float floor,
                  const float* num, const float* den, const void* saved, const void* dout, const float* dnum,
                  const float* dden, void* dq, void* dk, void* dv, float* dc0, float* dlam, float* dgam,
                  void* workspace, hipStream_t st, hipStream_t aux) {
  using namespace oal;
  SavedView sv = saved_view(g, const_cast<void*>(saved));
  WorkView w = work_view(g, workspace, GMAX <= 8);
  const T* qt = static_cast<const T*>(q);
  const T* kt = static_cast<const T*>(k);
  const T* vt = static_cast<const T*>(v);
  const long rows = (long)g.B * g.Hq * g.N;
  timed("k_gvec", st, [&] { hipLaunchKernelGGL(k_gvec<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, static_cast<const T*>(dout),
                     dnum, dden, num, den, rows, floor, w.G, w.Gz); });
  const bool need_coef = dc0 || dlam || dgam;
  if constexpr (GMAX <= 8) {
    // matrix-core route
    const oal::LaunchGeom lg = launch_geom(g);
    oal::F32BwdArgs<T> a{qt, kt, vt, w.G, w.Gz, sv.wq, sv.carry, sv.carry_z, labels, c0, lam, gam, groups, scale,
                         w.dT, w.dTz, oal::f32_bwd_plan(g.U, g.NB, g.R), w.segt, w.segtz,
                         need_coef ? w.dwq_part : nullptr, w.dql, w.dkl, w.dvl,
                         need_coef ? w.coefl : nullptr, w.coefs, static_cast<T*>(dq), static_cast<T*>(dk),
                         static_cast<T*>(dv)};
    oal::launch_f32_backward<T>(lg, a, st, aux, make_timer());
    if (need_coef) {
      timed("k_dwq_reduce", st, [&] { hipLaunchKernelGGL(k_dwq_reduce, dim3((kFP + 63) / 64, g.Hq), dim3(1024), 0, st, w.dwq_part, g.B, g.Hq,
                         g.NB, w.dwq); });
      timed("k_coef_grad", st, [&] { hipLaunchKernelGGL(k_coef_grad, dim3(g.Hq), dim3(256), 0, st, w.dwq, labels, groups, scale, dc0, dlam,
                         dgam, w.coefs); });
    }
    // the caller's stream ends after every kernel of the call
    if (aux != st) oal::stream_wait(st, aux);
    return launch_status("oal_backward launch");
  }
  if (dk || dv) {
    timed("k_state_bwd", st, [&] { hipLaunchKernelGGL(k_state_bwd<T>, dim3(kFP / 16, g.U), dim3(256), 0, st, qt, sv.wq, w.G, w.Gz, g.Hq, g.Hkv,
                       g.N, g.NB, w.dT, w.dTz); });
    timed("k_kv_bwd", st, [&] { hipLaunchKernelGGL((k_kv_bwd<T, GMAX>), dim3(g.NB, g.U), dim3(256), 0, st, qt, kt, vt, w.dT, w.dTz, w.G, w.Gz,
                       labels, c0, lam, gam, groups, g.Hq, g.Hkv, g.N, g.NB, scale, static_cast<T*>(dk),
                       static_cast<T*>(dv)); });
  }
  if (dq || need_coef) {
    timed("k_q_bwd", st, [&] { hipLaunchKernelGGL(k_q_bwd<T>, dim3(g.R, g.NB, g.U), dim3(256), 0, st, qt, kt, vt, sv.wq, sv.carry,
                       sv.carry_z, w.G, w.Gz, g.Hq, g.Hkv, g.N, g.NB, static_cast<T*>(dq), w.dwq_part); });
  }
  if (need_coef) {
    timed("k_dwq_reduce", st, [&] { hipLaunchKernelGGL(k_dwq_reduce, dim3((kFP + 63) / 64, g.Hq), dim3(1024), 0, st, w.dwq_part, g.B, g.Hq, g.NB,
                       w.dwq); });
    timed("k_coef_grad", st, [&] { hipLaunchKernelGGL(k_coef_grad, dim3(g.Hq), dim3(256), 0, st, w.dwq, labels, groups, scale, dc0, dlam, dgam); });
  }
  return launch_status("oal_backward launch");
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free backward (oal_backward_noalloc): a file-scope
// device array, one copy per GPU, held until the process ends. Host code never
// passes its name to a kernel (in host code the name is a stand-in, not a
// device address): the address each device holds it at is looked up once per
// device, with that device current, and kept in g_scratch.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[OAL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// The current device's scratch address, or nullptr (with the error set).
void* scratch_address() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    fail("oal_backward_noalloc: no current HIP device");
    return nullptr;
  }
  if (dev >= kMaxDevices) {
    fail("oal_backward_noalloc: device index beyond the supported 64");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      fail(std::string("oal_backward_noalloc: hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(err));
      return nullptr;
    }
    g_scratch[dev] = ptr;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" {

int oal_abi_version(void) { return 2; }

int oal_profile_enable(int enable) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  g_prof_on.store(enable != 0, std::memory_order_release);
  return 0;
}

int oal_profile_collect(char* buf, size_t buflen) {
  std::vector<ProfRecord> recs;
  {
    std::lock_guard<std::mutex> lock(g_prof_mu);
    recs.swap(g_prof_records);
  }
  std::map<std::string, std::pair<long, double>> agg;
  int rc = 0;
  for (auto& r : recs) {
    float ms = 0.f;
    if (hipEventSynchronize(r.stop) != hipSuccess || hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) {
      rc = fail("oal_profile_collect: event timing failed");
    }
    auto& a = agg[r.name];
    a.first += 1;
    a.second += ms;
  }
  {
    std::lock_guard<std::mutex> lock(g_prof_mu);
    for (auto& r : recs) {
      g_prof_pool.push_back(r.start);
      g_prof_pool.push_back(r.stop);
    }
  }
  std::string text;
  for (auto& kv : agg) {
    char line[256];
    snprintf(line, sizeof(line), "%s %ld %.6f\n", kv.first.c_str(), kv.second.first, kv.second.second);
    text += line;
  }
  if (buf && buflen) {
    size_t n = text.size() < buflen - 1 ? text.size() : buflen - 1;
    memcpy(buf, text.data(), n);
    buf[n] = 0;
  }
  return rc;
}

const char* oal_last_error(void) { return g_error.c_str(); }

int oal_feature_count(void) { return oal::kFeat; }

int oal_feature_stride(void) { return oal::kFP; }

int oal_chunk_size(void) { return oal::kC; }

// The kernels move token rows and state tiles with 16-byte loads and stores.
static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int check_common(int groups, int precision) {
  if (groups < 1 || groups > 64) return fail("groups must be in [1, 64]");
  if (precision != OAL_PRECISION_FP32 && precision != OAL_PRECISION_BF16)
    return fail("precision must be OAL_PRECISION_FP32 or OAL_PRECISION_BF16");
  return 0;
}

size_t oal_forward_saved_bytes(int batch, int q_heads, int kv_heads, int seq_len, int groups, int dtype,
                               int precision) {
  Geometry g;
  if (check_geometry(batch, q_heads, kv_heads, seq_len, dtype, &g) || check_common(groups, precision)) return 0;
  if (use_mfma(precision, groups, g)) return oal::mfma_saved_bytes(g.Hq, g.U, g.NB, g.R);
  return saved_bytes(g);
}

size_t oal_backward_workspace_bytes(int batch, int q_heads, int kv_heads, int seq_len, int groups, int dtype,
                                    int precision) {
  Geometry g;
  if (check_geometry(batch, q_heads, kv_heads, seq_len, dtype, &g) || check_common(groups, precision)) return 0;
  if (use_mfma(precision, groups, g))
    return oal::mfma_work_view(nullptr, g.B, g.Hq, g.U, g.N, g.NB, groups > 8).bytes;
  return work_view(g, nullptr, f32_mma(groups)).bytes;
}

int oal_forward(const void* q, const void* k, const void* v, const int32_t* labels, const float* c0,
                const float* lam, const float* gam, int groups, int batch, int q_heads, int kv_heads, int seq_len,
                int dtype, int precision, float scale, float floor, void* out, float* num, float* den, void* saved,
                void* stream) {
  Range range("oal_forward");
  Geometry g;
  if (check_geometry(batch, q_heads, kv_heads, seq_len, dtype, &g)) return 1;
  if (!q || !k || !v || !labels || !c0 || !lam || !gam || !out || !num || !den || !saved)
    return fail("oal_forward: null pointer argument");
  const void* ptrs[] = {q, k, v, num, den, out, saved};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail("oal_forward: tensor pointers must be 16-byte aligned");
  if (check_common(groups, precision)) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_mfma(precision, groups, g)) {
    const oal::LaunchGeom lg = launch_geom(g);
    if (dtype == OAL_DTYPE_F32)
      oal::launch_mfma_forward<float>(lg, q, k, v, labels, c0, lam, gam, groups, scale, floor, out, num, den, saved,
                                      st, make_timer());
    else
      oal::launch_mfma_forward<uint16_t>(lg, q, k, v, labels, c0, lam, gam, groups, scale, floor, out, num, den,
                                         saved, st, make_timer());
    return launch_status("oal_forward launch");
  }
  if (dtype == OAL_DTYPE_F32) {
    if (groups <= 8)
      return forward_impl<float, 8>(g, q, k, v, labels, c0, lam, gam, groups, scale, floor, out, num, den, saved, st, oal::aux_stream(st));
    return forward_impl<float, 64>(g, q, k, v, labels, c0, lam, gam, groups, scale, floor, out, num, den, saved, st, st);
  }
  if (groups <= 8)
    return forward_impl<uint16_t, 8>(g, q, k, v, labels, c0, lam, gam, groups, scale, floor, out, num, den, saved, st, oal::aux_stream(st));
  return forward_impl<uint16_t, 64>(g, q, k, v, labels, c0, lam, gam, groups, scale, floor, out, num, den, saved, st, st);
}

}  // extern "C"

namespace {

// The backward of both entry points; may_fork: the matrix-core path may put
// independent kernels on the device's second stream (the allocation-free entry
// point keeps every kernel on the caller's stream).
int backward_entry(const void* q, const void* k, const void* v, const int32_t* labels, const float* c0,
                   const float* lam, const float* gam, int groups, int batch, int q_heads, int kv_heads, int seq_len,
                   int dtype, int precision, float scale, float floor, const float* num, const float* den,
                   const void* saved, const void* dout, const float* dnum, const float* dden, void* dq, void* dk,
                   void* dv, float* dc0, float* dlam, float* dgam, void* workspace, void* stream, bool may_fork) {
  Range range("oal_backward");
  Geometry g;
  if (check_geometry(batch, q_heads, kv_heads, seq_len, dtype, &g)) return 1;
  if (!q || !k || !v || !labels || !c0 || !lam || !gam || !num || !den || !saved || !workspace)
    return fail("oal_backward: null pointer argument");
  const void* ptrs[] = {q, k, v, num, den, saved, workspace, dout, dnum, dden, dq, dk, dv};
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return fail("oal_backward: tensor pointers must be 16-byte aligned");
  if (check_common(groups, precision)) return 1;
  // argument combinations the kernels cannot serve are refused before anything is enqueued
  if ((dc0 || dlam || dgam) && !(dc0 && dlam && dgam)) return fail("dc0, dlam and dgam must be given together");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_mfma(precision, groups, g)) {
    if ((dk != nullptr) != (dv != nullptr))
      return fail("oal_backward: dk and dv must be requested together on the matrix-core path");
    const oal::LaunchGeom lg = launch_geom(g);
    const hipStream_t aux = may_fork ? oal::aux_stream(st) : st;
    int rc;
    if (dtype == OAL_DTYPE_F32)
      rc = oal::launch_mfma_backward<float>(lg, q, k, v, labels, c0, lam, gam, groups, scale, floor, num, den, saved,
                                            dout, dnum, dden, dq, dk, dv, dc0, dlam, dgam, workspace, st, aux,
                                            make_timer());
    else
      rc = oal::launch_mfma_backward<uint16_t>(lg, q, k, v, labels, c0, lam, gam, groups, scale, floor, num, den,
                                               saved, dout, dnum, dden, dq, dk, dv, dc0, dlam, dgam, workspace, st,
                                               aux, make_timer());
    if (rc == 2) return fail("oal_backward: dk and dv must be requested together on the matrix-core path");
    if (rc == 3) return fail("dc0, dlam and dgam must be given together");
    return launch_status("oal_backward launch");
  }
#define OAL_BWD_ARGS                                                                                       \
  g, q, k, v, labels, c0, lam, gam, groups, scale, floor, num, den, saved, dout, dnum, dden, dq, dk, dv, dc0, \
      dlam, dgam, workspace, st
  // the fp32 matrix-core route (up to 8 groups) may fork like the bf16 path;
  // the scalar kernels for more groups run on the caller's stream
  const hipStream_t aux8 = may_fork ? oal::aux_stream(st) : st;
  if (dtype == OAL_DTYPE_F32) {
    if (groups <= 8) return backward_impl<float, 8>(OAL_BWD_ARGS, aux8);
    return backward_impl<float, 64>(OAL_BWD_ARGS, st);
  }
  if (groups <= 8) return backward_impl<uint16_t, 8>(OAL_BWD_ARGS, aux8);
  return backward_impl<uint16_t, 64>(OAL_BWD_ARGS, st);
#undef OAL_BWD_ARGS
}

}  // namespace

extern "C" {

int oal_backward(const void* q, const void* k, const void* v, const int32_t* labels, const float* c0,
                 const float* lam, const float* gam, int groups, int batch, int q_heads, int kv_heads, int seq_len,
                 int dtype, int precision, float scale, float floor, const float* num, const float* den,
                 const void* saved, const void* dout, const float* dnum, const float* dden, void* dq, void* dk,
                 void* dv, float* dc0, float* dlam, float* dgam, void* workspace, void* stream) {
  return backward_entry(q, k, v, labels, c0, lam, gam, groups, batch, q_heads, kv_heads, seq_len, dtype, precision,
                        scale, floor, num, den, saved, dout, dnum, dden, dq, dk, dv, dc0, dlam, dgam, workspace,
                        stream, true);
}

int oal_backward_noalloc(const void* q, const void* k, const void* v, const int32_t* labels, const float* c0,
                         const float* lam, const float* gam, int groups, int batch, int q_heads, int kv_heads,
                         int seq_len, int dtype, int precision, float scale, float floor, const float* num,
                         const float* den, const void* saved, const void* dout, const float* dnum, const float* dden,
                         void* dq, void* dk, void* dv, float* dc0, float* dlam, float* dgam, void* stream) {
  const size_t need = oal_backward_workspace_bytes(batch, q_heads, kv_heads, seq_len, groups, dtype, precision);
  if (need == 0) return 1;  // invalid geometry; the size query set the error
  if (need > (size_t)OAL_NOALLOC_SCRATCH_BYTES) {
    char msg[256];
    snprintf(msg, sizeof(msg),
             "oal_backward_noalloc: this geometry needs %zu bytes of workspace; the static scratch holds %zu "
             "(use oal_backward with a caller-allocated workspace)",
             need, (size_t)OAL_NOALLOC_SCRATCH_BYTES);
    return fail(msg);
  }
  // the stream must run on the current device, whose scratch copy is used
  if (stream) {
    int sdev = -1, cur = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess || hipGetDevice(&cur) != hipSuccess)
      return fail("oal_backward_noalloc: cannot resolve the stream's device");
    if (sdev != cur) return fail("oal_backward_noalloc: the stream must belong to the current device");
  }
  void* ws = scratch_address();
  if (!ws) return 1;
  // every workspace byte the backward reads it has written first in the same
  // call, so the scratch needs no clearing between calls; every kernel stays
  // on the caller's stream (no second stream or event is created)
  return backward_entry(q, k, v, labels, c0, lam, gam, groups, batch, q_heads, kv_heads, seq_len, dtype, precision,
                        scale, floor, num, den, saved, dout, dnum, dden, dq, dk, dv, dc0, dlam, dgam, ws, stream,
                        false);
}

int oal_selftest(int* device_errors, void* stream) {
  if (!device_errors) return fail("oal_selftest: null pointer argument");
  if (oal::run_mfma_selftest(device_errors, static_cast<hipStream_t>(stream)))
    return fail("oal_selftest: launch failed");
  return 0;
}


// FP64 route. Geometry checks as the other entry points (any group count in
// [1, 64]); the kernels are in oal_f64.hip.
static int check_f64(int groups, int batch, int q_heads, int kv_heads, int seq_len, oal::F64Geom* g) {
  Geometry geo;
  if (check_geometry(batch, q_heads, kv_heads, seq_len, OAL_DTYPE_F32, &geo)) return 1;
  if (groups < 1 || groups > 64) return fail("groups must be in [1, 64]");
  const long tiles = (seq_len + 31) / 32;
  if (tiles > 65535 || (long)batch * q_heads > 65535) return fail("grid too large");
  *g = oal::F64Geom{batch, q_heads, kv_heads, seq_len};
  return 0;
}

int oal_forward_f64(const double* q, const double* k, const double* v, const int32_t* labels, const double* c0,
                    const double* lam, const double* gam, int groups, int batch, int q_heads, int kv_heads,
                    int seq_len, double scale, double* out, double* num, double* den, void* stream) {
  Range range("oal_forward_f64");
  oal::F64Geom g;
  if (check_f64(groups, batch, q_heads, kv_heads, seq_len, &g)) return 1;
  if (!q || !k || !v || !labels || !c0 || !lam || !gam || !out || !num || !den)
    return fail("oal_forward_f64: null pointer argument");
  const void* ptrs[] = {q, k, v, out, num, den};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail("oal_forward_f64: tensor pointers must be 16-byte aligned");
  oal::launch_f64_forward(g, q, k, v, labels, c0, lam, gam, groups, scale, out, num, den,
                          static_cast<hipStream_t>(stream), make_timer());
  return launch_status("oal_forward_f64 launch");
}

size_t oal_backward_f64_workspace_bytes(int batch, int q_heads, int kv_heads, int seq_len, int groups) {
  oal::F64Geom g;
  if (check_f64(groups, batch, q_heads, kv_heads, seq_len, &g)) return 0;
  return oal::f64_workspace_bytes(g.B, g.Hq, g.N);
}

int oal_backward_f64(const double* q, const double* k, const double* v, const int32_t* labels, const double* c0,
                     const double* lam, const double* gam, int groups, int batch, int q_heads, int kv_heads,
                     int seq_len, double scale, const double* num, const double* den, const double* dout,
                     const double* dnum, const double* dden, double* dq, double* dk, double* dv, double* dc0,
                     double* dlam, double* dgam, void* workspace, void* stream) {
  Range range("oal_backward_f64");
  oal::F64Geom g;
  if (check_f64(groups, batch, q_heads, kv_heads, seq_len, &g)) return 1;
  if (!q || !k || !v || !labels || !c0 || !lam || !gam || !num || !den || !workspace)
    return fail("oal_backward_f64: null pointer argument");
  const void* ptrs[] = {q, k, v, num, den, dout, dnum, dden, dq, dk, dv, workspace};
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return fail("oal_backward_f64: tensor pointers must be 16-byte aligned");
  if ((dc0 || dlam || dgam) && !(dc0 && dlam && dgam)) return fail("dc0, dlam and dgam must be given together");
  oal::launch_f64_backward(g, q, k, v, labels, c0, lam, gam, groups, scale, num, den, dout, dnum, dden, dq, dk, dv,
                           dc0, dlam, dgam, workspace, static_cast<hipStream_t>(stream), make_timer());
  return launch_status("oal_backward_f64 launch");
}

}  // extern "C"
