// Shared constants, the feature table and small device helpers for the OAL
// grouped quadratic attention kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oal {

// Head and value dimension handled by the kernels (callers pad smaller ones).
constexpr int kD = 64;
// A token row in LDS holds [x_0 .. x_63, 1, 0] so that every feature is the
// product x[r] * x[c] of two row entries (see FeatureTable).
constexpr int kRow = 66;
// Logical features: 1 constant + 64 linear + 64*65/2 pairs.
constexpr int kFeat = 1 + kD + kD * (kD + 1) / 2;  // 2145
// Padded feature stride of every per-feature buffer (multiple of 64).
constexpr int kFP = 2176;
// Token block (chunk).
constexpr int kC = 64;
// Feature tile staged through LDS.
constexpr int kTile = 64;

// Feature f is raw(x)[f] = x[r[f]] * x[c[f]] on a row [x_0..x_63, 1, 0]:
//   f = 0                 constant     (r, c) = (64, 64)
//   f = 1 + d             linear x_d   (r, c) = (d, 64)
//   f = 65 + r(r+1)/2 + c pair x_r x_c (r >= c), the reference pair order
//                         (grouped_reference.py:8-15, hd_block_gemm_cache.py:105-121)
//   f >= 2145             padding 0    (r, c) = (65, 65)
struct FeatureTable {
  uint8_t r[kFP];
  uint8_t c[kFP];
};

constexpr FeatureTable make_feature_table() {
  FeatureTable t{};
  t.r[0] = 64;
  t.c[0] = 64;
  for (int d = 0; d < kD; ++d) {
    t.r[1 + d] = static_cast<uint8_t>(d);
    t.c[1 + d] = 64;
  }
  int f = 1 + kD;
  for (int r = 0; r < kD; ++r) {
    for (int c = 0; c <= r; ++c) {
      t.r[f] = static_cast<uint8_t>(r);
      t.c[f] = static_cast<uint8_t>(c);
      ++f;
    }
  }
  for (; f < kFP; ++f) {
    t.r[f] = 65;
    t.c[f] = 65;
  }
  return t;
}

// Storage conversion. bf16 travels as its 16 raw bits.
__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }

template <typename T>
__device__ __forceinline__ T from_f(float x);

template <>
__device__ __forceinline__ float from_f<float>(float x) {
  return x;
}

// Round to nearest even; NaN stays a quiet NaN.
template <>
__device__ __forceinline__ uint16_t from_f<uint16_t>(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Per-head group structure staged in LDS for the intra-chunk term.
// perm lists the dimensions sorted by group; group g owns perm[gstart[g] ..
// gstart[g+1]).  gam is stored [g][h] with row stride G.
template <int GMAX>
struct HeadGroups {
  int lab[kD];
  int perm[kD];
  int gstart[GMAX + 1];
  float lam[GMAX];
  float gam[GMAX * GMAX];
  float c0;
};

// Loads one head's groups and coefficients; every thread of the block must
// call it. Labels are clamped into [0, G) so that a bad label cannot index
// out of bounds (the host validates them before calling).
template <int GMAX>
__device__ void load_head_groups(HeadGroups<GMAX>& hg, const int32_t* __restrict__ labels,
                                 const float* __restrict__ c0, const float* __restrict__ lam,
                                 const float* __restrict__ gam, int G, int h) {
  const int t = threadIdx.x;
  __syncthreads();
  if (t < kD) {
    int g = labels[h * kD + t];
    hg.lab[t] = g < 0 ? 0 : (g >= G ? G - 1 : g);
  }
  for (int i = t; i < G * G; i += blockDim.x) hg.gam[i] = gam[(size_t)h * G * G + i];
  if (t < G) hg.lam[t] = lam[(size_t)h * G + t];
  if (t == 0) hg.c0 = c0[h];
  __syncthreads();
  if (t < kD) {
    const int g = hg.lab[t];
    int pos = 0;
    for (int d = 0; d < kD; ++d) {
      const int gd = hg.lab[d];
      pos += (gd < g) | ((gd == g) & (d < t));
    }
    hg.perm[pos] = t;
  }
  if (t <= G) {
    int cnt = 0;
    for (int d = 0; d < kD; ++d) cnt += hg.lab[d] < t;
    hg.gstart[t] = cnt;
  }
  __syncthreads();
}

// s_g = scale * sum_{d in g} q[d] k[d]
template <int GMAX>
__device__ __forceinline__ void group_sums(const HeadGroups<GMAX>& hg, int G, const float* qrow,
                                           const float* krow, float scale, float (&s)[GMAX]) {
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    float acc = 0.f;
    if (g < G) {
      const int p1 = hg.gstart[g + 1];
      for (int p = hg.gstart[g]; p < p1; ++p) {
        const int d = hg.perm[p];
        acc += qrow[d] * krow[d];
      }
    }
    s[g] = acc * scale;
  }
}

// kappa = c0 + sum_g s_g (lam_g + sum_h gam_gh s_h)
template <int GMAX>
__device__ __forceinline__ float kappa_of(const HeadGroups<GMAX>& hg, int G, const float (&s)[GMAX]) {
  float kap = hg.c0;
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g < G) {
      float inner = hg.lam[g];
#pragma unroll
      for (int h = 0; h < GMAX; ++h) {
        if (h < G) inner += hg.gam[g * G + h] * s[h];
      }
      kap += s[g] * inner;
    }
  }
  return kap;
}

// d kappa / d s_g = lam_g + 2 sum_h gam_gh s_h   (gam symmetric)
template <int GMAX>
__device__ __forceinline__ float kappa_grad(const HeadGroups<GMAX>& hg, int G, int g, const float (&s)[GMAX]) {
  float acc = 0.f;
  const float* row = hg.gam + g * G;
#pragma unroll
  for (int h = 0; h < GMAX; ++h) {
    if (h < G) acc += row[h] * s[h];
  }
  return hg.lam[g] + 2.f * acc;
}

}  // namespace oal
