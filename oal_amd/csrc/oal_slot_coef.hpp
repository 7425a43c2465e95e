// Per-head slot coefficients of the bf16 (matrix-core) kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"

namespace oal {

// Per-head coefficients, one of 8 parts of query head h per 256-thread block
// (k2_fwd_prep runs them in blocks of their own):
//   wqs[h][slot]  wq of natural feature nat(slot) (0 for invalid slots);
//   ic[h]         c0, scale*lam[g], scale^2*Gam[g][g'] padded to 8 groups (the
//                 group-sum intra-chunk kernels; G > 8 keeps only c0);
//   gm[h][r][c]   scale^2 * Gam[g(r)][g(c)]  (denominator quadratic form);
//   lb[h][d]      scale * lam[g(d)].
// Any group count up to 64: labels d -> d with G = 64 gives per-pair coefficients.
// tab: the translation unit's constant-memory slot table.
__device__ __forceinline__ void slot_coefficients_part(const SlotTable& tab, const SlotCoefArgs& a, int h, int part) {
  const int32_t* __restrict__ labels = a.labels;
  const float* __restrict__ c0 = a.c0;
  const float* __restrict__ lam = a.lam;
  const float* __restrict__ gam = a.gam;
  const int G = a.G;
  const float scale = a.scale;
  float* __restrict__ wqs = a.wqs;
  float* __restrict__ ic = a.ic;
  float* __restrict__ gm = a.gm;
  float* __restrict__ lb = a.lb;
  // the head's coefficients are read once into LDS; every output then comes
  // from LDS (no dependent global gathers)
  __shared__ int lab[kD];
  __shared__ float cg[kD * kD], cl[kD], cc;
  // block (h, part): slots and gm rows of one eighth; part 0 also writes ic, lb
  const int t = threadIdx.x;
  if (t < kD) {
    const int g = labels[h * kD + t];
    lab[t] = g < 0 ? 0 : (g >= G ? G - 1 : g);
  }
  for (int e = t; e < G * G; e += blockDim.x) cg[e] = scale * scale * gam[(size_t)h * G * G + e];
  if (t < G) cl[t] = scale * lam[(size_t)h * G + t];
  if (t == 0) cc = c0[h];
  __syncthreads();
  constexpr int kSlotsPerPart = kS / 8;
  static_assert(kSlotsPerPart * 8 == kS, "slot parts");
  for (int s = part * kSlotsPerPart + t; s < (part + 1) * kSlotsPerPart; s += blockDim.x) {
    const int n = tab.nat[s];
    const int r = tab.ar[s], c = tab.ac[s];
    float w = 0.f;
    if (n == 0) {
      w = cc;
    } else if (n > 0 && n <= kD) {
      w = cl[lab[r]];
    } else if (n > kD) {
      w = (r == c ? 1.f : 2.f) * cg[lab[r] * G + lab[c]];
    }
    wqs[(size_t)h * kS + s] = w;
  }
  if (part == 0 && t < kIC) {
    float x = 0.f;
    if (t == 0) {
      x = cc;
    } else if (G <= 8 && t < kIcGam) {
      x = t - kIcLam < G ? cl[t - kIcLam] : 0.f;
    } else if (G <= 8 && t < kIcGam + 64) {
      const int g = (t - kIcGam) >> 3, g2 = (t - kIcGam) & 7;
      x = (g < G && g2 < G) ? cg[g * G + g2] : 0.f;
    }
    ic[(size_t)h * kIC + t] = x;
  }
  for (int e = part * (kD * kD / 8) + t; e < (part + 1) * (kD * kD / 8); e += blockDim.x) {
    const int r = e >> 6, c = e & 63;
    gm[(size_t)h * kD * kD + e] = cg[lab[r] * G + lab[c]];
  }
  if (part == 0 && t < kD) lb[(size_t)h * kD + t] = cl[lab[t]];
}

}  // namespace oal
