// Fold helpers shared by the query- and key-side VJP kernels (gfx950): a
// matrix-core product whose output holds 16 feature slots of one token per lane
// (lane column = token, registers = slots of a 32-slot M-tile in the fold row
// order) is folded through that token's rotated row into its gradient:
// dx[rb] += d x[cb], dx[cb] += d x[rb] for the base (rb, cb) of each slot.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "oal_mfma_common.hpp"

namespace oal {
namespace fold {

constexpr int LD = kD + 8;  // padded bf16 row stride in LDS

// 32 consecutive elements of a row (16-byte stores).
__device__ __forceinline__ void store32(float* dst, const float (&v)[32]) {
#pragma unroll
  for (int j = 0; j < 8; ++j)
    reinterpret_cast<float4*>(dst)[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
}
__device__ __forceinline__ void store32(uint16_t* dst, const float (&v)[32]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = uint32_t(from_f<uint16_t>(v[8 * j + 2 * i])) | (uint32_t(from_f<uint16_t>(v[8 * j + 2 * i + 1])) << 16);
    reinterpret_cast<uint4*>(dst)[j] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// 8 consecutive elements of a row as one bf16 fragment (zeros when !ok).
__device__ __forceinline__ bf16x8 frag8(const uint16_t* __restrict__ src, size_t off, bool ok) {
  const bf16x8 x = *reinterpret_cast<const bf16x8*>(src + off);
  return ok ? x : bf16x8{};
}
__device__ __forceinline__ bf16x8 frag8(const float* __restrict__ src, size_t off, bool ok) {
  const float4 a = reinterpret_cast<const float4*>(src + off)[0], b = reinterpret_cast<const float4*>(src + off)[1];
  float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const bf16x8 x = pack8(v);
  return ok ? x : bf16x8{};
}

// Rotated fp32 row x[m] = row[(m + 32 s) % 64], loaded in rotated order (the
// rotation is in the per-lane addresses, so every register index is static).
template <typename T>
__device__ __forceinline__ void load_rotated(const T* __restrict__ src, size_t row_base, bool ok, int s,
                                             float (&x)[kD]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bf16x8 r = frag8(src, row_base + ((8 * i + 32 * s) & 63), ok);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[8 * i + j] = (float)r[j];
  }
}


// Slot weights of M-tile M for this lane's rows (16 values), from LDS.
template <int M, bool WEIGHTED>
__device__ __forceinline__ void fold_weights(const float* wl, int s, float (&w16)[16]) {
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    if constexpr (WEIGHTED) {
      const float4 ww = *reinterpret_cast<const float4*>(wl + 16 * (2 * M + a / 2) + 8 * s + 4 * (a % 2));
      w16[4 * a + 0] = ww.x;
      w16[4 * a + 1] = ww.y;
      w16[4 * a + 2] = ww.z;
      w16[4 * a + 3] = ww.w;
    } else {
      w16[4 * a + 0] = w16[4 * a + 1] = w16[4 * a + 2] = w16[4 * a + 3] = 1.f;
    }
  }
}

// Slot weights of M-tile M in one register: lane j of each 16-lane row holds
// the weight of accumulator register j of the row's lane group s (slot
// 32 M + 16 (j / 8) + 8 s + j % 8), for fold_tile_row.
template <int M>
__device__ __forceinline__ float fold_weight_row(const float* wl, int lane) {
  const int j = lane & 15, s = lane >> 5;
  return wl[32 * M + 16 * (j >> 3) + 8 * s + (j & 7)];
}

// Fold of one 32-slot M-tile (rows permuted so that the rows a lane holds are
// slots of its rotation group): dx[rb] += d x[cb], dx[cb] += d x[rb].
template <int M>
__device__ __forceinline__ void fold_tile(const f32x16& D, const float (&x)[kD], float (&dx)[kD],
                                          const float (&w16)[16]) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (([&] {
       constexpr int a = I / 4, v = I % 4;
       constexpr int base = 8 * (2 * M + a / 2) + 4 * (a % 2) + v;
       constexpr int rb = kSlotHost.rb[base], cb = kSlotHost.cb[base];
       const float d = D[I] * w16[I];
       if constexpr (rb < 64 && cb < 64) {
         dx[rb] += d * x[cb];
         dx[cb] += d * x[rb];
       } else if constexpr (rb < 64 && cb == 64) {
         dx[rb] += d;
       }
     }()),
     ...);
  }(std::make_integer_sequence<int, 16>{});
}

// fold_tile with the slot weights of fold_weight_row.
template <int M>
__device__ __forceinline__ void fold_tile_row(const f32x16& D, const float (&x)[kD], float (&dx)[kD], float wrow) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (([&] {
       constexpr int a = I / 4, v = I % 4;
       constexpr int base = 8 * (2 * M + a / 2) + 4 * (a % 2) + v;
       constexpr int rb = kSlotHost.rb[base], cb = kSlotHost.cb[base];
       const float d = D[I] * row_bcast<I>(wrow);
       if constexpr (rb < 64 && cb < 64) {
         dx[rb] += d * x[cb];
         dx[cb] += d * x[rb];
       } else if constexpr (rb < 64 && cb == 64) {
         dx[rb] += d;
       }
     }()),
     ...);
  }(std::make_integer_sequence<int, 16>{});
}

// A-operand rows of M-tile: lane row r = 8a + 4s' + v reads within-tile slot
// 16(a/2) + 8s' + 4(a%2) + v of the PR tile (32 slots x 16 values per unit).
__device__ __forceinline__ int fold_row(int r) {
  const int a = r >> 3, sp = (r >> 2) & 1, v = r & 3;
  return 16 * (a >> 1) + 8 * sp + 4 * (a & 1) + v;
}

// The two rotation groups of a token (lanes l and l + 32) hold its gradient
// in rotated order: lane group s has dimension (m + 32 s) % 64 at index m.
// Returns, in lane group s, the full gradient of dimensions 32 s + m (m < 32).
__device__ __forceinline__ void combine_rotation_groups(const float (&dx)[kD], int s, float (&out)[32]) {
#pragma unroll
  for (int m = 0; m < 32; ++m) {
    // partner's dx[m + 32]: lanes < 32 receive it in the second result,
    // lanes >= 32 in the first
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(dx[m + 32]), __float_as_uint(dx[m + 32]),
                                                    false, false);
    out[m] = dx[m] + __uint_as_float(s ? r[0] : r[1]);
  }
}

// Rows of the Mz operand for the Z^T = Mz K^T products: product md, accumulator
// row m = 8 a + 4 s + v (lane group s, register 4 a + v) holds dimension
// 32 s + 16 md + 4 a + v, so that lane group s ends up with dimensions
// 32 s .. 32 s + 31 of its token (registers 16 md + i), the layout of the fold.
__device__ __forceinline__ int mz_dim(int md, int m) {
  const int a = m >> 3, sg = (m >> 2) & 1, v = m & 3;
  return 32 * sg + 16 * md + 4 * a + v;
}

}  // namespace fold
}  // namespace oal
