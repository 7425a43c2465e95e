// Feature-form (per-pair coefficient) intra-chunk VJP on the gfx950 matrix cores.
//
// With more than 8 dimension groups -- the reference HD Function's logical
// per-pair coefficients are labels d -> d with 64 groups -- the local score of
// query token i and key token j of one chunk is
//   kappa(i, j) = sum_slot raw(q_i)[slot] wq[slot] raw(k_j)[slot]
// (phi_Q . phi_K^T, reference hd_block_gemm_runtime.py:530-540; the forward
// forms it in k2_intra_fwd<T, true>). Its VJP with ds(i, j) = g_i . v_j + gz_i
// (j <= i, g and gz from the normalization VJP) is, as in
// hd_block_gemm_backward_wave.py:253-477,
//   dphi_Q(i) = sum_j ds(i, j) raw(k_j),  dphi_K(j) = sum_i ds(i, j) wq o raw(q_i),
// folded through the features into dq and dk, and the local slot-coefficient
// gradient  dwq[slot] += sum_ij ds(i, j) raw(q_i)[slot] raw(k_j)[slot].
//
// k2p_local_dq   one block per (query head, chunk), two waves (query tiles):
//                D^T[slot][i] = sum_j raw(k_j)[slot] ds(i, j) on the matrix cores
//                (A: key features of the lane's slot from the chunk's k^T rows
//                staged in LDS; B: ds as K-major fragments built from the
//                accumulators of ds^T = V G^T), folded through q_i with the slot
//                weights; the coefficient partials from the same D; plus the
//                denominator state's dq, gz_i (bz + 2 Mz q_i).
// k2p_local_dk   one block per (query head, chunk), two waves (key tiles):
//                D^T[slot][j] = sum_i wq[slot] raw(q_i)[slot] ds(i, j), folded
//                through k_j: a per-head dk partial.
// k2p_dk_reduce  the per-head partials summed over the unit's heads, fixed order.
// k2p_coef_grad  per head: slot gradients (state + local, and the denominator's
//                natural-order partials) -> dc0, dlam, dGam for any group count.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"
#include "oal_mfma_fold.hpp"

namespace oal {

static __constant__ SlotTable kSlot = make_slot_table();
using namespace fold;

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPRow = kC + 4;   // fp32 LDS row stride of a staged transposed operand
constexpr int kPRows = kD + 2;  // rows 0..63 the operand, 64 = one, 65 = zero
constexpr int kERow = 36;       // LDS row stride of the coefficient-partial transpose

// K-step t (rows 16 t .. 16 t + 15) of a 32-row accumulator tile as an MFMA
// operand whose K index is the accumulator row: lane group s must hold rows
// 16 t + 8 s .. + 7; the accumulator gives it rows 16 t + 4 s + (0..3) and
// 16 t + 8 + 4 s + (0..3), so one quad is exchanged with the other lane group.
__device__ __forceinline__ bf16x8 acc_kfrag(const float (&x)[16], int t, int s) {
  const uint32_t a0 = pack_bf16x2(x[8 * t + 0], x[8 * t + 1]);
  const uint32_t a1 = pack_bf16x2(x[8 * t + 2], x[8 * t + 3]);
  const uint32_t b0 = pack_bf16x2(x[8 * t + 4], x[8 * t + 5]);
  const uint32_t b1 = pack_bf16x2(x[8 * t + 6], x[8 * t + 7]);
  const uint32_t r0 = __shfl_xor(s ? a0 : b0, 32, 64);
  const uint32_t r1 = __shfl_xor(s ? a1 : b1, 32, 64);
  const u32x4 fr = s ? u32x4{r0, r1, b0, b1} : u32x4{a0, a1, r0, r1};
  return __builtin_bit_cast(bf16x8, fr);
}

// 8 consecutive elements of a row as a bf16 fragment (zeros when !ok).
__device__ __forceinline__ bf16x8 row8(const uint16_t* __restrict__ p, bool ok) {
  const bf16x8 x = *reinterpret_cast<const bf16x8*>(p);
  return ok ? x : bf16x8{};
}
__device__ __forceinline__ bf16x8 row8(const float* __restrict__ p, bool ok) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const bf16x8 x = pack8(v);
  return ok ? x : bf16x8{};
}

// Raw features of the 16 registers of M-tile M (fold order) on a rotated row.
template <int M>
__device__ __forceinline__ void fold_raw(const float (&x)[kD], float (&r16)[16]) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    ((r16[I] = base_value<8 * (2 * M + (I / 4) / 2) + 4 * ((I / 4) % 2) + I % 4>(x)), ...);
  }(std::make_integer_sequence<int, 16>{});
}

// The 8 features of slot rows (ar, ac) on tokens tok .. tok + 7 of a transposed
// operand staged in LDS, times w: the A fragment of this lane's slot row.
__device__ __forceinline__ bf16x8 lds_feature(const float* P, int ar, int ac, int tok, float w) {
  const float4* pa = reinterpret_cast<const float4*>(P + ar * kPRow + tok);
  const float4* pc = reinterpret_cast<const float4*>(P + ac * kPRow + tok);
  const float4 a0 = pa[0], a1 = pa[1], c0 = pc[0], c1 = pc[1];
  float f[8] = {a0.x * c0.x * w, a0.y * c0.y * w, a0.z * c0.z * w, a0.w * c0.w * w,
                a1.x * c1.x * w, a1.y * c1.y * w, a1.z * c1.z * w, a1.w * c1.w * w};
  return pack8(f);
}

// Stages rows 0 .. rows-1 of a transposed bf16 operand ([row][NB * 64] tokens,
// chunk ch) as fp32 rows of P; rows past `rows` up to 64 are left alone.
__device__ __forceinline__ void stage_rows(float* P, const uint16_t* __restrict__ src, size_t np, int tok0, int rows,
                                           int tid, int nthreads) {
  for (int idx = tid; idx < rows * 8; idx += nthreads) {
    const int r = idx >> 3, c8 = idx & 7;
    const u32x4 w = *reinterpret_cast<const u32x4*>(src + (size_t)r * np + tok0 + 8 * c8);
    float4* d = reinterpret_cast<float4*>(P + r * kPRow + 8 * c8);
    d[0] = make_float4(__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                       __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u));
    d[1] = make_float4(__uint_as_float(w[2] << 16), __uint_as_float(w[2] & 0xffff0000u),
                       __uint_as_float(w[3] << 16), __uint_as_float(w[3] & 0xffff0000u));
  }
}

// The slot table's row pair (ar, ac) of every slot, and the head's slot weights.
__device__ __forceinline__ void stage_slots(uint8_t* sar, uint8_t* sac, float* wl, const float* __restrict__ wqs,
                                            int h, int tid, int nthreads) {
  for (int i = tid; i < kS; i += nthreads) {
    sar[i] = kSlot.ar[i];
    sac[i] = kSlot.ac[i];
  }
  if (wl) {
    for (int i = tid; i < kS / 4; i += nthreads)
      reinterpret_cast<float4*>(wl)[i] = reinterpret_cast<const float4*>(wqs + (size_t)h * kS)[i];
  }
}

// ---------------------------------------------------------------------------
// k2p_local_dq: M-tile M of one wave (query tile), NKB k-blocks of 16 key tokens.
// ---------------------------------------------------------------------------
template <int NKB, bool COEF, int M>
__device__ __forceinline__ void pdq_tile(const float* Kf, const uint8_t* sar, const uint8_t* sac, float wrow,
                                         const bf16x8 (&bds)[4], const float (&x)[kD], float (&dx)[kD], int lane,
                                         float* Ered, float* __restrict__ coef_out) {
  const int s = lane >> 5, row = lane & 31;
  const int slot = 32 * M + fold_row(row);
  const int ar = sar[slot], ac = sac[slot];
  f32x16 D = f32x16{};
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) D = mfma32(lds_feature(Kf, ar, ac, 16 * kb + 8 * s, 1.f), bds[kb], D);
  if constexpr (COEF) {
    // partial of slot 32 M + r: sum over this wave's 32 query tokens of
    // raw(q_i)[slot] D[slot][i], transposed through LDS (row = slot row,
    // column = token), each row summed in a fixed order
    float r16[16];
    fold_raw<M>(x, r16);
#pragma unroll
    for (int I = 0; I < 16; ++I) Ered[fold_row(c32_row(I, lane)) * kERow + row] = D[I] * r16[I];
    __builtin_amdgcn_wave_barrier();
    const float4* er = reinterpret_cast<const float4*>(Ered + row * kERow + 16 * s);
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 e = er[c];
      acc += (e.x + e.y) + (e.z + e.w);
    }
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
    if (s == 0) coef_out[32 * M + row] = acc + __uint_as_float(r[1]);
    __builtin_amdgcn_wave_barrier();
  }
  fold_tile_row<M>(D, x, dx, wrow);
}

// The slot weights of each M-tile (one register per lane, fold_weight_row)
// come from global memory (L2), read two M-tiles ahead.
template <int NKB, bool COEF, int... Ms>
__device__ __forceinline__ void pdq_all_impl(const float* Kf, const uint8_t* sar, const uint8_t* sac,
                                             const float* __restrict__ wg, const bf16x8 (&bds)[4],
                                             const float (&x)[kD], float (&dx)[kD], int lane, float* Ered,
                                             float* coef_out, std::integer_sequence<int, Ms...>) {
  constexpr int NT = kS / 32;
  float w0 = fold_weight_row<0>(wg, lane), w1 = fold_weight_row<1>(wg, lane);
  ((pin64(dx), [&] {
     const float wc = w0;
     w0 = w1;
     if constexpr (Ms + 2 < NT) w1 = fold_weight_row<Ms + 2>(wg, lane);
     pdq_tile<NKB, COEF, Ms>(Kf, sar, sac, wc, bds, x, dx, lane, Ered, coef_out);
   }()),
   ...);
}

// ---------------------------------------------------------------------------
// k2p_local_dk: M-tile M of one wave (key tile), NKB k-blocks of 16 query tokens
// starting at query token i0 of the chunk.
// ---------------------------------------------------------------------------
template <int NKB, int M>
__device__ __forceinline__ void pdk_tile(const float* Qf, const uint8_t* sar, const uint8_t* sac, const float* wl,
                                         const bf16x8 (&bds)[4], int i0, const float (&x)[kD], float (&dx)[kD],
                                         int lane) {
  const int s = lane >> 5, row = lane & 31;
  const int slot = 32 * M + fold_row(row);
  const int ar = sar[slot], ac = sac[slot];
  const float w = wl[slot];
  f32x16 D = f32x16{};
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) D = mfma32(lds_feature(Qf, ar, ac, i0 + 16 * kb + 8 * s, w), bds[kb], D);
  float ones[16];
  fold_weights<M, false>(nullptr, s, ones);
  fold_tile<M>(D, x, dx, ones);
}

template <int NKB, int... Ms>
__device__ __forceinline__ void pdk_all_impl(const float* Qf, const uint8_t* sar, const uint8_t* sac, const float* wl,
                                             const bf16x8 (&bds)[4], int i0, const float (&x)[kD], float (&dx)[kD],
                                             int lane, std::integer_sequence<int, Ms...>) {
  ((pin64(dx), pdk_tile<NKB, Ms>(Qf, sar, sac, wl, bds, i0, x, dx, lane)), ...);
}

}  // namespace

// ---------------------------------------------------------------------------
// dq local part (feature form) + denominator-state dq, one block per (query
// head, chunk), grid R * NB * U (XCD-ordered), 2 waves = query tiles.
// COEF: also the local slot-coefficient partials, one row per (batch, chunk,
// query tile): dwql[h][(b * NB + ch) * 2 + tile][slot].
// ---------------------------------------------------------------------------
template <typename T, bool COEF>
__global__ __launch_bounds__(128, 2) void k2p_local_dq(const T* __restrict__ q, const T* __restrict__ v,
                                                      const uint16_t* __restrict__ G16, const float* __restrict__ Gz,
                                                      const uint16_t* __restrict__ KT16, const float* __restrict__ PZ,
                                                      const float* __restrict__ PZm, const float* __restrict__ gm,
                                                      const float* __restrict__ lb, const float* __restrict__ wqs,
                                                      int Hq, int Hkv, int N, int NB, float* __restrict__ dqf,
                                                      float* __restrict__ dwql) {
  __shared__ __attribute__((aligned(16))) float Kf[kPRows * kPRow];
  __shared__ uint8_t sar[kS], sac[kS];
  __shared__ float bz[kD];
  // Mz is staged into Kf's LDS once the fold has ended every read of Kf (the
  // block then needs 32 KB of LDS, so that the register limit, four blocks per
  // CU, binds instead of the LDS)
  static_assert(sizeof(__bf16) * kD * LD <= sizeof(float) * kPRows * kPRow, "Mz fits Kf");
  __bf16 (*Mz)[LD] = reinterpret_cast<__bf16 (*)[LD]>(Kf);
  __shared__ __attribute__((aligned(16))) float Ered[COEF ? 2 : 1][COEF ? 32 * kERow : 4];

  int hh, ch, u;
  head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;
  const size_t cbase = (size_t)u * NB + ch;
  const size_t np = (size_t)NB * kC;

  // key side k^T of the chunk (fp32), then the one and zero rows
  stage_rows(Kf, KT16 + (size_t)u * kD * np, np, tok0, kD, tid, 128);
  for (int i = tid; i < kC; i += 128) {
    Kf[kD * kPRow + i] = 1.f;
    Kf[(kD + 1) * kPRow + i] = 0.f;
  }
  stage_slots(sar, sac, nullptr, wqs, h, tid, 128);
  if (tid < kD) bz[tid] = lb[(size_t)h * kD + tid] * PZ[cbase * kFP + 1 + tid];
  __syncthreads();

  const int it = wv;
  const int irel = 32 * it + row, ir = tok0 + irel;  // this lane's query token (B-operand column)
  const bool iok = ir < N;
  const size_t io = (size_t)(iok ? ir : N - 1) * kD;
  const float gzi = iok ? Gz[(size_t)(b * Hq + h) * N + ir] : 0.f;
  // ds^T tiles, rows j (key), column i: C[j][i] = v_j . g_i + gz_i on j <= i
  bf16x8 bds[4];
#pragma unroll
  for (int jt = 0; jt < 2; ++jt) {
    if (jt <= it) {
      const int jr = tok0 + 32 * jt + row;
      const bool jok = jr < N;
      const size_t jo = (size_t)(jok ? jr : N - 1) * kD;
      f32x16 ds = f32x16{};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int c = 16 * kk + 8 * s;
        ds = mfma32(row8(v + kbase + jo + c, jok), row8(G16 + qbase + io + c, iok), ds);
      }
      float dsv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = 32 * jt + c32_row(r, l);
        dsv[r] = (j <= irel && iok) ? ds[r] + gzi : 0.f;
      }
      bds[2 * jt] = acc_kfrag(dsv, 0, s);
      bds[2 * jt + 1] = acc_kfrag(dsv, 1, s);
    } else {
      bds[2 * jt] = bf16x8{};
      bds[2 * jt + 1] = bf16x8{};
    }
  }
  float x[kD], dx[kD];
  load_rotated(q, qbase + io, iok, s, x);
#pragma unroll
  for (int m = 0; m < kD; ++m) dx[m] = 0.f;
  const int R2 = (int)(gridDim.x / (R * NB) / Hkv) * NB * 2;  // partial rows per head
  float* coef_out = COEF ? dwql + ((size_t)h * R2 + ((size_t)b * NB + ch) * 2 + it) * kS : nullptr;
  float* ered = COEF ? &Ered[COEF ? wv : 0][0] : nullptr;
  const float* wg = wqs + (size_t)h * kS;
  if (it == 0)
    pdq_all_impl<2, COEF>(Kf, sar, sac, wg, bds, x, dx, l, ered, coef_out, std::make_integer_sequence<int, kS / 32>{});
  else
    pdq_all_impl<4, COEF>(Kf, sar, sac, wg, bds, x, dx, l, ered, coef_out, std::make_integer_sequence<int, kS / 32>{});
  __syncthreads();  // every read of Kf has ended
  // Mz = gm o PZm (bf16), row r holding dimension mz_dim(r / 32, r % 32)
  for (int e = tid; e < kD * kD; e += 128) {
    const int r = e >> 6, c = e & 63;
    const int d = mz_dim(r >> 5, r & 31);
    Mz[r][c] = (__bf16)(gm[((size_t)h * kD + d) * kD + c] * PZm[(cbase * kD + d) * kD + c]);
  }
  __syncthreads();

  // lane group s: dimensions 32 s .. 32 s + 31 of its token
  float full[32];
  combine_rotation_groups(dx, s, full);
  // denominator-state dq of token i: gz_i (bz_d + 2 (Mz q_i)_d); Z^T = Mz Q^T
  // puts dimension 32 s + 16 md + r in register r of product md
  bf16x8 qb[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) qb[kk] = frag8(q, qbase + io + 16 * kk + 8 * s, iok);
#pragma unroll
  for (int md = 0; md < 2; ++md) {
    f32x16 z = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      z = mfma32(*reinterpret_cast<const bf16x8*>(&Mz[32 * md + row][16 * kk + 8 * s]), qb[kk], z);
#pragma unroll
    for (int r = 0; r < 16; ++r) full[16 * md + r] += gzi * (bz[32 * s + 16 * md + r] + 2.f * z[r]);
  }
  if (iok) store32(dqf + qbase + (size_t)ir * kD + 32 * s, full);
}

// ---------------------------------------------------------------------------
// dk local part (feature form) of one query head, one block per (query head,
// chunk), 2 waves = key tiles: dkp[b][h][j][64] (f32).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(128, 2) void k2p_local_dk(const T* __restrict__ k, const T* __restrict__ v,
                                                      const uint16_t* __restrict__ G16, const float* __restrict__ Gz,
                                                      const uint16_t* __restrict__ QT16, const float* __restrict__ wqs,
                                                      int Hq, int Hkv, int N, int NB, float* __restrict__ dkp) {
  __shared__ __attribute__((aligned(16))) float Qf[kPRows * kPRow];
  __shared__ __attribute__((aligned(16))) float wl[kS];
  __shared__ uint8_t sar[kS], sac[kS];
  __shared__ float gzs[kC];

  int hh, ch, u;
  head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;
  const size_t np = (size_t)NB * kC;

  // query side [q^T; 1 (token < N); 0] of the chunk (fp32)
  stage_rows(Qf, QT16 + (size_t)(b * Hq + h) * kPRows * np, np, tok0, kPRows, tid, 128);
  stage_slots(sar, sac, wl, wqs, h, tid, 128);
  if (tid < kC) gzs[tid] = tok0 + tid < N ? Gz[(size_t)(b * Hq + h) * N + tok0 + tid] : 0.f;
  __syncthreads();

  const int jt = wv;
  const int jrel = 32 * jt + row, jr = tok0 + jrel;  // this lane's key token (B-operand column)
  const bool jok = jr < N;
  const size_t jo = (size_t)(jok ? jr : N - 1) * kD;
  // ds tiles, rows i (query), column j: C[i][j] = g_i . v_j + gz_i on j <= i;
  // K-block kb of the dk product covers query tokens 32 jt + 16 kb ..
  bf16x8 bds[4];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    if (it >= jt) {
      const int ir = tok0 + 32 * it + row;
      const bool iok = ir < N;
      const size_t io = (size_t)(iok ? ir : N - 1) * kD;
      f32x16 ds = f32x16{};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int c = 16 * kk + 8 * s;
        ds = mfma32(row8(G16 + qbase + io + c, iok), row8(v + kbase + jo + c, jok), ds);
      }
      float dsv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int irel = 32 * it + c32_row(r, l);
        dsv[r] = (jrel <= irel && tok0 + irel < N) ? ds[r] + gzs[irel] : 0.f;
      }
      const int kb0 = 2 * (it - jt);
      bds[kb0] = acc_kfrag(dsv, 0, s);
      bds[kb0 + 1] = acc_kfrag(dsv, 1, s);
    }
  }
  if (jt == 1) {
    bds[2] = bf16x8{};
    bds[3] = bf16x8{};
  }
  float x[kD], dx[kD];
  load_rotated(k, kbase + jo, jok, s, x);
#pragma unroll
  for (int m = 0; m < kD; ++m) dx[m] = 0.f;
  if (jt == 0)
    pdk_all_impl<4>(Qf, sar, sac, wl, bds, 0, x, dx, l, std::make_integer_sequence<int, kS / 32>{});
  else
    pdk_all_impl<2>(Qf, sar, sac, wl, bds, 32, x, dx, l, std::make_integer_sequence<int, kS / 32>{});
  float full[32];
  combine_rotation_groups(dx, s, full);
  if (jok) store32(dkp + ((size_t)(b * Hq + h) * N + jr) * kD + 32 * s, full);
}

// dkl[u][j][d] = sum over the unit's query heads of dkp (in head order).
__global__ __launch_bounds__(256) void k2p_dk_reduce(const float* __restrict__ dkp, int Hq, int Hkv, int N,
                                                     float* __restrict__ dkl) {
  const size_t per_unit = (size_t)N * kD / 4;  // float4 per unit
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int u = blockIdx.y, R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  if (idx >= per_unit) return;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int hh = 0; hh < R; ++hh) {
    const float4 x = reinterpret_cast<const float4*>(dkp + (size_t)(b * Hq + kh * R + hh) * N * kD)[idx];
    acc.x += x.x;
    acc.y += x.y;
    acc.z += x.z;
    acc.w += x.w;
  }
  reinterpret_cast<float4*>(dkl + (size_t)u * N * kD)[idx] = acc;
}

// ---------------------------------------------------------------------------
// Coefficient gradients for any group count (1..64), one block per query head,
// every sum in a fixed order. wn[f] (natural feature order) = the slot
// gradient dwq (state and local parts) + the denominator's dwqz. Then
// dc0 = wn[0], dlam[g] = scale sum_{g(d)=g} wn[1+d], and pair (r >= c) routes
// scale^2 m_rc wn[pair(r, c)] to raw[g(r)][g(c)] through
// X[r][g] = sum_{c <= r, g(c) = g} m_rc wn[pair(r, c)]; dGam is raw in the
// symmetric convention (off-diagonal entries the mean of both routings).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k2p_coef_grad(const float* __restrict__ dwq, const float* __restrict__ dwqz,
                                                     const int32_t* __restrict__ labels, int G, float scale,
                                                     float* __restrict__ dc0, float* __restrict__ dlam,
                                                     float* __restrict__ dgam) {
  __shared__ float wn[kFeat];
  __shared__ float X[kD][kD + 1];
  __shared__ float raw[kD * kD];
  __shared__ int lab[kD];
  const int h = blockIdx.x, t = threadIdx.x;
  if (t < kD) {
    const int g = labels[h * kD + t];
    lab[t] = g < 0 ? 0 : (g >= G ? G - 1 : g);
  }
  for (int i = t; i < kS; i += 256) {
    const int n = kSlot.nat[i];
    if (n >= 0) wn[n] = dwq[(size_t)h * kS + i];
  }
  __syncthreads();
  for (int n = t; n < kFeat; n += 256) wn[n] += dwqz[(size_t)h * kFP + n];
  __syncthreads();
  if (t < kD) {
    const int r = t;
    for (int g = 0; g < G; ++g) X[r][g] = 0.f;
    const float* rw = wn + 1 + kD + pair_index(r, 0);
    for (int c = 0; c <= r; ++c) X[r][lab[c]] += (c == r ? 1.f : 2.f) * rw[c];
  }
  __syncthreads();
  for (int e = t; e < G * G; e += 256) {
    const int gr = e / G, gc = e % G;
    float acc = 0.f;
    for (int r = 0; r < kD; ++r) acc += lab[r] == gr ? X[r][gc] : 0.f;
    raw[e] = acc * scale * scale;
  }
  if (t == 0) dc0[h] = wn[0];
  if (t < G) {
    float acc = 0.f;
    for (int d = 0; d < kD; ++d) acc += lab[d] == t ? wn[1 + d] : 0.f;
    dlam[(size_t)h * G + t] = acc * scale;
  }
  __syncthreads();
  for (int e = t; e < G * G; e += 256) {
    const int gr = e / G, gc = e % G;
    dgam[(size_t)h * G * G + e] = gr == gc ? raw[e] : 0.5f * (raw[e] + raw[gc * G + gr]);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
template <typename T>
void launch_pair_local_bwd(const LaunchGeom& g, const T* q, const T* k, const T* v, const LocalBwdArgs& a,
                           bool need_dq, bool need_dkv, hipStream_t st, const Timer& timed) {
  // the coefficient partials come from the dq kernel's products, also when dq
  // itself is not requested (its dq then goes to the workspace unused)
  const bool coef = a.dwql != nullptr;
  if (need_dq || coef) {
    timed("k2p_local_dq", st, [&] {
      if (coef)
        hipLaunchKernelGGL((k2p_local_dq<T, true>), dim3(g.R * g.NB * g.U), dim3(128), 0, st, q, v, a.G16, a.Gz,
                           a.KT16, a.PZ, a.PZm, a.gm, a.lb, a.wqs, g.Hq, g.Hkv, g.N, g.NB, a.dqf, a.dwql);
      else
        hipLaunchKernelGGL((k2p_local_dq<T, false>), dim3(g.R * g.NB * g.U), dim3(128), 0, st, q, v, a.G16, a.Gz,
                           a.KT16, a.PZ, a.PZm, a.gm, a.lb, a.wqs, g.Hq, g.Hkv, g.N, g.NB, a.dqf, nullptr);
    });
  }
  if (need_dkv) {
    timed("k2p_local_dk", st, [&] {
      hipLaunchKernelGGL(k2p_local_dk<T>, dim3(g.R * g.NB * g.U), dim3(128), 0, st, k, v, a.G16, a.Gz, a.QT16,
                         a.wqs, g.Hq, g.Hkv, g.N, g.NB, a.dkp);
    });
    timed("k2p_dk_reduce", st, [&] {
      const unsigned blocks = (unsigned)(((size_t)g.N * kD / 4 + 255) / 256);
      hipLaunchKernelGGL(k2p_dk_reduce, dim3(blocks, g.U), dim3(256), 0, st, a.dkp, g.Hq, g.Hkv, g.N, a.dkl);
    });
  }
}

template void launch_pair_local_bwd<float>(const LaunchGeom&, const float*, const float*, const float*,
                                           const LocalBwdArgs&, bool, bool, hipStream_t, const Timer&);
template void launch_pair_local_bwd<uint16_t>(const LaunchGeom&, const uint16_t*, const uint16_t*,
                                              const uint16_t*, const LocalBwdArgs&, bool, bool, hipStream_t,
                                              const Timer&);

void launch_pair_coef_grad(const LaunchGeom& g, const float* dwq, const float* dwqz, const int32_t* labels, int G,
                           float scale, float* dc0, float* dlam, float* dgam, hipStream_t st, const Timer& timed) {
  timed("k2p_coef_grad", st, [&] {
    hipLaunchKernelGGL(k2p_coef_grad, dim3(g.Hq), dim3(256), 0, st, dwq, dwqz, labels, G, scale, dc0, dlam, dgam);
  });
}

}  // namespace oal
