// bf16 matrix-core (MFMA) forward for gfx950.
//
// (k2_fwd_prep, which also forms the per-head slot coefficients and the
// intra-chunk coefficient packs of oal_slot_coef.hpp in blocks of its own, and
// the chunk-state scan producing P_c are in oal_mfma_scan.hip)
// k2_intra_fwd         : per (query head, chunk, unit): intra-chunk kernel from
//                        MFMA group sums, kappa . V, and the denominator's state
//                        term as a 64x64 quadratic form; writes num, den.
// k2_out_fwd           : per (query head, chunk, unit): state readout
//                        phi_Q . P_c with query features generated in
//                        registers, added to num, then out = num / den.
//
// Saved layouts (per unit u and chunk c; "tile" = 32 slots, "k-step" = 16 slots):
//   PR [u][c][kS/32][4][32][16 e]   bf16  (backward A operand: values contiguous; the
//                                          readouts take their B fragments from it
//                                          with transposed LDS reads)
//   PZ [u][c][kFP]                  f32   (denominator state, natural feature order)
//   PZm [u][c][64][64]              f32   (its pair entries as a symmetric matrix; PZ and
//                                          PZm are k2_den_scan's prefixes of k2_fwd_prep's
//                                          per-chunk K^T K, sum k and token count)
//   KAP [b][h][c][3][64][16]        bf16  (intra-chunk kappa of the 3 lower 32x32 tile
//                                          pairs as the backward dv product's A fragments)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"
#include "oal_slot_coef.hpp"

namespace oal {

static __constant__ SlotTable kSlot = make_slot_table();

template <typename T>
__device__ __forceinline__ float ldf(const T* p, size_t i) {
  return to_f(p[i]);
}

// One 64-wide token row as 8 bf16 fragments, with 16-byte loads. The row index
// is clamped so that every load is issued unconditionally; rows at or past N
// come back as zeros.
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ src, size_t row_base, bool ok,
                                         bf16x8 (&r)[8]) {
  const bf16x8* p = reinterpret_cast<const bf16x8*>(src + row_base);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bf16x8 x = p[i];
    r[i] = ok ? x : bf16x8{};
  }
}
__device__ __forceinline__ void load_row(const float* __restrict__ src, size_t row_base, bool ok, bf16x8 (&r)[8]) {
  const float4* p = reinterpret_cast<const float4*>(src + row_base);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 a = p[2 * i], b = p[2 * i + 1];
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const bf16x8 x = pack8(v);
    r[i] = ok ? x : bf16x8{};
  }
}

// ---------------------------------------------------------------------------
// Forward readout: one block of two waves per (query head, chunk, unit); wave w
// owns tokens 32w..32w+31 (one token per lane row). The per-chunk P^T tiles are
// streamed through an LDS ring of kNSR stages of kRG k-steps shared by both waves.
// ---------------------------------------------------------------------------
constexpr int kRG = 4;                        // k-steps per ring group
constexpr int kRingGroups = (kKS + kRG - 1) / kRG;
constexpr int kRingStep = 64 * 16;            // bf16 per k-step tile

// 8 consecutive elements of a row as a bf16 MFMA fragment.
__device__ __forceinline__ bf16x8 load8(const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ bf16x8 load8(const float* p) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return pack8(v);
}

// LDS stages of the readout ring: three (24 KB) keep a block of two waves at
// 33 KB of LDS with the slot weights, so that four blocks (two waves per SIMD,
// the register limit) fit a CU; one group of four k-steps stays in flight.
constexpr int kNSR = 3;

// Ring group G (k-steps G * kRG ..) into LDS stage G % kNSR; each k-step tile is
// 4 pieces of 512 bytes = 128 lanes x 16 bytes (wave w copies pieces 2w, 2w + 1).
template <int G>
__device__ __forceinline__ void ring_issue(const uint16_t* pr, const LdsRing<kNSR>& ring, int tid) {
  const int wv = tid >> 6, l = tid & 63;
  __bf16* st = ring.st[G % kNSR];
#pragma unroll
  for (int i = 0; i < kRG; ++i) {
    const int t = G * kRG + i;
    if (t < kKS) copy16_to_lds(pr + rpiece(t, 2 * wv + (l >> 5), l & 31), st + i * kRingStep + 64 * wv * 8);
  }
}

// Operands of k-step T: the slot weights of this lane's row (lane j of the row
// holds the weight of slot 16 T + 8 s + j, j < 8; one 4-byte read per lane
// instead of the 32 bytes of every weight of its lane group) and the two P^T
// fragments (value halves) of the staged tile.
struct ReadoutOps {
  float w;
  bf16x8 b0, b1;
};

template <int T, int NS, int RG = kRG>
__device__ __forceinline__ void readout_read(const float* wl, const LdsRing<NS>& ring, int lane, ReadoutOps& o) {
  const int s = lane >> 5;
  o.w = wl[16 * T + 8 * s + (lane & 7)];
  const __bf16* tile = ring.st[(T / RG) % NS] + (T % RG) * kRingStep;
  o.b0 = tr_fragment(tile, lane, 0);
  o.b1 = tr_fragment(tile, lane, 1);
}
template <int T>
__device__ __forceinline__ void readout_step(const float (&x)[kD], const ReadoutOps& o, f32x16 (&acc)[2]) {
  const bf16x8 a = feature_fragment_row<T>(x, o.w);
  acc[0] = mfma32(a, o.b0, acc[0]);
  acc[1] = mfma32(a, o.b1, acc[1]);
}

// Copies one thread issues for ring group G.
template <int G>
constexpr int group_copies() {
  return (G < kRingGroups) ? ((G + 1) * kRG <= kKS ? kRG : kKS - G * kRG) : 0;
}
template <int G, int... I>
constexpr int copies_in_flight(std::integer_sequence<int, I...>) {
  return (group_copies<G + 1 + I>() + ... + 0);
}

// Ring pipeline over the k-step groups: groups G + 1 .. G + kNSR - 2 may still
// be in flight while group G is read; group G + kNSR - 1 is issued after the
// barrier that retires every read of its stage.
template <int G>
__device__ __forceinline__ void readout_group(const float (&x)[kD], const float* wl, const LdsRing<kNSR>& ring,
                                              const uint16_t* pt, int tid, int lane, f32x16 (&acc)[2]) {
  ring_sync<copies_in_flight<G>(std::make_integer_sequence<int, kNSR - 2>{})>();
  if constexpr (G + kNSR - 1 < kRingGroups) ring_issue<G + kNSR - 1>(pt, ring, tid);
  // the operands of k-step i + 1 are read before k-step i is computed
  constexpr int n = (G + 1) * kRG <= kKS ? kRG : kKS - G * kRG;
  ReadoutOps o[2];
  readout_read<G * kRG>(wl, ring, lane, o[0]);
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (([&] {
       if constexpr (I + 1 < n) readout_read<G * kRG + I + 1>(wl, ring, lane, o[(I + 1) & 1]);
       readout_step<G * kRG + I>(x, o[I & 1], acc);
     }()),
     ...);
  }(std::make_integer_sequence<int, n>{});
  if constexpr (G + 1 < kRingGroups) readout_group<G + 1>(x, wl, ring, pt, tid, lane, acc);
}

// 16 consecutive elements of a row as two bf16 fragments (16-byte loads).
__device__ __forceinline__ void load16(const uint16_t* __restrict__ src, size_t off, bool ok, bf16x8 (&r)[2]) {
  const bf16x8* p = reinterpret_cast<const bf16x8*>(src + off);
  const bf16x8 a = p[0], b = p[1];
  r[0] = ok ? a : bf16x8{};
  r[1] = ok ? b : bf16x8{};
}
__device__ __forceinline__ void load16(const float* __restrict__ src, size_t off, bool ok, bf16x8 (&r)[2]) {
  const float4* p = reinterpret_cast<const float4*>(src + off);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 a = p[2 * i], b = p[2 * i + 1];
    float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const bf16x8 y = pack8(x);
    r[i] = ok ? y : bf16x8{};
  }
}

// ---------------------------------------------------------------------------
// Feature-form local score of a 32 x 32 tile (per-pair coefficients):
//   kappa^T[j][i] = sum_slot raw(k_j)[slot] wq[slot] raw(q_i)[slot]
// on v_mfma_f32_32x32x16_bf16 over the 138 k-steps of 16 slots: the A operand
// is the key row's raw features (lane row = key token j), the B operand the
// query row's weighted features (lane column = query token i), both generated
// from rotated rows held in registers (static indices) with the weights of the
// lane group's eight slots read from LDS. Reference: the local score
// phi_Q . phi_K^T of hd_block_gemm_runtime.py:530-540.
// ---------------------------------------------------------------------------
// Rotated fp32 row x[m] = row[(m + 32 s) % 64] of a bf16 row in LDS.
__device__ __forceinline__ void lds_rotated_row(const __bf16* rowp, int s, float (&x)[kD]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bf16x8 r = *reinterpret_cast<const bf16x8*>(rowp + ((8 * i + 32 * s) & 63));
#pragma unroll
    for (int j = 0; j < 8; ++j) x[8 * i + j] = (float)r[j];
  }
}
template <int T>
__device__ __forceinline__ f32x16 pair_step(const float (&xk)[kD], const float (&xq)[kD], const float* wl, int s,
                                            f32x16 S) {
  const float4 w0 = *reinterpret_cast<const float4*>(wl + 16 * T + 8 * s);
  const float4 w1 = *reinterpret_cast<const float4*>(wl + 16 * T + 8 * s + 4);
  const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  return mfma32(raw_fragment<T>(xk), feature_fragment<T>(xq, w), S);
}
template <int... T>
__device__ __forceinline__ f32x16 pair_score_impl(const float (&xk)[kD], const float (&xq)[kD], const float* wl, int s,
                                                  std::integer_sequence<int, T...>) {
  f32x16 S = f32x16{};
  ((S = pair_step<T>(xk, xq, wl, s, S)), ...);
  return S;
}
__device__ __forceinline__ f32x16 pair_score(const float (&xk)[kD], const float (&xq)[kD], const float* wl, int s) {
  return pair_score_impl(xk, xq, wl, s, std::make_integer_sequence<int, kKS>{});
}

// ---------------------------------------------------------------------------
// Intra-chunk forward, one block of 4 waves per (query head, chunk, unit).
// Waves 0-2 each own one lower 32x32 tile of kappa^T (rows j = key token,
// columns i = query token), (j-tile, i-tile) = (0,0), (0,1), (1,1):
//   s_g^T = (K o mask_g) Q^T on v_mfma_f32_32x32x16_bf16 (8 groups x 4 k-steps),
//   kappa = c0 + sum_g s_g (lam'_g + Gam'_gg s_g + 2 sum_{h>g} Gam'_gh s_h)
// (lam' = scale lam, Gam' = scale^2 Gam, padded to 8 groups with zeros), then
// num^T = V^T kappa^T with kappa^T handed to the MFMA straight from the
// accumulators, and the denominator row sums. Wave 3 evaluates the state part
// of the denominator as the quadratic form az + q . (bz + Mz q), Mz = gm o PZm.
// Writes the intra part of num and the full den (k2_out_fwd adds the readout),
// and saves the bf16 kappa tiles for the backward (KAP).
// PAIRWISE (more than 8 groups, per-pair coefficients): waves 0-2 form their
// kappa^T tile in feature form (pair_score) from the slot weights wqs instead
// of the group sums; everything else is shared.
// ---------------------------------------------------------------------------
template <typename T, bool PAIRWISE>
__global__ __launch_bounds__(256, PAIRWISE ? 2 : 3) void k2_intra_fwd(const T* __restrict__ q, const T* __restrict__ k,
                                                    const T* __restrict__ v, const float* __restrict__ PZ,
                                                    const float* __restrict__ PZm, const int32_t* __restrict__ labels,
                                                    const float* __restrict__ ic, const float* __restrict__ gm,
                                                    const float* __restrict__ lb, const float* __restrict__ wqs,
                                                    int G, int Hq, int Hkv, int N, int NB, float* __restrict__ num,
                                                    float* __restrict__ den, uint16_t* __restrict__ kapf) {
  constexpr int LD = kD + 8;  // bf16 row stride (bank spread)
  __shared__ __attribute__((aligned(16))) __bf16 Qs[kC][LD];
  __shared__ __attribute__((aligned(16))) __bf16 Ks[kC][LD];
  __shared__ __attribute__((aligned(16))) __bf16 VT[kD][LD];
  __shared__ __attribute__((aligned(16))) __bf16 Mz[kD][LD];
  __shared__ __attribute__((aligned(16))) uint32_t mk[4][8][2][4];
  __shared__ float bz[kD], dsS[kC], dp2[32];
  // wave 2's half of the i-tile 1 numerator, handed to wave 1 after the
  // barrier that ends every read of Qs (8 KB of its 9 KB)
  static_assert(sizeof(float) * 2 * 16 * 64 <= sizeof(Qs), "the reduction buffer fits Qs");
  float (*red)[16][64] = reinterpret_cast<float (*)[16][64]>(&Qs[0][0]);
  __shared__ __attribute__((aligned(16))) __bf16 kapT[3][32][40];  // kappa^T tiles [j][i], bf16
  __shared__ __attribute__((aligned(16))) float wl[PAIRWISE ? kS : 4];  // the head's slot weights

  int hh, ch, u;
  head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;
  const size_t cbase = (size_t)u * NB + ch;
  const float* cf = ic + (size_t)h * kIC;

  // --- staging ------------------------------------------------------------
  {
    const int r = tid >> 2, qq = tid & 3;
    const int tok = tok0 + r;
    const bool ok = tok < N;
    const size_t roff = (size_t)(ok ? tok : N - 1) * kD + 16 * qq;
    bf16x8 x[2];
    load16(q, qbase + roff, ok, x);
    *reinterpret_cast<bf16x8*>(&Qs[r][16 * qq]) = x[0];
    *reinterpret_cast<bf16x8*>(&Qs[r][16 * qq + 8]) = x[1];
    load16(k, kbase + roff, ok, x);
    *reinterpret_cast<bf16x8*>(&Ks[r][16 * qq]) = x[0];
    *reinterpret_cast<bf16x8*>(&Ks[r][16 * qq + 8]) = x[1];
    load16(v, kbase + roff, ok, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      VT[16 * qq + e][r] = x[0][e];
      VT[16 * qq + 8 + e][r] = x[1][e];
    }
    // Mz[r][c] = gm[h][r][c] * PZm[r][c], c = 16 qq .. 16 qq + 15
    const float4* gp = reinterpret_cast<const float4*>(gm + ((size_t)h * kD + r) * kD + 16 * qq);
    const float4* zp = reinterpret_cast<const float4*>(PZm + (cbase * kD + r) * kD + 16 * qq);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float4 g0 = gp[2 * i], g1 = gp[2 * i + 1], z0 = zp[2 * i], z1 = zp[2 * i + 1];
      float y[8] = {g0.x * z0.x, g0.y * z0.y, g0.z * z0.z, g0.w * z0.w,
                    g1.x * z1.x, g1.y * z1.y, g1.z * z1.z, g1.w * z1.w};
      *reinterpret_cast<bf16x8*>(&Mz[r][16 * qq + 8 * i]) = pack8(y);
    }
    if constexpr (PAIRWISE) {
      stage_f4<256, kS / 4>(reinterpret_cast<float4*>(wl), reinterpret_cast<const float4*>(wqs + (size_t)h * kS), tid);
    }
    // group masks: entry (kk, g, ss, w) covers dims d, d + 1 with d = 16 kk + 8 ss + 2 w
    if constexpr (!PAIRWISE) {
      const int kk = tid >> 6, g = (tid >> 3) & 7, ss = (tid >> 2) & 1, w = tid & 3;
      const int d = 16 * kk + 8 * ss + 2 * w;
      int g0 = labels[h * kD + d], g1 = labels[h * kD + d + 1];
      g0 = g0 < 0 ? 0 : (g0 >= G ? G - 1 : g0);
      g1 = g1 < 0 ? 0 : (g1 >= G ? G - 1 : g1);
      mk[kk][g][ss][w] = (g0 == g ? 0x0000ffffu : 0u) | (g1 == g ? 0xffff0000u : 0u);
    }
    if (tid < kD) bz[tid] = lb[(size_t)h * kD + tid] * PZ[cbase * kFP + 1 + tid];
  }
  __syncthreads();

  f32x16 acc[2] = {f32x16{}, f32x16{}};
  float dsum = 0.f;
  if (wv < 3) {
    const int tj = wv == 2 ? 1 : 0, ti = wv == 0 ? 0 : 1;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const int i = 32 * ti + row;
    const bool irow = tok0 + i < N;
    float kv[16];  // kappa^T[j][i], j = 32 tj + c32_row(r)
    if constexpr (PAIRWISE) {
      float xk[kD], xq[kD];
      lds_rotated_row(&Ks[32 * tj + row][0], s, xk);
      lds_rotated_row(&Qs[32 * ti + row][0], s, xq);
      const f32x16 S = pair_score(xk, xq, wl, s);
#pragma unroll
      for (int r = 0; r < 16; ++r) kv[r] = S[r];
    } else {
      f32x16 sg[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) sg[g] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(&Ks[32 * tj + row][16 * kk + 8 * s]);
        const bf16x8 qf = *reinterpret_cast<const bf16x8*>(&Qs[32 * ti + row][16 * kk + 8 * s]);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const u32x4 m = *reinterpret_cast<const u32x4*>(&mk[kk][g][s][0]);
          sg[g] = mfma32(__builtin_bit_cast(bf16x8, kf & m), qf, sg[g]);
        }
      }
      float lamc[8], gd[8], g2[8][8];
      const float c0h = cf[0];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        lamc[g] = cf[kIcLam + g];
        gd[g] = cf[kIcGam + 9 * g];
#pragma unroll
        for (int h2 = 0; h2 < 8; ++h2) g2[g][h2] = 2.f * cf[kIcGam + 8 * g + h2];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = c0h;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          float inner = fmaf(gd[g], sg[g][r], lamc[g]);
#pragma unroll
          for (int h2 = g + 1; h2 < 8; ++h2) inner = fmaf(g2[g][h2], sg[h2][r], inner);
          x = fmaf(sg[g][r], inner, x);
        }
        kv[r] = x;
      }
    }
    float kap[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = 32 * tj + c32_row(r, l);
      kap[r] = (j <= i && irow) ? kv[r] : 0.f;
      dsum += kap[r];
      kapT[wv][c32_row(r, l)][row] = (__bf16)kap[r];
    }
    dsum += __shfl_xor(dsum, 32, 64);
    // kappa^T as the B operand of num^T = V^T kappa^T: k-step t covers
    // j = 16 t .. 16 t + 15; lane group s must hold j = 16 t + 8 s .. + 7, the
    // accumulators give it j = 16 t + 4 s + (0..3) and 16 t + 8 + 4 s + (0..3).
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t a0 = pack_bf16x2(kap[8 * t + 0], kap[8 * t + 1]);
      const uint32_t a1 = pack_bf16x2(kap[8 * t + 2], kap[8 * t + 3]);
      const uint32_t b0 = pack_bf16x2(kap[8 * t + 4], kap[8 * t + 5]);
      const uint32_t b1 = pack_bf16x2(kap[8 * t + 6], kap[8 * t + 7]);
      const uint32_t r0 = __shfl_xor(s ? a0 : b0, 32, 64);
      const uint32_t r1 = __shfl_xor(s ? a1 : b1, 32, 64);
      const u32x4 fr = s ? u32x4{r0, r1, b0, b1} : u32x4{a0, a1, r0, r1};
      const bf16x8 bfr = __builtin_bit_cast(bf16x8, fr);
#pragma unroll
      for (int et = 0; et < 2; ++et) {
        const bf16x8 af = *reinterpret_cast<const bf16x8*>(&VT[32 * et + row][32 * tj + 16 * t + 8 * s]);
        acc[et] = mfma32(af, bfr, acc[et]);
      }
    }
  } else {
    // state part of the denominator: Z[d][i] = (Mz Q^T)[d][i]
    const float az = cf[0] * PZ[cbase * kFP];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      float part = 0.f;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        f32x16 z = f32x16{};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(&Mz[32 * dt + row][16 * kk + 8 * s]);
          const bf16x8 bq = *reinterpret_cast<const bf16x8*>(&Qs[32 * it + row][16 * kk + 8 * s]);
          z = mfma32(a, bq, z);
        }
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d0 = 32 * dt + 8 * a + 4 * s;
          const bf16x4 q4 = *reinterpret_cast<const bf16x4*>(&Qs[32 * it + row][d0]);
#pragma unroll
          for (int vv = 0; vv < 4; ++vv) part = fmaf((float)q4[vv], bz[d0 + vv] + z[4 * a + vv], part);
        }
      }
      part += __shfl_xor(part, 32, 64);
      if (s == 0) dsS[32 * it + row] = az + part;
    }
  }
  __syncthreads();
  if (wv == 2) {
#pragma unroll
    for (int et = 0; et < 2; ++et)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[et][r][l] = acc[et][r];
    if (s == 0) dp2[row] = dsum;
  }
  if (wv < 3) {
    // kappa for the backward's dv = kappa^T G (k2_local_dv): lane (key row j,
    // group s) holds kappa[i][j] for query rows i = 16 t + 8 s .. + 7, t = 0, 1
    // (the K-major A fragments of that product), read back transposed
    const bf16x8 f0 = *reinterpret_cast<const bf16x8*>(&kapT[wv][row][8 * s]);
    const bf16x8 f1 = *reinterpret_cast<const bf16x8*>(&kapT[wv][row][16 + 8 * s]);
    uint16_t* dst = kapf + ((((size_t)(b * Hq + h) * NB + ch) * 3 + wv) * 64 + l) * 16;
    *reinterpret_cast<bf16x8*>(dst) = f0;
    *reinterpret_cast<bf16x8*>(dst + 8) = f1;
  }
  __syncthreads();
  if (wv < 2) {
    const int i = 32 * wv + row, tok = tok0 + i;
    if (wv == 1) {
#pragma unroll
      for (int et = 0; et < 2; ++et)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[et][r] += red[et][r][l];
      dsum += dp2[row];
    }
    if (tok < N) {
      float* o = num + qbase + (size_t)tok * kD;
#pragma unroll
      for (int et = 0; et < 2; ++et)
#pragma unroll
        for (int a = 0; a < 4; ++a)
          *reinterpret_cast<float4*>(o + 32 * et + 8 * a + 4 * s) =
              make_float4(acc[et][4 * a], acc[et][4 * a + 1], acc[et][4 * a + 2], acc[et][4 * a + 3]);
      if (s == 0) den[(size_t)(b * Hq + h) * N + tok] = dsS[i] + dsum;
    }
  }
}

// ---------------------------------------------------------------------------
// State readout: one block of two waves per (query head, chunk, unit); wave w
// owns tokens 32w..32w+31 (one token per lane row): num += phi_Q(q) . P_c,
// then out = num / den.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(128, 2) void k2_out_fwd(const T* __restrict__ q, const float* __restrict__ wqs,
                                                  const uint16_t* __restrict__ PR, int Hq, int Hkv, int N, int NB,
                                                  float floor, T* __restrict__ out, float* __restrict__ num,
                                                  const float* __restrict__ den) {
  __shared__ __attribute__((aligned(16))) __bf16 ring0[kRG * kRingStep], ring1[kRG * kRingStep],
      ring2[kRG * kRingStep], ring3[kRG * kRingStep], ring4[kRG * kRingStep], ring5[kRG * kRingStep],
      ring6[kRG * kRingStep], ring7[kRG * kRingStep];
  static_assert(kNSR >= 3 && kNSR <= 8, "readout ring depth");
  __bf16* const stages[8] = {ring0, ring1, ring2, ring3, ring4, ring5, ring6, ring7};
  LdsRing<kNSR> ring;
#pragma unroll
  for (int i = 0; i < kNSR; ++i) ring.st[i] = stages[i];
  __shared__ __attribute__((aligned(16))) float wl[kS];

  int hh, ch, u;
  head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const uint16_t* pt = PR + ((size_t)u * NB + ch) * ((size_t)kKS * kRingStep);

  stage_f4<128, kS / 4>(reinterpret_cast<float4*>(wl), reinterpret_cast<const float4*>(wqs + (size_t)h * kS), tid);
  // rotated query row of this lane's token
  float x[kD];
  {
    const int tok = tok0 + 32 * wv + row;
    const bool ok = tok < N;
    const int tc = ok ? tok : N - 1;
    bf16x8 qr[8];
    load_row(q, qbase + (size_t)tc * kD, ok, qr);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // rotation by 32 s: half i of the lane's row is stored at (8 i + 32 s) mod 64
        const float val = (float)qr[i][j];
        x[(8 * i + j) & 63] = val;
      }
    if (s == 1) {
#pragma unroll
      for (int m = 0; m < 32; ++m) {
        const float t = x[m];
        x[m] = x[m + 32];
        x[m + 32] = t;
      }
    }
  }
  // accumulators start from the intra-chunk numerator
  // the state part accumulates from zero; the intra part already in num is
  // added in the epilogue, its loads sharing the denominators' round trip
  // (as the accumulators' initial value the first product waited for them)
  f32x16 acc[2] = {f32x16{}, f32x16{}};
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (ring_issue<I>(pt, ring, tid), ...);
  }(std::make_integer_sequence<int, kNSR - 1>{});
  readout_group<0>(x, wl, ring, pt, tid, l, acc);

  const size_t dbase = (size_t)(b * Hq + h) * N;
  // the row denominators are loaded together (rows clamped into range): a load
  // inside the row test would wait for each one in turn
  float dv16[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) dv16[i] = den[dbase + min(tok0 + 32 * wv + c32_row(i, l), N - 1)];
  // rows past N read row N - 1 and are never stored: a load inside the row
  // test would wait for each one in turn
  float nm[2][16];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int i = 0; i < 16; ++i) nm[nt][i] = num[qbase + (size_t)min(tok0 + 32 * wv + c32_row(i, l), N - 1) * kD + 32 * nt + row];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tok = tok0 + 32 * wv + c32_row(i, l);
    if (tok < N) {
      const float dd = dv16[i];
      const float inv = 1.f / (floor > 0.f ? fmaxf(dd, floor) : dd);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const size_t o = qbase + (size_t)tok * kD + 32 * nt + row;
        acc[nt][i] += nm[nt][i];
        num[o] = acc[nt][i];
        out[o] = from_f<T>(acc[nt][i] * inv);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Forward readout with the query heads of a unit sharing each copy of P_c: one
// block per (token half, chunk, unit) of R + 1 waves (R <= kMaxRS query heads
// per kv head). Wave w < R reads out head kh R + w for the half's 32 tokens as
// k2_out_fwd does; wave R only streams the P^T tiles into an LDS ring of kNSS
// stages (it issues every copy, so its vmcnt alone paces the ring). Each
// chunk's state then leaves L2 twice, once per token half, instead of once per
// query head, and the deeper ring keeps more of it in flight. The ring holds
// kNSS stages of kRGS k-steps (48 KB): one ring barrier per eight k-steps.
// The slot weights come from global memory (L2), a ring group ahead, one
// register per k-step pair broadcast along each lane row (row_bcast), so the
// block needs only the ring's LDS and two blocks (four waves per SIMD, 128
// VGPRs) fit a CU.
// ---------------------------------------------------------------------------
constexpr int kNSS = 3;
constexpr int kRGS = 8;  // k-steps per ring group of the shared readout
constexpr int kRingGroupsS = (kKS + kRGS - 1) / kRGS;
constexpr int kMaxRS = 7;

// Copies per k-step tile (two 1 KiB wave copies) of ring group G.
template <int G>
constexpr int group_steps_shared() {
  return (G < kRingGroupsS) ? ((G + 1) * kRGS <= kKS ? kRGS : kKS - G * kRGS) : 0;
}

// Ring group G into stage G % kNSS by the copy wave: two 1 KiB wave copies per
// k-step tile.
template <int G>
__device__ __forceinline__ void ring_issue_shared(const uint16_t* pt, const LdsRing<kNSS>& ring, int lane) {
  __bf16* st = ring.st[G % kNSS];
#pragma unroll
  for (int i = 0; i < kRGS; ++i) {
    const int t = G * kRGS + i;
    if (t < kKS) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        copy16_to_lds(pt + rpiece(t, 2 * hf + (lane >> 5), lane & 31), st + i * kRingStep + 64 * hf * 8);
    }
  }
}
template <int G, int... I>
constexpr int shared_copies_in_flight(std::integer_sequence<int, I...>) {
  return ((2 * group_steps_shared<G + 1 + I>()) + ... + 0);
}
// The copy wave: one ring barrier per group (as many as the readout waves),
// then the copies of the group kNSS - 1 ahead into the stage just released.
template <int G>
__device__ __forceinline__ void ring_produce(const uint16_t* pt, const LdsRing<kNSS>& ring, int lane) {
  ring_sync<shared_copies_in_flight<G>(std::make_integer_sequence<int, kNSS - 2>{})>();
  if constexpr (G + kNSS - 1 < kRingGroupsS) ring_issue_shared<G + kNSS - 1>(pt, ring, lane);
  if constexpr (G + 1 < kRingGroupsS) ring_produce<G + 1>(pt, ring, lane);
}
// Slot weights of ring group G of the shared readout, read from global memory
// (L2) one group ahead: register p holds k-step pair 4 G + p, lane j of each
// row the weight of slot 16 (2 (4 G + p) + j / 8) + 8 s + j % 8. The pair
// index is clamped so that every load is issued.
template <int G>
__device__ __forceinline__ void readout_weights_shared(const float* __restrict__ wg, int lane, float (&w)[kRGS / 2]) {
  const int j = lane & 15, s = lane >> 5;
#pragma unroll
  for (int p = 0; p < kRGS / 2; ++p) {
    constexpr int kPairs = kKS / 2;
    const int pr = min(G * (kRGS / 2) + p, kPairs - 1);
    w[p] = wg[32 * pr + 16 * (j >> 3) + 8 * s + (j & 7)];
  }
}
template <int T>
__device__ __forceinline__ void readout_tiles_shared(const LdsRing<kNSS>& ring, int lane, bf16x8 (&b)[2]) {
  const __bf16* tile = ring.st[(T / kRGS) % kNSS] + (T % kRGS) * kRingStep;
  b[0] = tr_fragment(tile, lane, 0);
  b[1] = tr_fragment(tile, lane, 1);
}
template <int G>
__device__ __forceinline__ void readout_group_shared(const float (&x)[kD], const float* __restrict__ wg,
                                                     const LdsRing<kNSS>& ring, int lane, f32x16 (&acc)[2],
                                                     const float (&wc)[kRGS / 2]) {
  static_assert(kKS % 2 == 0 && kRGS % 2 == 0, "weights come in k-step pairs");
  ring_sync<shared_copies_in_flight<G>(std::make_integer_sequence<int, kNSS - 2>{})>();
  float wn[kRGS / 2];
  if constexpr (G + 1 < kRingGroupsS) readout_weights_shared<G + 1>(wg, lane, wn);
  constexpr int n = group_steps_shared<G>();
  bf16x8 b[2][2];
  readout_tiles_shared<G * kRGS>(ring, lane, b[0]);
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (([&] {
       if constexpr (I + 1 < n) readout_tiles_shared<G * kRGS + I + 1>(ring, lane, b[(I + 1) & 1]);
       const bf16x8 a = feature_fragment_row<G * kRGS + I, 8 * (I & 1)>(x, wc[I / 2]);
       acc[0] = mfma32(a, b[I & 1][0], acc[0]);
       acc[1] = mfma32(a, b[I & 1][1], acc[1]);
     }()),
     ...);
  }(std::make_integer_sequence<int, n>{});
  if constexpr (G + 1 < kRingGroupsS) readout_group_shared<G + 1>(x, wg, ring, lane, acc, wn);
}

template <typename T>
__global__ __launch_bounds__(64 * (kMaxRS + 1), 4) void k2_out_fwd_shared(
    const T* __restrict__ q, const float* __restrict__ wqs, const uint16_t* __restrict__ PR, int Hq, int Hkv, int N,
    int NB, float floor, T* __restrict__ out, float* __restrict__ num, const float* __restrict__ den) {
  __shared__ __attribute__((aligned(16))) __bf16 rs[kNSS][kRGS * kRingStep];
  LdsRing<kNSS> ring;
#pragma unroll
  for (int i = 0; i < kNSS; ++i) ring.st[i] = rs[i];

  int th, ch, u;
  head_chunk_unit(2, NB, (int)(gridDim.x / (2 * NB)), th, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC + 32 * th;
  const uint16_t* pt = PR + ((size_t)u * NB + ch) * ((size_t)kKS * kRingStep);

  if (wv == R) {
    // the copy wave
    [&]<int... I>(std::integer_sequence<int, I...>) {
      (ring_issue_shared<I>(pt, ring, l), ...);
    }(std::make_integer_sequence<int, kNSS - 1>{});
    ring_produce<0>(pt, ring, l);
    return;
  }
  const int h = kh * R + wv;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const float* wg = wqs + (size_t)h * kS;
  float w0[kRGS / 2];
  readout_weights_shared<0>(wg, l, w0);
  float x[kD];
  {
    const int tok = tok0 + row;
    const bool ok = tok < N;
    const int tc = ok ? tok : N - 1;
    bf16x8 qr[8];
    load_row(q, qbase + (size_t)tc * kD, ok, qr);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) x[(8 * i + j) & 63] = (float)qr[i][j];
    if (s == 1) {
#pragma unroll
      for (int m = 0; m < 32; ++m) {
        const float t = x[m];
        x[m] = x[m + 32];
        x[m + 32] = t;
      }
    }
  }
  // the state part accumulates from zero; the intra part already in num is
  // added in the epilogue, its loads sharing the denominators' round trip
  // (as the accumulators' initial value the first product waited for them)
  f32x16 acc[2] = {f32x16{}, f32x16{}};
  readout_group_shared<0>(x, wg, ring, l, acc, w0);

  const size_t dbase = (size_t)(b * Hq + h) * N;
  // the row denominators are loaded together (rows clamped into range): a load
  // inside the row test would wait for each one in turn
  float dv16[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) dv16[i] = den[dbase + min(tok0 + c32_row(i, l), N - 1)];
  // rows past N read row N - 1 and are never stored: a load inside the row
  // test would wait for each one in turn
  float nm[2][16];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int i = 0; i < 16; ++i) nm[nt][i] = num[qbase + (size_t)min(tok0 + c32_row(i, l), N - 1) * kD + 32 * nt + row];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tok = tok0 + c32_row(i, l);
    if (tok < N) {
      const float dd = dv16[i];
      const float inv = 1.f / (floor > 0.f ? fmaxf(dd, floor) : dd);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const size_t o = qbase + (size_t)tok * kD + 32 * nt + row;
        acc[nt][i] += nm[nt][i];
        num[o] = acc[nt][i];
        out[o] = from_f<T>(acc[nt][i] * inv);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA layout self-test: checks the accumulator layouts assumed above and the
// lane mapping of the transposed LDS reads (tr_fragment).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k2_selftest(int* __restrict__ errors) {
  __shared__ float A[32][32], B[32][32];
  const int l = threadIdx.x;
  for (int i = l; i < 32 * 32; i += 64) {
    A[i / 32][i % 32] = (float)((i * 7) % 13) - 6.f;
    B[i / 32][i % 32] = (float)((i * 5) % 11) - 5.f;
  }
  __syncthreads();
  int bad = 0;
  {  // 32x32x16 with K = 16
    float fa[8], fb[8];
    for (int j = 0; j < 8; ++j) {
      fa[j] = A[l % 32][8 * (l / 32) + j];
      fb[j] = B[8 * (l / 32) + j][l % 32];
    }
    f32x16 c = mfma32(pack8(fa), pack8(fb), f32x16{});
    for (int i = 0; i < 16; ++i) {
      const int r = c32_row(i, l), col = l % 32;
      float ref = 0.f;
      for (int kk = 0; kk < 16; ++kk) ref += A[r][kk] * B[kk][col];
      bad += (c[i] != ref);
    }
  }
  {  // 32x32x2 f32 with K = 2 (the fp32 matrix-core route)
    const float a = A[l % 32][l / 32], bb = B[l / 32][l % 32];
    f32x16 c = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bb, f32x16{}, 0, 0, 0);
    for (int i = 0; i < 16; ++i) {
      const int r = c32_row(i, l), col = l % 32;
      bad += (c[i] != A[r][0] * B[0][col] + A[r][1] * B[1][col]);
    }
  }
  {  // 16x16x32 with K = 32
    float fa[8], fb[8];
    for (int j = 0; j < 8; ++j) {
      fa[j] = A[l % 16][8 * (l / 16) + j];
      fb[j] = B[8 * (l / 16) + j][l % 16];
    }
    f32x4 c = mfma16(pack8(fa), pack8(fb), f32x4{});
    for (int i = 0; i < 4; ++i) {
      const int r = c16_row(i, l), col = l % 16;
      float ref = 0.f;
      for (int kk = 0; kk < 32; ++kk) ref += A[r][kk] * B[kk][col];
      bad += (c[i] != ref);
    }
  }
  {  // 16x16x16 with K = 16
    float fa[4], fb[4];
    for (int j = 0; j < 4; ++j) {
      fa[j] = A[l % 16][4 * (l / 16) + j];
      fb[j] = B[4 * (l / 16) + j][l % 16];
    }
    f32x4 c = mfma16k16(pack4(fa), pack4(fb), f32x4{});
    for (int i = 0; i < 4; ++i) {
      const int r = c16_row(i, l), col = l % 16;
      float ref = 0.f;
      for (int kk = 0; kk < 16; ++kk) ref += A[r][kk] * B[kk][col];
      bad += (c[i] != ref);
    }
  }
  {  // transposed LDS reads (tr_fragment) of a staged k-step tile: entry
     // (slot, value) holds the bits slot * 64 + value
    __shared__ __attribute__((aligned(16))) uint16_t tile[4 * 16 * 16];
    for (int i = l; i < 4 * 16 * 16; i += 64) {
      const int vb = i / 256, slot = (i / 16) % 16, vv = i % 16;
      tile[i] = (uint16_t)(slot * 64 + 16 * vb + vv);
    }
    __syncthreads();
    for (int n = 0; n < 2; ++n) {
      // compared as 32-bit words (two 16-bit elements each)
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 w = __builtin_bit_cast(u32x4, tr_fragment(reinterpret_cast<const __bf16*>(tile), l, n));
      for (int j = 0; j < 8; ++j) {
        const uint32_t got = (w[j >> 1] >> (16 * (j & 1))) & 0xffffu;
        bad += (got != (uint32_t)((8 * (l / 32) + j) * 64 + 32 * n + l % 32));
      }
    }
  }
  atomicAdd(errors, bad);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
MfmaSaved mfma_saved_view(void* base, int Hq, int U, int NB, int R) {
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    void* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  const size_t chunk = (size_t)kKS * 64 * 16 * sizeof(uint16_t);
  const size_t units = (size_t)U * NB;
  MfmaSaved v;
  v.wqs = static_cast<float*>(take(sizeof(float) * (size_t)Hq * kS));
  v.ic = static_cast<float*>(take(sizeof(float) * (size_t)Hq * kIC));
  v.gm = static_cast<float*>(take(sizeof(float) * (size_t)Hq * kD * kD));
  v.lb = static_cast<float*>(take(sizeof(float) * (size_t)Hq * kD));
  v.PR = static_cast<uint16_t*>(take(chunk * units));
  v.PZ = static_cast<float*>(take(sizeof(float) * units * kFP));
  v.PZm = static_cast<float*>(take(sizeof(float) * units * kD * kD));
  v.KT16 = static_cast<uint16_t*>(take(sizeof(uint16_t) * units * kD * kC));
  v.VT16 = static_cast<uint16_t*>(take(sizeof(uint16_t) * units * (kD + 1) * kC));
  v.KAP = static_cast<uint16_t*>(take(sizeof(uint16_t) * units * R * 3 * 64 * 16));
  v.Zt = static_cast<float*>(take(sizeof(float) * units * kZt));
  v.bytes = off;
  return v;
}

size_t mfma_saved_bytes(int Hq, int U, int NB, int R) { return mfma_saved_view(nullptr, Hq, U, NB, R).bytes; }

template <typename T>
void launch_mfma_forward(const LaunchGeom& g, const void* q, const void* k, const void* v, const int32_t* labels,
                         const float* c0, const float* lam, const float* gam, int groups, float scale, float floor,
                         void* out, float* num, float* den, void* saved, hipStream_t st, const Timer& timed) {
  MfmaSaved sv = mfma_saved_view(saved, g.Hq, g.U, g.NB, g.R);
  const T* qt = static_cast<const T*>(q);
  const T* kt = static_cast<const T*>(k);
  const T* vt = static_cast<const T*>(v);
  // the per-head slot coefficients in blocks of the same launch
  launch_fwd_prep<T>(g, kt, vt, sv.KT16, sv.VT16, sv.Zt,
                     SlotCoefArgs{labels, c0, lam, gam, groups, scale, sv.wqs, sv.ic, sv.gm, sv.lb}, st, timed);
  // denominator state (pair-matrix form): PZ, PZm as exclusive chunk prefixes
  launch_den_scan(true, g, sv.Zt, sv.PZ, sv.PZm, st, timed);
  {
    // num is written only later (k2_intra_fwd), so it doubles as the scan's
    // segment scratch
    const ScanPlan plan = scan_plan(g.U, g.NB, sizeof(float) * (size_t)g.B * g.Hq * g.N * kD, true);
    ScanArgs a{sv.KT16, kD, sv.VT16, kD + 1, nullptr, nullptr, g.U, g.Hq, g.Hkv, g.N, g.NB,
               sv.PR, num, nullptr, nullptr};
    launch_scan<true>(plan, a, st, timed);
  }
  timed("k2_intra_fwd", st, [&] {
    // more than 8 groups: per-pair coefficients, the feature-form local score
    if (groups > 8)
      hipLaunchKernelGGL((k2_intra_fwd<T, true>), dim3(g.R * g.NB * g.U), dim3(256), 0, st, qt, kt, vt, sv.PZ,
                         sv.PZm, labels, sv.ic, sv.gm, sv.lb, sv.wqs, groups, g.Hq, g.Hkv, g.N, g.NB, num, den,
                         sv.KAP);
    else
      hipLaunchKernelGGL((k2_intra_fwd<T, false>), dim3(g.R * g.NB * g.U), dim3(256), 0, st, qt, kt, vt, sv.PZ,
                         sv.PZm, labels, sv.ic, sv.gm, sv.lb, sv.wqs, groups, g.Hq, g.Hkv, g.N, g.NB, num, den,
                         sv.KAP);
  });
  timed("k2_out_fwd", st, [&] {
    // up to kMaxRS query heads per kv head: the heads share each copy of P_c
    if (g.R <= kMaxRS) {
      hipLaunchKernelGGL(k2_out_fwd_shared<T>, dim3(2 * g.NB * g.U), dim3(64 * (g.R + 1)), 0, st, qt, sv.wqs, sv.PR,
                         g.Hq, g.Hkv, g.N, g.NB, floor, static_cast<T*>(out), num, den);
      return;
    }
    hipLaunchKernelGGL(k2_out_fwd<T>, dim3(g.R * g.NB * g.U), dim3(128), 0, st, qt, sv.wqs, sv.PR, g.Hq, g.Hkv, g.N,
                       g.NB, floor, static_cast<T*>(out), num, den);
  });
}

template void launch_mfma_forward<float>(const LaunchGeom&, const void*, const void*, const void*, const int32_t*,
                                         const float*, const float*, const float*, int, float, float, void*, float*,
                                         float*, void*, hipStream_t, const Timer&);
template void launch_mfma_forward<uint16_t>(const LaunchGeom&, const void*, const void*, const void*, const int32_t*,
                                            const float*, const float*, const float*, int, float, float, void*,
                                            float*, float*, void*, hipStream_t, const Timer&);

int run_mfma_selftest(int* dev_errors, hipStream_t st) {
  hipLaunchKernelGGL(k2_selftest, dim3(1), dim3(64), 0, st, dev_errors);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace oal
