// bf16 matrix-core (MFMA) backward for gfx950.
//
// k2_bwd_prep   normalization VJP: G (bf16 token rows and transposed), Gz; transposed q.
// (the reverse chunk scan dT_c = sum_{c' > c} dCarry_c' and the per-slot
// coefficient partials are in oal_mfma_scan.hip)
// (the intra-chunk VJP, k2_local_dq / k2_local_dk / k2_local_dv, is in oal_mfma_local.hip)
// k2_q_fold     dq state part: D^T = P G^T on the MFMA, folded through the query
//               features (rotated rows, static register indices) + local dq.
// k2_kv_fold    dk state part (D^T = dT V^T folded through the key features)
//               and dv = raw(K) dT from one staged copy of the chunk's state,
//               the dTz quadratic form, + local dk, dv.
// k2_dwq_reduce sum of the per-segment slot-coefficient partials.
// k2_coef_grad  per head: slot gradients -> (dc0, dlam, dGam) + local parts.
//
// dGam follows the symmetric-Gam convention: off-diagonal entries carry the
// mean of the (g, h) and (h, g) routings, so that dGam = d/dGam of
// sum_{g,h} Gam_gh s_g s_h. (Gradients reaching a factor L with Gam = L L^T, or
// a per-pair coefficient c, are the same under either routing.)

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"
#include "oal_mfma_fold.hpp"

namespace oal {

static __constant__ SlotTable kSlot = make_slot_table();
using namespace fold;


// 16 consecutive elements of a row as fp32 (zeros when !ok).
__device__ __forceinline__ void load16f(const uint16_t* __restrict__ src, size_t off, bool ok, float (&x)[16]) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4* p = reinterpret_cast<const u32x4*>(src + off);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const u32x4 w = ok ? p[i] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
      x[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
}
__device__ __forceinline__ void load16f(const float* __restrict__ src, size_t off, bool ok, float (&x)[16]) {
  const float4* p = reinterpret_cast<const float4*>(src + off);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 a = ok ? p[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    x[4 * i] = a.x;
    x[4 * i + 1] = a.y;
    x[4 * i + 2] = a.z;
    x[4 * i + 3] = a.w;
  }
}

// Rows of the transposed per-head operands (QT16 / GT16): 64 feature or value
// rows, then row 64 (QT: 1 for tokens < N; GT: Gz) and row 65 (zeros).
constexpr int kTRows = kD + 2;

// ---------------------------------------------------------------------------
// Backward preparation, one block per (batch, query head, chunk):
// normalization VJP (reference hd_block_gemm_normalization_ops.py:32-71)
//   G = dO / den' + dnum,  Gz = -(dO . num) / den'^2 [den >= floor] + dden,
// den' = max(den, floor) (floor <= 0: den' = den, no mask), written as G16
// (token rows, bf16) and Gz (f32), plus the transposed bf16 operands of the
// backward state scan, GT16 = [G^T; Gz; 0] and QT16 = [q^T; 1; 0], each
// [B][Hq][66][NB * 64].
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k2_bwd_prep(const T* __restrict__ q, const T* __restrict__ dout,
                                                   const float* __restrict__ dnum, const float* __restrict__ dden,
                                                   const float* __restrict__ num, const float* __restrict__ den, int N,
                                                   int NB, float floor, uint16_t* __restrict__ G16,
                                                   float* __restrict__ Gz, uint16_t* __restrict__ GT16,
                                                   uint16_t* __restrict__ QT16) {
  constexpr int LT = kC + 8;
  __shared__ __attribute__((aligned(16))) __bf16 gT[kTRows][LT];
  __shared__ __attribute__((aligned(16))) __bf16 qT[kTRows][LT];
  const int bh = blockIdx.x / NB, ch = blockIdx.x % NB;
  const int tid = threadIdx.x, j = tid >> 2, qq = tid & 3;
  const int tok = ch * kC + j;
  const bool ok = tok < N;
  const size_t roff = ((size_t)bh * N + (ok ? tok : N - 1)) * kD + 16 * qq;
  float dO[16], nm[16], qv[16];
  if (dout) {
    load16f(dout, roff, ok, dO);
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) dO[e] = 0.f;
  }
  load16f(num, roff, ok, nm);
  load16f(q, roff, ok, qv);
  const float dd = ok ? den[(size_t)bh * N + tok] : 1.f;
  const float dp = floor > 0.f ? fmaxf(dd, floor) : dd;
  const float inv = 1.f / dp;
  float g[16], dot = 0.f;
  if (dnum) {
    float dn[16];
    load16f(dnum, roff, ok, dn);
#pragma unroll
    for (int e = 0; e < 16; ++e) g[e] = dO[e] * inv + dn[e];
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) g[e] = dO[e] * inv;
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) dot = fmaf(dO[e], nm[e], dot);
  dot += __shfl_xor(dot, 1, 64);
  dot += __shfl_xor(dot, 2, 64);
  float gz = -dot / (dp * dp);
  if (floor > 0.f && !(dd >= floor)) gz = 0.f;
  if (dden && ok) gz += dden[(size_t)bh * N + tok];
  if (!ok) gz = 0.f;
  {
    float y0[8], y1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y0[e] = ok ? g[e] : 0.f;
      y1[e] = ok ? g[8 + e] : 0.f;
    }
    const bf16x8 p0 = pack8(y0), p1 = pack8(y1);
    if (ok) {
      bf16x8* dst = reinterpret_cast<bf16x8*>(G16 + roff);
      dst[0] = p0;
      dst[1] = p1;
      if (qq == 0) Gz[(size_t)bh * N + tok] = gz;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      gT[16 * qq + e][j] = p0[e];
      gT[16 * qq + 8 + e][j] = p1[e];
      qT[16 * qq + e][j] = (__bf16)qv[e];
      qT[16 * qq + 8 + e][j] = (__bf16)qv[8 + e];
    }
    if (qq == 0) {
      gT[kD][j] = (__bf16)gz;
      gT[kD + 1][j] = (__bf16)0.f;
      qT[kD][j] = (__bf16)(ok ? 1.f : 0.f);
      qT[kD + 1][j] = (__bf16)0.f;
    }
  }
  __syncthreads();
  const size_t np = (size_t)NB * kC;
  for (int idx = tid; idx < kTRows * 8; idx += 256) {
    const int r = idx >> 3, c8 = idx & 7;
    const size_t o = ((size_t)bh * kTRows + r) * np + (size_t)ch * kC + 8 * c8;
    *reinterpret_cast<bf16x8*>(GT16 + o) = *reinterpret_cast<const bf16x8*>(&gT[r][8 * c8]);
    *reinterpret_cast<bf16x8*>(QT16 + o) = *reinterpret_cast<const bf16x8*>(&qT[r][8 * c8]);
  }
}

// ---------------------------------------------------------------------------
// Ring staging of k-blocked tiles (shared by the two waves of a fold block).
// One unit = 1024 bf16 (a PR M-tile k-slice of 32 x 16, or the four 512-byte
// R-layout pieces of a k-step).
// ---------------------------------------------------------------------------
constexpr int kFG = 4;  // units per ring group
constexpr int kNS = 4;  // LDS stages of a ring

// Fold ring: one 32-slot M-tile of a PR-layout state (4 k-slices x 32 rows x
// 16 values = 2048 bf16) per stage, kNS stages; 128 threads move 32 B each.
constexpr int kTileElems = 4 * 32 * 16;

// With CARRY, the stage also holds the same M-tile of a second state (the
// segment carry of k2_kv_fold) right after the first, and the products of both
// accumulate into one D: D = (A + A') B.
template <bool CARRY>
__device__ __forceinline__ void fold_issue(const uint16_t* src, const uint16_t* csrc, int m, __bf16* st, int tid) {
  const int wv = tid >> 6;
  const uint16_t* g = src + (size_t)m * kTileElems;
  copy16_to_lds(g + tid * 8, st + 64 * wv * 8);
  copy16_to_lds(g + (tid + 128) * 8, st + (128 + 64 * wv) * 8);
  if constexpr (CARRY) {
    const uint16_t* c = csrc + (size_t)m * kTileElems;
    copy16_to_lds(c + tid * 8, st + kTileElems + 64 * wv * 8);
    copy16_to_lds(c + (tid + 128) * 8, st + kTileElems + (128 + 64 * wv) * 8);
  }
}
template <bool CARRY>
constexpr int fold_copies() {
  return CARRY ? 4 : 2;
}

// D^T of M-tile M: 32 slots (rows, fold_row order) x 32 tokens (lane column).
template <int M, bool CARRY>
__device__ __forceinline__ f32x16 fold_mfma(const bf16x8 (&bfr)[4], const __bf16* tile, int lane) {
  const int s = lane >> 5, arow = fold_row(lane & 31);
  f32x16 D = f32x16{};
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    D = mfma32(*reinterpret_cast<const bf16x8*>(tile + kk * 512 + arow * 16 + 8 * s), bfr[kk], D);
  if constexpr (CARRY) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      D = mfma32(*reinterpret_cast<const bf16x8*>(tile + kTileElems + kk * 512 + arow * 16 + 8 * s), bfr[kk], D);
  }
  return D;
}

// Ring pipeline over the 69 M-tiles with NS LDS stages. Group G enters with
// the product of tile G in flight (Dc) and its slot weights read (wc, one
// register: fold_weight_row); it waits for tile G + 1, refills the stage of
// tile G (whose reads ended before the barrier) with tile G + NS, issues the
// product of tile G + 1 and reads its weights, then folds tile G, so the fold's
// VALU work overlaps the next tile's matrix products and LDS reads. Up to
// NS - 2 tiles stay in flight.
template <int G, int NS, bool CARRY>
__device__ __forceinline__ void fold_group(const bf16x8 (&bfr)[4], const float (&x)[kD], float (&dx)[kD],
                                           const float* wl, const LdsRing<NS>& ring, const uint16_t* src,
                                           const uint16_t* csrc, int tid, int lane, const f32x16& Dc, float wc) {
  constexpr int NT = kS / 32;  // 69 M-tiles
  if constexpr (G + 1 < NT) {
    constexpr int issued = (G + NS - 1 < NT - 1) ? G + NS - 1 : NT - 1;  // last tile issued so far
    pin64(dx);  // the fold of tile G - 1 stays in group G - 1
    ring_sync<fold_copies<CARRY>() * (issued - (G + 1))>();
    if constexpr (G + NS < NT) fold_issue<CARRY>(src, csrc, G + NS, ring.st[(G + NS) % NS], tid);
    const f32x16 Dn = fold_mfma<G + 1, CARRY>(bfr, ring.st[(G + 1) % NS], lane);
    const float wn = fold_weight_row<G + 1>(wl, lane);
    fold_tile_row<G>(Dc, x, dx, wc);
    fold_group<G + 1, NS, CARRY>(bfr, x, dx, wl, ring, src, csrc, tid, lane, Dn, wn);
  } else {
    fold_tile_row<G>(Dc, x, dx, wc);
  }
}

// Whole fold: tiles 0 .. NS - 1 in flight, product of tile 0, then the groups.
template <int NS, bool CARRY>
__device__ __forceinline__ void fold_all(const bf16x8 (&bfr)[4], const float (&x)[kD], float (&dx)[kD],
                                         const float* wl, const LdsRing<NS>& ring, const uint16_t* src,
                                         const uint16_t* csrc, int tid, int lane) {
  static_assert(NS >= 3 && NS <= kS / 32, "ring depth");
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (fold_issue<CARRY>(src, csrc, I, ring.st[I], tid), ...);
  }(std::make_integer_sequence<int, NS>{});
  ring_sync<fold_copies<CARRY>() * (NS - 1)>();
  const f32x16 D0 = fold_mfma<0, CARRY>(bfr, ring.st[0], lane);
  const float w0 = fold_weight_row<0>(wl, lane);
  fold_group<0, NS, CARRY>(bfr, x, dx, wl, ring, src, csrc, tid, lane, D0, w0);
}

// ---------------------------------------------------------------------------
// dq: state part of the query-side VJP, folded, plus the local part.
// grid (R, NB, U), 2 waves; wave w owns tokens 32w..32w+31 (lane column).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(128, 2) void k2_q_fold(const T* __restrict__ q, const uint16_t* __restrict__ G16,
                                                 const float* __restrict__ wqs, const uint16_t* __restrict__ PR,
                                                 const float* __restrict__ dqf, int Hq, int Hkv, int N, int NB,
                                                 int i0, int ni, T* __restrict__ dq) {
  __shared__ __attribute__((aligned(16))) __bf16 ring0[kTileElems], ring1[kTileElems], ring2[kTileElems],
      ring3[kTileElems], ring4[kTileElems], ring5[kTileElems];
  __shared__ __attribute__((aligned(16))) float wl[kS];
  const LdsRing<6> ring{{ring0, ring1, ring2, ring3, ring4, ring5}};

  int hh, ch, u;
  {
    // the launch covers items i0 .. i0 + ni - 1 of (unit, chunk, head), head
    // fastest; block ids are dealt to the 8 XCDs round-robin (see head_chunk_unit)
    const int id = blockIdx.x;
    const int w = i0 + ((ni & 7) == 0 ? (id & 7) * (ni >> 3) + (id >> 3) : id);
    const int R0 = Hq / Hkv;
    hh = w % R0;
    ch = (w / R0) % NB;
    u = w / (R0 * NB);
  }
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const uint16_t* src = PR + ((size_t)u * NB + ch) * ((size_t)kKS * 64 * 16);

  stage_f4<128, kS / 4>(reinterpret_cast<float4*>(wl), reinterpret_cast<const float4*>(wqs + (size_t)h * kS), tid);
  const int tok = tok0 + 32 * wv + row;
  const bool ok = tok < N;
  const size_t rowoff = qbase + (size_t)(ok ? tok : N - 1) * kD;
  float x[kD], dx[kD];
  bf16x8 bfr[4];
  load_rotated(q, rowoff, ok, s, x);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) bfr[kk] = frag8(G16, rowoff + 16 * kk + 8 * s, ok);
#pragma unroll
  for (int m = 0; m < kD; ++m) dx[m] = 0.f;
  fold_all<6, false>(bfr, x, dx, wl, ring, src, nullptr, tid, l);

  // lane group s writes dimensions 32 s .. 32 s + 31 of its token
  float full[32];
  combine_rotation_groups(dx, s, full);
  if (ok) {
    const size_t o = rowoff + 32 * s;
    const float4* lf = reinterpret_cast<const float4*>(dqf + o);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 a = lf[j];
      full[4 * j] += a.x;
      full[4 * j + 1] += a.y;
      full[4 * j + 2] += a.z;
      full[4 * j + 3] += a.w;
    }
    store32(dq + o, full);
  }
}

// ---------------------------------------------------------------------------
// dk, dv: the key-side state parts plus the per-head local parts, with the
// chunk's state read once. One block of 4 waves per (chunk, unit):
//   waves 0, 1 (tokens 32 w ..): dk = fold of dT V^T through the key features
//     + z1 + Mz k + local dk, Mz[r][c] = dTz[pair(r, c)] (r != c),
//     2 dTz[pair(r, r)] on the diagonal;
//   waves 2, 3 (tokens 32 (w - 2) ..): dv = raw(K) dT (values 0..63) + local dv.
// Both read one LDS ring of 32-slot M-tiles of dT; the dv waves take the B
// fragments of a tile's two k-steps by transposed reads at the M-tile's
// value-block stride. (Two blocks per chunk, one per part, each streaming the
// state: 79.4 -> 75.1 us at config 2.)
// CARRY: dT of chunk ch is the backward scan's segment-local state plus the
// carry of the chunk's segment (ch / SL, cR [U][S]); each ring stage holds the
// same M-tile of both, and both products of each step accumulate into the same
// registers, so the carry costs matrix products and staging only.
// ---------------------------------------------------------------------------
// B fragment of value half n of k-step half `half` (slots 16 half ..) of a
// staged M-tile [4 value blocks][32 slots][16 values]; the lane mapping of
// tr_fragment.
__device__ __forceinline__ bf16x8 tr_fragment_mtile(const __bf16* mtile, int half, int lane, int n) {
  const int g = lane >> 4, i = lane & 15;
  const __bf16* p = mtile + half * 256 + (2 * n + (g & 1)) * 512 + (8 * (g >> 1) + (i >> 2)) * 16 + 4 * (i & 3);
  typedef __attribute__((address_space(3))) trv4 lds_trv4;
  const trv4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_trv4*)(p));
  const trv4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_trv4*)(p + 4 * 16));
  typedef short trv8 __attribute__((ext_vector_type(8)));
  const trv8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}
template <int T, bool CARRY>
__device__ __forceinline__ void kvm_du_step(const float (&x)[kD], const __bf16* st, int lane, f32x16 (&acc)[2]) {
  const bf16x8 a = raw_fragment<T>(x);
  acc[0] = mfma32(a, tr_fragment_mtile(st, T & 1, lane, 0), acc[0]);
  acc[1] = mfma32(a, tr_fragment_mtile(st, T & 1, lane, 1), acc[1]);
  if constexpr (CARRY) {
    acc[0] = mfma32(a, tr_fragment_mtile(st + kTileElems, T & 1, lane, 0), acc[0]);
    acc[1] = mfma32(a, tr_fragment_mtile(st + kTileElems, T & 1, lane, 1), acc[1]);
  }
}
// M-tile m of the state (and of the carry) into stage st: 256 threads, one
// 16-byte copy each per tile.
template <bool CARRY>
__device__ __forceinline__ void kvm_issue(const uint16_t* src, const uint16_t* csrc, int m, __bf16* st, int tid) {
  const int wv = tid >> 6;
  copy16_to_lds(src + (size_t)m * kTileElems + tid * 8, st + 64 * wv * 8);
  if constexpr (CARRY) copy16_to_lds(csrc + (size_t)m * kTileElems + tid * 8, st + kTileElems + 64 * wv * 8);
}
template <bool CARRY>
constexpr int kvm_copies() {
  return CARRY ? 2 : 1;
}
// Group G: wait for tile G + 1, refill the stage of tile G with tile G + 4,
// then the dk waves issue the product of tile G + 1 and fold tile G, the dv
// waves take the products of tile G + 1's two k-steps. The two accumulator
// tiles acc serve both kinds of wave: the dv waves' dv accumulators, and the
// dk waves' products in flight (tile G's in acc[G % 2]), so that the kernel
// needs no more registers than the dk fold alone.
template <int G, bool CARRY>
__device__ __forceinline__ void kvm_group(bool dkw, const bf16x8 (&bfr)[4], const float (&x)[kD], float (&dx)[kD],
                                          f32x16 (&acc)[2], const LdsRing<4>& ring, const uint16_t* src,
                                          const uint16_t* csrc, int tid, int lane) {
  constexpr int NS = 4, NT = kS / 32;
  float w1[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) w1[i] = 1.f;
  if constexpr (G + 1 < NT) {
    constexpr int issued = (G + NS - 1 < NT - 1) ? G + NS - 1 : NT - 1;
    pin64(dx);
    ring_sync<kvm_copies<CARRY>() * (issued - (G + 1))>();
    if constexpr (G + NS < NT) kvm_issue<CARRY>(src, csrc, G + NS, ring.st[(G + NS) % NS], tid);
    if (dkw) {
      acc[(G + 1) & 1] = fold_mfma<G + 1, CARRY>(bfr, ring.st[(G + 1) % NS], lane);
      fold_tile<G>(acc[G & 1], x, dx, w1);
    } else {
      kvm_du_step<2 * (G + 1), CARRY>(x, ring.st[(G + 1) % NS], lane, acc);
      kvm_du_step<2 * (G + 1) + 1, CARRY>(x, ring.st[(G + 1) % NS], lane, acc);
    }
    kvm_group<G + 1, CARRY>(dkw, bfr, x, dx, acc, ring, src, csrc, tid, lane);
  } else {
    if (dkw) fold_tile<G>(acc[G & 1], x, dx, w1);
  }
}

// grid NB * U blocks of 4 waves. Block ids are dealt to the 8 XCDs
// round-robin; item w = (id % 8) * (total / 8) + id / 8 (chunk fastest, then
// unit) gives each XCD consecutive chunks of a unit, so that the chunks of a
// segment read its carry through one L2.
template <typename T, bool CARRY>
__global__ __launch_bounds__(256, 2) void k2_kv_fold(const T* __restrict__ k, const T* __restrict__ v,
                                                            const uint16_t* __restrict__ dTR,
                                                            const uint16_t* __restrict__ cR, int SL, int S,
                                                            const float* __restrict__ dTz,
                                                            const float* __restrict__ dkl,
                                                            const float* __restrict__ dvl, int Hq, int Hkv, int N,
                                                            int NB, T* __restrict__ dk, T* __restrict__ dv) {
  __shared__ __attribute__((aligned(16))) __bf16 ring0[kFG * 1024], ring1[kFG * 1024], ring2[kFG * 1024],
      ring3[kFG * 1024];
  __shared__ __attribute__((aligned(16))) __bf16 mz[kD][kD];

  int ch, u;
  {
    const int total = gridDim.x, id = blockIdx.x;
    const int w = (total & 7) == 0 ? (id & 7) * (total >> 3) + (id >> 3) : id;
    ch = w % NB;
    u = w / NB;
  }
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const bool dkw = wv < 2;
  const int tw = wv & 1;  // token half of the wave
  const int tok0 = ch * kC;
  const size_t kbase = (size_t)u * N * kD;
  const size_t cbase = ((size_t)u * NB + ch) * ((size_t)kKS * 64 * 16);
  const size_t sbase = ((size_t)u * S + (CARRY ? ch / SL : 0)) * ((size_t)kKS * 64 * 16);
  const int tok = tok0 + 32 * tw + row;
  const bool ok = tok < N;
  const size_t rowoff = kbase + (size_t)(ok ? tok : N - 1) * kD;
  float x[kD];
  load_rotated(k, rowoff, ok, s, x);
  const LdsRing<4> ring{{ring0, ring1, ring2, ring3}};
  const uint16_t* src = dTR + cbase;
  const uint16_t* csrc = CARRY ? cR + sbase : nullptr;

  const float* tz = dTz + ((size_t)u * NB + ch) * kFP;
  for (int idx = tid; idx < kD * kD; idx += 256) {
    const int r = idx >> 6, c = idx & 63;
    const int d = mz_dim(r >> 5, r & 31);
    const int hi = d > c ? d : c, lo = d > c ? c : d;
    const float val = tz[1 + kD + pair_index(hi, lo)];
    mz[r][(((c >> 3) ^ (r & 7)) << 3) | (c & 7)] = (__bf16)(d == c ? 2.f * val : val);
  }
  const float zv = tz[1 + (tid & 63)];
  bf16x8 bfr[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) bfr[kk] = frag8(v, rowoff + 16 * kk + 8 * s, ok);
  float dx[kD];
#pragma unroll
  for (int m = 0; m < kD; ++m) dx[m] = 0.f;
  f32x16 acc[2] = {f32x16{}, f32x16{}};
  static_assert(2 * kTileElems <= kFG * 1024, "a state tile and its carry tile fit one ring stage");
  kvm_issue<CARRY>(src, csrc, 0, ring.st[0], tid);
  kvm_issue<CARRY>(src, csrc, 1, ring.st[1], tid);
  kvm_issue<CARRY>(src, csrc, 2, ring.st[2], tid);
  kvm_issue<CARRY>(src, csrc, 3, ring.st[3], tid);
  ring_sync<kvm_copies<CARRY>() * 3>();
  if (dkw) {
    acc[0] = fold_mfma<0, CARRY>(bfr, ring.st[0], l);
  } else {
    kvm_du_step<0, CARRY>(x, ring.st[0], l, acc);
    kvm_du_step<1, CARRY>(x, ring.st[0], l, acc);
  }
  kvm_group<0, CARRY>(dkw, bfr, x, dx, acc, ring, src, csrc, tid, l);

  float* zl = reinterpret_cast<float*>(ring0);
  __syncthreads();
  if (tid < kD) zl[tid] = zv;
  __syncthreads();
  if (!dkw) {
    float lv[2][16];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int tj = min(tok0 + 32 * tw + c32_row(i, l), N - 1);
        lv[nt][i] = dvl[kbase + (size_t)tj * kD + 32 * nt + row];
      }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int tj = tok0 + 32 * tw + c32_row(i, l);
        if (tj < N) dv[kbase + (size_t)tj * kD + 32 * nt + row] = from_f<T>(acc[nt][i] + lv[nt][i]);
      }
    return;
  }
  float full[32];
  combine_rotation_groups(dx, s, full);
  bf16x8 kb[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) kb[kk] = frag8(k, rowoff + 16 * kk + 8 * s, ok);
#pragma unroll
  for (int md = 0; md < 2; ++md) {
    f32x16 z = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      z = mfma32(*reinterpret_cast<const bf16x8*>(&mz[32 * md + row][((2 * kk + s) ^ (row & 7)) << 3]), kb[kk], z);
#pragma unroll
    for (int i = 0; i < 16; ++i) full[16 * md + i] += z[i];
  }
  if (ok) {
    const size_t o = rowoff + 32 * s;
    const float4* lf = reinterpret_cast<const float4*>(dkl + o);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 a = lf[j];
      full[4 * j] += a.x + zl[32 * s + 4 * j];
      full[4 * j + 1] += a.y + zl[32 * s + 4 * j + 1];
      full[4 * j + 2] += a.z + zl[32 * s + 4 * j + 2];
      full[4 * j + 3] += a.w + zl[32 * s + 4 * j + 3];
    }
    store32(dk + o, full);
  }
}

// Grid (slot blocks + ncol + den blocks, Hq). Slot blocks: dwq[h][slot] = sum
// over (segment, batch) of the state-scan partials (per-pair path: plus the
// sum over (batch, chunk, query tile) of the local slot partials dwql). The next 73 blocks of a
// head: one column of the per-(batch, chunk) local partials each, coefs[h][j]
// = sum_r coefl[h][j][r]. The den blocks (64 entries each): dwqz[h][nat] =
// sum over (batch, chunk) of the denominator partials dwz [U][NB][R][kFP], the
// (batch, chunk) rows split over the block's 4 waves (8 loads in flight each),
// then combined. Every sum in a fixed order.
constexpr int kDwqSlotBlocks = (kS + 255) / 256;
constexpr int kDwqDenBlocks = (kFeat + 63) / 64;
__global__ __launch_bounds__(256) void k2_dwq_reduce(const float* __restrict__ dwqs, int rowsets, int Hq,
                                                     float* __restrict__ dwq, const float* __restrict__ coefl, int bn,
                                                     float* __restrict__ coefs, const float* __restrict__ dwz, int B,
                                                     int Hkv, int NB, float* __restrict__ dwqz,
                                                     const float* __restrict__ dwql, int lrows, int ncol) {
  const int h = blockIdx.y;
  if (blockIdx.x >= kDwqSlotBlocks + ncol) {
    // 64 entries per block; lane l reads entries 4 (l % 16) .. as a float4 of
    // row-group l / 16 + 4 wave, rows (batch, chunk) i = group + 16 x
    __shared__ float dpart[16][64];
    const int l = threadIdx.x & 63, wv = threadIdx.x >> 6, grp = (l >> 4) + 4 * wv, e4 = 4 * (l & 15);
    const int n0 = (blockIdx.x - kDwqSlotBlocks - ncol) * 64;
    const int R = Hq / Hkv, kh = h / R, hh = h % R;
    const int rows = B * NB;  // row i = (batch i / NB, chunk i % NB)
    auto row_ptr = [&](int i) {
      const int bb = i / NB, c = i % NB;
      return dwz + (((size_t)(bb * Hkv + kh) * NB + c) * R + hh) * kFP + n0 + e4;
    };
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int i = grp;
    for (; i + 16 * 7 < rows; i += 16 * 8) {
      float4 v[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) v[x] = *reinterpret_cast<const float4*>(row_ptr(i + 16 * x));
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        acc.x += v[x].x;
        acc.y += v[x].y;
        acc.z += v[x].z;
        acc.w += v[x].w;
      }
    }
    for (; i < rows; i += 16) {
      const float4 v = *reinterpret_cast<const float4*>(row_ptr(i));
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    *reinterpret_cast<float4*>(&dpart[grp][e4]) = acc;
    __syncthreads();
    const int n = n0 + threadIdx.x;
    if (threadIdx.x < 64 && n < kFeat) {
      float t = 0.f;
#pragma unroll
      for (int g = 0; g < 16; ++g) t += dpart[g][threadIdx.x];
      dwqz[(size_t)h * kFP + n] = t;
    }
    return;
  }
  if (blockIdx.x >= kDwqSlotBlocks) {
    __shared__ float wsum[4];
    const int j = blockIdx.x - kDwqSlotBlocks;
    const float* p = coefl + ((size_t)h * 73 + j) * bn;
    float acc = 0.f;
    for (int r = threadIdx.x; r < bn; r += 256) acc += p[r];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) coefs[(size_t)h * 73 + j] = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    return;
  }
  const int sl = blockIdx.x * 256 + threadIdx.x;
  if (sl >= kS) return;
  // fixed order; eight loads in flight at a time
  const float* p = dwqs + (size_t)h * kS + sl;
  const size_t st = (size_t)Hq * kS;
  float acc = 0.f;
  int r = 0;
  for (; r + 8 <= rowsets; r += 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = p[(size_t)(r + i) * st];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += v[i];
  }
  for (; r < rowsets; ++r) acc += p[(size_t)r * st];
  if (dwql) {
    // per-pair path: the local partials of every (batch, chunk, query tile) row
    const float* lp = dwql + (size_t)h * lrows * kS + sl;
    float lacc = 0.f;
    int i = 0;
    for (; i + 8 <= lrows; i += 8) {
      float v[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) v[x] = lp[(size_t)(i + x) * kS];
#pragma unroll
      for (int x = 0; x < 8; ++x) lacc += v[x];
    }
    for (; i < lrows; ++i) lacc += lp[(size_t)i * kS];
    acc += lacc;
  }
  dwq[(size_t)h * kS + sl] = acc;
}

// ---------------------------------------------------------------------------
// Coefficient gradients, one block per query head, every sum in a fixed order.
// State part: the per-slot gradients (summed over the batch) are laid out in
// natural feature order wn[f]; dc0 = wn[0], dlam[g] = scale sum_{g(d)=g} wn[1+d],
// and the pair part routes pair (r >= c) to [g(r)][g(c)] through
// X[r][g] = sum_{c <= r, g(c) = g} m_rc wn[pair(r, c)], raw = E^T X with E the
// one-hot label matrix. Local part: the column sums of the per-chunk partials
// (coefs, from k2_dwq_reduce).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k2_coef_grad(const float* __restrict__ dwq, const float* __restrict__ dwqz,
                                                    const float* __restrict__ coefs,
                                                    const int32_t* __restrict__ labels, int Hq, int G, float scale,
                                                    float* __restrict__ dc0, float* __restrict__ dlam,
                                                    float* __restrict__ dgam) {
  __shared__ float wn[kFeat];
  __shared__ float loc[73];
  __shared__ float xr[kD][9];
  __shared__ float xq[4][kD][9];
  __shared__ float raw[64];
  __shared__ int lab[kD];
  const int h = blockIdx.x, t = threadIdx.x;
  if (t < kD) {
    int g = labels[h * kD + t];
    lab[t] = g < 0 ? 0 : (g >= G ? G - 1 : g);
  }
  // every global load of the thread in flight together (clamped indices, the
  // clamped copies unused)
  constexpr int kJS = (kS + 255) / 256, kJF = (kFeat + 255) / 256;
  float a[kJS], z[kJF];
#pragma unroll
  for (int j = 0; j < kJS; ++j) a[j] = dwq[(size_t)h * kS + min(t + 256 * j, kS - 1)];
#pragma unroll
  for (int j = 0; j < kJF; ++j) z[j] = dwqz[(size_t)h * kFP + min(t + 256 * j, kFeat - 1)];
  const float lc = coefs[(size_t)h * 73 + min(t, 72)];
  int nat[kJS];
#pragma unroll
  for (int j = 0; j < kJS; ++j) nat[j] = kSlot.nat[min(t + 256 * j, kS - 1)];
#pragma unroll
  for (int j = 0; j < kJS; ++j)
    if (t + 256 * j < kS && nat[j] >= 0) wn[nat[j]] = a[j];
  if (t < 73) loc[t] = lc;
  __syncthreads();
  // plus the denominator state's partials (natural order)
#pragma unroll
  for (int j = 0; j < kJF; ++j)
    if (t + 256 * j < kFeat) wn[t + 256 * j] += z[j];
  __syncthreads();
  // xr[r][g] = sum_{c <= r, g(c) = g} m_rc wn[pair(r, c)]: thread (r, q) sums the
  // columns c = q mod 4 into eight group bins, then the four quarters are added
  // in a fixed order
  {
    const int r = t >> 2, q = t & 3;
    float bin[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) bin[g] = 0.f;
    const float* row = wn + 1 + kD + pair_index(r, 0);
    for (int c = q; c <= r; c += 4) {
      const float x = (c == r ? 1.f : 2.f) * row[c];
      const int lc = lab[c];
#pragma unroll
      for (int g = 0; g < 8; ++g) bin[g] += lc == g ? x : 0.f;
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) xq[q][r][g] = bin[g];
  }
  __syncthreads();
  for (int e = t; e < kD * 8; e += 256) {
    const int r = e >> 3, g = e & 7;
    xr[r][g] = g < G ? (xq[0][r][g] + xq[1][r][g]) + (xq[2][r][g] + xq[3][r][g]) : 0.f;
  }
  __syncthreads();
  // raw[gr][gc] = scale^2 sum_{r: g(r) = gr} xr[r][gc]: thread (gr, gc, q) sums
  // the rows r = q mod 4, then the quarters in a fixed order
  {
    const int e = t >> 2, q = t & 3, gr = e >> 3, gc = e & 7;
    float acc = 0.f;
    for (int r = q; r < kD; r += 4) acc += lab[r] == gr ? xr[r][gc] : 0.f;
    xq[q][e][0] = acc;
  }
  __syncthreads();
  if (t < G * G) {
    const int gr = t / G, gc = t % G, e = 8 * gr + gc;
    raw[t] = ((xq[0][e][0] + xq[1][e][0]) + (xq[2][e][0] + xq[3][e][0])) * scale * scale;
  }
  if (t == 64) dc0[h] = wn[0] + loc[0];
  if (t >= 128 && t < 128 + G) {
    const int g = t - 128;
    float acc = 0.f;
    for (int d = 0; d < kD; ++d)
      if (lab[d] == g) acc += wn[1 + d];
    dlam[(size_t)h * G + g] = acc * scale + loc[1 + g];
  }
  __syncthreads();
  if (t < G * G) {
    const int gr = t / G, gc = t % G;
    const float sym = gr == gc ? raw[t] : 0.5f * (raw[t] + raw[gc * G + gr]);
    dgam[(size_t)h * G * G + t] = sym + loc[9 + 8 * gr + gc];
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Workspace carve-up of the backward; the state scan's segment count comes
// from scan_plan (oal_mfma_scan.hip), which sizes the segment-totals buffer.
MfmaWork mfma_work_view(void* base, int B, int Hq, int U, int N, int NB, bool pairwise) {
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    void* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  const size_t rows = (size_t)B * Hq * N;
  const size_t trows = (size_t)B * Hq * kTRows * NB * kC;
  const size_t chunk = (size_t)kKS * 64 * 16 * sizeof(uint16_t);
  MfmaWork w;
  const ScanPlan plan = bwd_scan_plan(U, NB, B * Hq / U);
  w.S = plan.S;
  w.SL = plan.SL;
  w.G16 = static_cast<uint16_t*>(take(rows * kD * sizeof(uint16_t)));
  w.Gz = static_cast<float*>(take(rows * sizeof(float)));
  w.GT16 = static_cast<uint16_t*>(take(trows * sizeof(uint16_t)));
  w.QT16 = static_cast<uint16_t*>(take(trows * sizeof(uint16_t)));
  w.dTR = static_cast<uint16_t*>(take(chunk * U * NB));
  w.dTz = static_cast<float*>(take(sizeof(float) * (size_t)U * NB * kFP));
  w.dCt = static_cast<float*>(take(sizeof(float) * (size_t)U * NB * kZt));
  w.dwz = static_cast<float*>(take(sizeof(float) * (size_t)B * Hq * NB * kFP));
  w.dwqz = static_cast<float*>(take(sizeof(float) * (size_t)Hq * kFP));
  w.dwqs = static_cast<float*>(take(sizeof(float) * (size_t)w.S * B * Hq * kS));
  w.dwq = static_cast<float*>(take(sizeof(float) * (size_t)Hq * kS));
  w.segtot = static_cast<float*>(take(plan.seg_bytes));
  w.dqf = static_cast<float*>(take(rows * kD * sizeof(float)));
  w.dkl = static_cast<float*>(take((size_t)U * N * kD * sizeof(float)));
  w.dvl = static_cast<float*>(take((size_t)U * N * kD * sizeof(float)));
  w.coefl = static_cast<float*>(take(sizeof(float) * (size_t)B * Hq * NB * 73));
  w.coefs = static_cast<float*>(take(sizeof(float) * (size_t)Hq * 73));
  w.dkp = pairwise ? static_cast<float*>(take(rows * kD * sizeof(float))) : nullptr;
  w.dwql = pairwise ? static_cast<float*>(take(sizeof(float) * (size_t)Hq * B * NB * 2 * kS)) : nullptr;
  w.dCR = plan.S > 1 ? static_cast<uint16_t*>(take(chunk * U * plan.S)) : nullptr;
  w.bytes = off;
  return w;
}

template <typename T>
int launch_mfma_backward(const LaunchGeom& g, const void* q, const void* k, const void* v, const int32_t* labels,
                         const float* c0, const float* lam, const float* gam, int groups, float scale, float floor,
                         const float* num, const float* den, const void* saved, const void* dout, const float* dnum,
                         const float* dden, void* dq, void* dk, void* dv, float* dc0, float* dlam, float* dgam,
                         void* workspace, hipStream_t st, hipStream_t aux, const Timer& timed) {
  if ((dk != nullptr) != (dv != nullptr)) return 2;
  const bool need_coef = dc0 || dlam || dgam;
  if (need_coef && !(dc0 && dlam && dgam)) return 3;
  MfmaSaved sv = mfma_saved_view(const_cast<void*>(saved), g.Hq, g.U, g.NB, g.R);
  const bool pairwise = groups > 8;
  MfmaWork w = mfma_work_view(workspace, g.B, g.Hq, g.U, g.N, g.NB, pairwise);
  const T* qt = static_cast<const T*>(q);
  const T* kt = static_cast<const T*>(k);
  const T* vt = static_cast<const T*>(v);
  const bool forked = aux != st;
  // the fork, the second stream's mid-call events and the join are recorded
  // by the launches of the kernels they follow (not while st is capturing)
  const bool sig = forked && !capturing(st);
  const hipEvent_t ev_fork = sig ? next_event() : nullptr;
  timed("k2_bwd_prep", st, [&] {
    launch_signal(k2_bwd_prep<T>, dim3(g.B * g.Hq * g.NB), dim3(256), st, ev_fork, qt, static_cast<const T*>(dout),
                  dnum, dden, num, den, g.N, g.NB, floor, w.G16, w.Gz, w.GT16, w.QT16);
  });
  // Two streams, joined only at the end. The second stream: (group-sum path)
  // the intra-chunk dv, whose small footprint (58 VGPRs, 8 KB of LDS) fits
  // beside the state scan's blocks; (at up to 128 chunks per unit) the
  // denominator kernels, which need only what k2_bwd_prep and the forward
  // wrote; the intra-chunk dk, then dq, then the query-side fold (or the
  // first 7/8 or 3/4 of its items). The caller's stream: the state scan and
  // its carry, (otherwise the denominator kernels,) (per pair) the intra-chunk
  // dv, the key-side fold after an event recorded behind the dk kernel, then
  // the rest of the query-side fold and the coefficient reductions after the
  // dq kernel's event. (Measured, per config-2 step, same
  // box: 0.8505 ms with the denominator kernels on the caller's stream and the
  // whole query-side fold on the second stream, 0.8441 with the denominator
  // kernels moved, 0.8363 with the fold also split 6/2 over the 8 units (a 4/4
  // or 5/3 split: 0.844 and 0.849); on another box 0.8090 -> 0.7954 ms with
  // the dv kernel moved to the caller's stream.)
  const LocalBwdArgs la{w.G16, w.Gz, w.QT16, w.GT16, sv.KT16, sv.KAP, sv.PZ, sv.PZm, labels, lam, gam, sv.ic, sv.gm,
                        sv.lb, groups, scale, w.dqf, w.dkl, w.dvl, (need_coef && !pairwise) ? w.coefl : nullptr,
                        pairwise, sv.wqs, w.dkp, (need_coef && pairwise) ? w.dwql : nullptr};
  // the query-side fold of items i0 .. i0 + ni - 1 of (unit, chunk, head)
  auto q_fold = [&](hipStream_t s, int i0, int ni, hipEvent_t stop) {
    if (dq && ni > 0) {
      timed("k2_q_fold", s, [&] {
        launch_signal(k2_q_fold<T>, dim3(ni), dim3(128), s, stop, qt, w.G16, sv.wqs, sv.PR, w.dqf, g.Hq, g.Hkv, g.N,
                      g.NB, i0, ni, static_cast<T*>(dq));
      });
    }
  };
  const int nq = g.R * g.NB * g.U;  // query-side fold items
  // denominator state (pair-matrix form): per-chunk dCarry and coefficient
  // partials, then dTz as the exclusive chunk suffix
  auto den_state = [&](hipStream_t s) {
    launch_den_bwd(g, w.QT16, w.GT16, kTRows, sv.gm, sv.lb, sv.ic, kIC, sv.PZ, sv.PZm, w.dCt,
                   need_coef ? w.dwz : nullptr, s, timed);
    launch_den_scan(false, g, w.dCt, w.dTz, nullptr, s, timed);
  };
  hipEvent_t ev_dkv = nullptr, ev_dq = nullptr;
  // The denominator kernels go to the second stream for the group-sum path at
  // up to 128 chunks per unit, and follow the scan on the caller's stream
  // otherwise: measured at N = 4096 (64 chunks) the second stream is 22 us per
  // step faster, at N = 32768 (512 chunks) 50 us slower, and on the per-pair
  // path (whose key-side fold waits for the dq part) no faster. The dv kernel
  // heads the second stream on the group-sum path (config 2 0.8015 -> 0.7886
  // ms per step with the fold split 7/8, config 3 1.660 -> 1.640 ms with the
  // fold whole; on the caller's stream after the scan before). The second
  // stream runs the query-side fold's first items: 7/8 of them (rounded up)
  // where it also has the denominator kernels, all of them on the group-sum
  // path otherwise, 3/4 on the per-pair path; the rest follows the key-side
  // fold on the caller's stream.
  const bool den_aux = forked && !pairwise && g.NB <= 128;
  const bool dv_aux = forked && !pairwise;
  const bool dv_main = forked && !dv_aux;
  const int na = !forked ? nq : pairwise ? (3 * nq + 3) / 4 : den_aux ? (7 * nq + 7) / 8 : nq;
  hipEvent_t ev_join = nullptr;
  if (forked) {
    if (ev_fork)
      wait_event(aux, ev_fork);
    else
      stream_wait(aux, st);
    if (dv_aux) launch_local_bwd<T>(g, qt, kt, vt, la, dq != nullptr, dk != nullptr, kLocalDv, aux, timed);
    if (den_aux) den_state(aux);
    ev_dkv = sig ? next_event() : nullptr;
    if (!launch_local_bwd<T>(g, qt, kt, vt, la, dq != nullptr, dk != nullptr, kLocalDk, aux, timed, ev_dkv))
      ev_dkv = record_event(aux);
    ev_dq = sig ? next_event() : nullptr;
    if (!launch_local_bwd<T>(g, qt, kt, vt, la, dq != nullptr, dk != nullptr, kLocalDq, aux, timed, ev_dq))
      ev_dq = record_event(aux);
    // the fold is the second stream's last kernel: its launch records the join
    ev_join = sig && dq && na > 0 ? next_event() : nullptr;
    q_fold(aux, 0, na, ev_join);
  }
  {
    const ScanPlan plan{w.S, w.SL, 0};
    // without a coefficient gradient the scan forms no coefficient partials
    ScanArgs a{w.QT16, kTRows, w.GT16, kTRows, sv.wqs, sv.PR, g.U, g.Hq, g.Hkv, g.N, g.NB,
               w.dTR, w.segtot, need_coef ? w.dwqs : nullptr, w.dCR};
    launch_scan<false>(plan, a, st, timed);
    if (!den_aux) den_state(st);
  }
  // per pair, the dv kernel (it needs only the forward's kappa and
  // k2_bwd_prep's G^T) on the caller's stream, which would otherwise wait for
  // the dq part's event
  if (dv_main) launch_local_bwd<T>(g, qt, kt, vt, la, dq != nullptr, dk != nullptr, kLocalDv, st, timed);
  if (!forked) {
    // one stream (the allocation-free entry point, the profiling mode, a call
    // made during a graph capture before the second stream exists): the state
    // side first, then the intra-chunk VJP and the query-side fold (on one
    // stream 0.950-0.951 ms per config-2 step, against 0.955 with the
    // intra-chunk VJP first)
    launch_local_bwd<T>(g, qt, kt, vt, la, dq != nullptr, dk != nullptr, kLocalDq | kLocalDkv, st, timed);
    q_fold(st, 0, nq, nullptr);
  }
  if (dk) {
    // the per-pair path forms its local dk in the dq part's launch
    if (forked) wait_event(st, pairwise ? ev_dq : ev_dkv);
    timed("k2_kv_fold", st, [&] {
      if (w.S > 1)
        hipLaunchKernelGGL((k2_kv_fold<T, true>), dim3(g.NB * g.U), dim3(256), 0, st, kt, vt, w.dTR, w.dCR, w.SL,
                           w.S, w.dTz, w.dkl, w.dvl, g.Hq, g.Hkv, g.N, g.NB, static_cast<T*>(dk),
                           static_cast<T*>(dv));
      else
        hipLaunchKernelGGL((k2_kv_fold<T, false>), dim3(g.NB * g.U), dim3(256), 0, st, kt, vt, w.dTR, nullptr, 1,
                           1, w.dTz, w.dkl, w.dvl, g.Hq, g.Hkv, g.N, g.NB, static_cast<T*>(dk),
                           static_cast<T*>(dv));
    });
  }
  if (forked && (need_coef || na < nq)) wait_event(st, ev_dq);
  if (forked) q_fold(st, na, nq - na, nullptr);
  if (need_coef) {
    // group-sum path: the 73 local coefficient columns; per-pair path: the
    // local slot partials added to the state's
    const int ncol = pairwise ? 0 : 73;
    timed("k2_dwq_reduce", st, [&] {
      hipLaunchKernelGGL(k2_dwq_reduce, dim3(kDwqSlotBlocks + ncol + kDwqDenBlocks, g.Hq), dim3(256), 0, st, w.dwqs,
                         g.B * w.S, g.Hq, w.dwq, w.coefl, g.B * g.NB, w.coefs, w.dwz, g.B, g.Hkv, g.NB, w.dwqz,
                         pairwise ? w.dwql : nullptr, g.B * g.NB * 2, ncol);
    });
    if (pairwise) {
      launch_pair_coef_grad(g, w.dwq, w.dwqz, labels, groups, scale, dc0, dlam, dgam, st, timed);
    } else {
      timed("k2_coef_grad", st, [&] {
        hipLaunchKernelGGL(k2_coef_grad, dim3(g.Hq), dim3(256), 0, st, w.dwq, w.dwqz, w.coefs, labels, g.Hq, groups,
                           scale, dc0, dlam, dgam);
      });
    }
  }
  // the caller's stream ends after every kernel of the call
  if (ev_join)
    wait_event(st, ev_join);
  else if (forked)
    stream_wait(st, aux);
  return 0;
}

template int launch_mfma_backward<float>(const LaunchGeom&, const void*, const void*, const void*, const int32_t*,
                                         const float*, const float*, const float*, int, float, float, const float*,
                                         const float*, const void*, const void*, const float*, const float*, void*,
                                         void*, void*, float*, float*, float*, void*, hipStream_t, hipStream_t,
                                         const Timer&);
template int launch_mfma_backward<uint16_t>(const LaunchGeom&, const void*, const void*, const void*, const int32_t*,
                                            const float*, const float*, const float*, int, float, float,
                                            const float*, const float*, const void*, const void*, const float*,
                                            const float*, void*, void*, void*, float*, float*, float*, void*,
                                            hipStream_t, hipStream_t, const Timer&);

}  // namespace oal
