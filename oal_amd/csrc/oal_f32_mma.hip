// fp32 route on the gfx950 matrix cores (v_mfma_f32_32x32x2f32), for up to 8
// groups: the same chunked feature form as the scalar fp32 kernels of
// oal_kernels.hip (and the same natural-order fp32 state buffers, so the
// saved state is interchangeable), with the 2145-wide state contractions on
// the matrix cores and the intra-chunk terms in group-sum form.
//
//   k3_state_fwd   P_c = sum_{c' < c} raw(K_c')^T [V_c', 1]          (exclusive prefix)
//   k3_intra_fwd   intra-chunk num and den (group sums on the matrix cores)
//   k3_state_bwd   dT_c = sum_{c' > c} sum_h wq_h o raw(Q_h,c')^T [G, Gz]_h,c'
//                  in chunk segments (k3_seg_carry turns the segment totals
//                  into carries, which the dk and dv kernels add as they
//                  stage dT) and the state part of the feature-coefficient
//                  gradient dwq_part[b][h][c][f] = <P_c[f], raw(Q_h,c)^T [G, Gz]_h,c[f]>
//   k3_readout     num += phi(x) . S (out: num / den), or dv = raw(K) dT + local
//   k3_fold        dq = fold of (P [G, Gz]^T) through wq o raw(q) + local,
//                  dk = fold of (dT [V, 1]^T) through raw(k) + local
//   k3_local       local dq (part 0), and dk, dv and coefficient partials
//                  (part 1), group sums on the matrix cores
//   k3_coef_reduce per-head sums of those partials
//
// Matrix layout of v_mfma_f32_32x32x2f32: lane l supplies A[l % 32][l / 32]
// and B[l / 32][l % 32]; accumulator register i of lane l holds
// C[8 (i / 4) + 4 (l / 32) + i % 4][l % 32] (the 32 x 32 layout of the bf16
// kernels). The K index pairs (k, lane group s) are mapped to the contracted
// dimension in whatever order keeps the operand loads contiguous; both
// operands use the same map.
//
// Reference: the feature-form state terms follow hd_block_gemm_runtime.py
// :271-320 (block totals, exclusive prefix), :411-614 (query readout) and
// hd_block_gemm_backward.py :473-761 (query-side VJP), :764-908 (dCarry and
// its right scan), :1031-1452 (key/value-side VJP); the local terms follow
// the closed-form VJP of grouped_reference.py:214-318 in group-sum form.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "oal_common.hpp"
#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"
#include "oal_mfma_fold.hpp"

namespace oal {

namespace {

__constant__ FeatureTable kTab3 = make_feature_table();
__constant__ SlotTable kSlot3 = make_slot_table();

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// The other lane group's value of x (lanes l and l ^ 32).
__device__ __forceinline__ float partner(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// 16 consecutive elements of a token row as fp32 (zeros when !ok).
__device__ __forceinline__ void load16(const float* __restrict__ src, size_t off, bool ok, float (&v)[16]) {
  const float4* p = reinterpret_cast<const float4*>(src + off);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 a = p[i];
    v[4 * i] = ok ? a.x : 0.f;
    v[4 * i + 1] = ok ? a.y : 0.f;
    v[4 * i + 2] = ok ? a.z : 0.f;
    v[4 * i + 3] = ok ? a.w : 0.f;
  }
}
__device__ __forceinline__ void load16(const uint16_t* __restrict__ src, size_t off, bool ok, float (&v)[16]) {
  const uint4* p = reinterpret_cast<const uint4*>(src + off);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint4 a = p[i];
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[8 * i + 2 * e] = ok ? __uint_as_float(w[e] << 16) : 0.f;
      v[8 * i + 2 * e + 1] = ok ? __uint_as_float(w[e] & 0xffff0000u) : 0.f;
    }
  }
}

// Rotated fp32 row x[m] = row[(m + 32 s) % 64], exact (the bf16 route's
// load_rotated rounds its input to bf16).
template <typename T>
__device__ __forceinline__ void load_rotated_f32(const T* __restrict__ src, size_t row_base, bool ok, int s,
                                                 float (&x)[kD]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v[16];
    load16(src, row_base + ((16 * i + 32 * s) & 63), ok, v);
#pragma unroll
    for (int j = 0; j < 16; ++j) x[16 * i + j] = v[j];
  }
}

// Thread t of a 256-thread block holds dims 16 (t % 4) .. + 15 of token t / 4
// of a chunk; rows past N are zero.
template <typename T>
__device__ __forceinline__ void load_chunk_rows(const T* __restrict__ src, size_t base, int tok0, int N,
                                                float (&v)[16]) {
  const int j = threadIdx.x >> 2, q4 = threadIdx.x & 3, tok = tok0 + j;
  const bool ok = tok < N;
  load16(src, base + (size_t)(ok ? tok : N - 1) * kD + 16 * q4, ok, v);
}
template <int LDW>
__device__ __forceinline__ void store_chunk_rows(float (*dst)[LDW], const float (&v)[16]) {
  const int j = threadIdx.x >> 2, q4 = threadIdx.x & 3;
#pragma unroll
  for (int i = 0; i < 16; ++i) dst[j][16 * q4 + i] = v[i];
}

// Stores this lane's accumulator values (rows 32 m + 8 a + 4 s + 0..3 of
// the value dimension) into row f of a [.][64] state.
__device__ __forceinline__ void store_state_row(float* __restrict__ row, int m, int s, const f32x16& acc) {
#pragma unroll
  for (int a = 0; a < 4; ++a)
    *reinterpret_cast<float4*>(row + 32 * m + 8 * a + 4 * s) =
        make_float4(acc[4 * a], acc[4 * a + 1], acc[4 * a + 2], acc[4 * a + 3]);
}

}  // namespace

// ---------------------------------------------------------------------------
// Forward state scan: block (64-feature slice, unit), 4 waves; wave w owns
// features 64 x + 32 (w / 2) + lane % 32 (lane column) and values
// 32 (w % 2) .. + 31 (accumulator rows). Per chunk: emit the prefix, then add
// raw(K_c)^T [V_c, 1] as D^T[e][f] = sum_t V[t][e] raw_f(k_t) (K = tokens,
// token 32 s + k at step k), the ones column as a per-lane sum.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k3_state_fwd(const T* __restrict__ k, const T* __restrict__ v, int N, int NB,
                                                    float* __restrict__ carry, float* __restrict__ carry_z) {
  __shared__ float kx[kC][kRow];   // [k, 1 (token < N), 0]
  __shared__ float vx[kC][kD + 1];
  const int u = blockIdx.y, tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int m = wv & 1, f = blockIdx.x * 64 + 32 * (wv >> 1) + row;
  const int r = kTab3.r[f], c = kTab3.c[f];
  const size_t base = (size_t)u * N * kD;
  float kr[16], vr[16];
  load_chunk_rows(k, base, 0, N, kr);
  load_chunk_rows(v, base, 0, N, vr);
  f32x16 acc = f32x16{};
  float accz = 0.f;
  for (int ch = 0; ch < NB; ++ch) {
    const size_t cb = (size_t)u * NB + ch;
    store_state_row(carry + (cb * kFP + f) * kD, m, s, acc);
    const float zt = accz + partner(accz);
    if (m == 0 && s == 0) carry_z[cb * kFP + f] = zt;
    lds_sync();
    store_chunk_rows(kx, kr);
    store_chunk_rows(vx, vr);
    if ((tid & 3) == 0) {
      kx[tid >> 2][kD] = ch * kC + (tid >> 2) < N ? 1.f : 0.f;
      kx[tid >> 2][kD + 1] = 0.f;
    }
    lds_sync();
    if (ch + 1 < NB) {
      load_chunk_rows(k, base, (ch + 1) * kC, N, kr);
      load_chunk_rows(v, base, (ch + 1) * kC, N, vr);
    }
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      const int t = 32 * s + kk;
      const float phi = kx[t][r] * kx[t][c];
      acc = mfma_f32(vx[t][32 * m + row], phi, acc);
      accz += phi;
    }
  }
}

// ---------------------------------------------------------------------------
// Backward state scan: block (64-feature slice, unit, segment), waves as
// above; walks the segment's chunks downwards, the unit's query heads within a
// chunk. Per item (chunk, head): H = raw(Q)^T [G, Gz] (kept apart),
// dT += wq_h o H; before a chunk's first item the suffix of the segment's later
// chunks is emitted, and after the segment its total goes to segt (several
// segments: k3_seg_carry turns the totals into each segment's carry, the sum
// of the later segments' totals, which the readers of dT add). With dwq_part the item also writes
// <P_c[f], H[f]> (values of both waves and the ones column, in a fixed order).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k3_state_bwd(const T* __restrict__ q, const float* __restrict__ G,
                                                    const float* __restrict__ Gz, const float* __restrict__ wq,
                                                    const float* __restrict__ P, const float* __restrict__ Pz, int Hq,
                                                    int Hkv, int N, int NB, int SL, float* __restrict__ dT,
                                                    float* __restrict__ dTz, float* __restrict__ segt,
                                                    float* __restrict__ segtz, float* __restrict__ dwq_part) {
  __shared__ float qx[kC][kRow];
  __shared__ float gs[kC][kD + 1];  // [G, Gz]
  __shared__ float xch[2][32];
  const int u = blockIdx.y, R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int seg = blockIdx.z, S = gridDim.z;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int m = wv & 1, ft = wv >> 1, f = blockIdx.x * 64 + 32 * ft + row;
  const int r = kTab3.r[f], c = kTab3.c[f];
  const int c_lo = seg * SL, c_hi = min(NB, c_lo + SL);
  const int NI = (c_hi - c_lo) * R;
  float qr[16], gr[16], gzr = 0.f;
  auto load_item = [&](int it) {
    const int ch = c_hi - 1 - it / R, h = kh * R + it % R;
    const size_t hb = (size_t)(b * Hq + h) * N;
    load_chunk_rows(q, hb * kD, ch * kC, N, qr);
    load_chunk_rows(G, hb * kD, ch * kC, N, gr);
    const int tok = ch * kC + (tid >> 2);
    gzr = (tid & 3) == 0 && tok < N ? Gz[hb + tok] : 0.f;
  };
  load_item(0);
  f32x16 acc = f32x16{};
  float accz = 0.f;
  float pr[16];
  float pz = 0.f;
  for (int it = 0; it < NI; ++it) {
    const int ch = c_hi - 1 - it / R, hh = it % R, h = kh * R + hh;
    const size_t cb = (size_t)u * NB + ch;
    if (hh == 0) {
      store_state_row(dT + (cb * kFP + f) * kD, m, s, acc);
      const float zt = accz + partner(accz);
      if (m == 0 && s == 0) dTz[cb * kFP + f] = zt;
      if (dwq_part) {
        const float* prow = P + (cb * kFP + f) * kD + 32 * m + 4 * s;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float4 x = *reinterpret_cast<const float4*>(prow + 8 * a);
          pr[4 * a] = x.x;
          pr[4 * a + 1] = x.y;
          pr[4 * a + 2] = x.z;
          pr[4 * a + 3] = x.w;
        }
        pz = Pz[cb * kFP + f];
      }
    }
    const float w = wq[(size_t)h * kFP + f];
    lds_sync();
    store_chunk_rows(qx, qr);
    store_chunk_rows(gs, gr);
    if ((tid & 3) == 0) {
      qx[tid >> 2][kD] = ch * kC + (tid >> 2) < N ? 1.f : 0.f;
      qx[tid >> 2][kD + 1] = 0.f;
      gs[tid >> 2][kD] = gzr;
    }
    lds_sync();
    if (it + 1 < NI) load_item(it + 1);
    f32x16 hT = f32x16{};
    float hz = 0.f;
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      const int t = 32 * s + kk;
      const float phi = qx[t][r] * qx[t][c];
      hT = mfma_f32(gs[t][32 * m + row], phi, hT);
      hz += phi * gs[t][kD];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = fmaf(w, hT[i], acc[i]);
    accz = fmaf(w, hz, accz);
    if (dwq_part) {
      float dp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 16; ++i) dp[i & 3] = fmaf(pr[i], hT[i], dp[i & 3]);
      float p = (dp[0] + dp[1]) + (dp[2] + dp[3]);
      p += partner(p);
      const float hzt = hz + partner(hz);
      if (m == 1 && s == 0) xch[ft][row] = p;
      lds_sync();
      if (m == 0 && s == 0) dwq_part[((size_t)(b * Hq + h) * NB + ch) * kFP + f] = p + xch[ft][row] + pz * hzt;
    }
  }
  if (S > 1) {
    const size_t sb = (size_t)u * S + seg;
    store_state_row(segt + (sb * kFP + f) * kD, m, s, acc);
    const float zt = accz + partner(accz);
    if (m == 0 && s == 0) segtz[sb * kFP + f] = zt;
  }
}

// Segment totals -> carries, in place: entry (u, seg) becomes the sum of the
// totals of the segments after seg (a running sum from the last segment, so a
// fixed order). One thread per (unit, feature, value or ones column).
__global__ __launch_bounds__(256) void k3_seg_carry(float* __restrict__ segt, float* __restrict__ segtz, int U, int S) {
  const size_t per_u = (size_t)kFP * (kD + 1);
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= per_u * U) return;
  const int u = (int)(idx / per_u);
  const size_t e = idx % per_u;
  float* base;
  size_t stride;
  if (e < (size_t)kFP * kD) {
    base = segt + (size_t)u * S * kFP * kD + e;
    stride = (size_t)kFP * kD;
  } else {
    base = segtz + (size_t)u * S * kFP + (e - (size_t)kFP * kD);
    stride = kFP;
  }
  float run = 0.f;
  for (int sg = S - 1; sg >= 0; --sg) {
    const float t = base[sg * stride];
    base[sg * stride] = run;
    run += t;
  }
}

// ---------------------------------------------------------------------------
// Slot-ordered state tiles. M-tile M holds the 32 slots 32 M .. 32 M + 31
// (bases 16 M .. 16 M + 15): row j = the natural-order state row of slot
// 32 M + j (64 values, then the ones column; zero for an invalid slot),
// gathered into LDS rows of kStRow floats.
// ---------------------------------------------------------------------------
constexpr int kStRow = kD + 4;
constexpr int kMT = kS / 32;  // 69

// NT threads stage one tile: thread t moves 2048 / NT values (float4s) and,
// for t < 32, the ones column of row t. With wqh (a query head's feature
// coefficients) each row is scaled by its slot's coefficient: the products
// that read the tile are linear in it, so the weighted tile gives the
// weighted readout or fold directly. With ADD each row also adds its row of
// the backward state's segment carry (row block sb). load_tile only
// issues the loads; store_tile, a tile later, forms (row + carry) * weight and
// writes LDS, so the loads stay in flight over a whole tile of products.
template <int NT>
struct TileRegs {
  float4 v[512 / NT];
  float4 c[512 / NT];  // carry rows (ADD)
  float w[512 / NT];   // slot weights (W)
  float z, zc, zw;
};
struct SegCarry {
  const float* C;   // [unit * segments + segment][kFP][kD] (read only with ADD)
  const float* Cz;  // [unit * segments + segment][kFP]
  size_t sb;
};
// natl: the slot table's natural indices staged in LDS (a lane-indexed read of
// the constant table is a global load, and each one's wait would also wait for
// every state load issued before it). Every load is issued unconditionally: an
// invalid slot reads feature row kFeat, a padding row, which every state, carry
// and coefficient buffer holds as zero, so the loads stay whole 16-byte loads
// with no branches between them.
template <int NT, bool ADD, bool W>
__device__ __forceinline__ void load_tile(const float* __restrict__ S, const float* __restrict__ Sz, size_t cb, int M,
                                          const float* __restrict__ wqh, const int16_t* natl, TileRegs<NT>& tr,
                                          const SegCarry& sc) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 512 / NT; ++i) {
    const int idx = t + NT * i, j = idx >> 4, c4 = idx & 15;
    const int nat = natl[32 * M + j], natc = nat >= 0 ? nat : kFeat;
    tr.v[i] = *reinterpret_cast<const float4*>(S + (cb * kFP + natc) * kD + 4 * c4);
    if constexpr (ADD) tr.c[i] = *reinterpret_cast<const float4*>(sc.C + (sc.sb * kFP + natc) * kD + 4 * c4);
    if constexpr (W) tr.w[i] = wqh[natc];
  }
  // every thread loads the ones column of row t % 32 (threads t < 32 store it)
  const int nat = natl[32 * M + (t & 31)], natc = nat >= 0 ? nat : kFeat;
  tr.z = Sz[cb * kFP + natc];
  if constexpr (ADD) tr.zc = sc.Cz[sc.sb * kFP + natc];
  if constexpr (W) tr.zw = wqh[natc];
}
template <int NT, bool ADD, bool W>
__device__ __forceinline__ void store_tile(float* __restrict__ st, const TileRegs<NT>& tr) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 512 / NT; ++i) {
    const int idx = t + NT * i, j = idx >> 4, c4 = idx & 15;
    float4 a = tr.v[i];
    if constexpr (ADD) a = make_float4(a.x + tr.c[i].x, a.y + tr.c[i].y, a.z + tr.c[i].z, a.w + tr.c[i].w);
    if constexpr (W) a = make_float4(a.x * tr.w[i], a.y * tr.w[i], a.z * tr.w[i], a.w * tr.w[i]);
    *reinterpret_cast<float4*>(st + j * kStRow + 4 * c4) = a;
  }
  float z = tr.z;
  if constexpr (ADD) z += tr.zc;
  if constexpr (W) z *= tr.zw;
  if (t < 32) st[t * kStRow + kD] = z;
}

// The carry chunk ch of unit u adds: that of its segment (segments of SL
// chunks, nseg of them; the last segment's carry is zero).
__device__ __forceinline__ SegCarry seg_carry(const float* cS, const float* cSz, int u, int ch, int SL, int nseg) {
  SegCarry sc;
  sc.C = cS;
  sc.Cz = cSz;
  sc.sb = (size_t)u * nseg + ch / SL;
  return sc;
}


// ---------------------------------------------------------------------------
// Readout: block of 4 waves per (query head, chunk, unit) (MODE 0) or (chunk,
// unit) (MODE 1); wave w owns values 32 (w % 2) .. + 31 (accumulator rows)
// and tokens 32 (w / 2) + lane % 32 (lane column):
//   D^T[e][t] = sum_slots S[slot][e] phi_slot(x_t),
// one base per step: lane group s evaluates slot (base, s) on its rotated row
// (static registers); the tile rows carry the slot weights (MODE 0). MODE 0
// adds D to the local numerator in num, the ones column to den, and writes
// out = num / den'; MODE 1 writes dv = D + dvl.
// ---------------------------------------------------------------------------
template <int B, int MODE>
__device__ __forceinline__ void readout_base(const float (&x)[kD], const float* st, int m, int s, int row,
                                             f32x16& acc, float& zacc) {
  constexpr int lb = B % 16;
  const int sr = 16 * (lb / 8) + 8 * s + lb % 8;  // row of slot (B, s) in the tile
  const float phi = base_value<B>(x);
  acc = mfma_f32(st[sr * kStRow + 32 * m + row], phi, acc);
  if constexpr (MODE == 0) {
    zacc = fmaf(st[sr * kStRow + kD], phi, zacc);
    // keep the chain in step with the products (deferring it holds every
    // product live and spills)
    asm volatile("" : "+v"(zacc));
  }
}

// PD (1 or 2) tiles of loads in flight: set (M + 1) % PD holds tile M + 1 and
// then takes tile M + 1 + PD. Two help the dv readout (one block per chunk and
// unit, few waves per CU); the query readout, with seven times the blocks,
// keeps one and its fourth wave per SIMD.
template <int M, int MODE, bool ADD, int PD>
__device__ __forceinline__ void readout_tiles(const float (&x)[kD], float* st0, float* st1,
                                              const float* __restrict__ S, const float* __restrict__ Sz, size_t cb,
                                              const float* wqh, int m, int s, int row, TileRegs<256> (&tr)[PD],
                                              f32x16& acc, float& zacc, const int16_t* natl, const SegCarry& sc) {
  const float* st = (M & 1) ? st1 : st0;
  [&]<int... J>(std::integer_sequence<int, J...>) {
    (readout_base<16 * M + J, MODE>(x, st, m, s, row, acc, zacc), ...);
  }(std::make_integer_sequence<int, 16>{});
  if constexpr (M + 1 < kMT) {
    store_tile<256, ADD, MODE == 0>((M & 1) ? st0 : st1, tr[(M + 1) % PD]);
    if constexpr (M + 1 + PD < kMT)
      load_tile<256, ADD, MODE == 0>(S, Sz, cb, M + 1 + PD, wqh, natl, tr[(M + 1) % PD], sc);
    lds_sync();
    __builtin_amdgcn_sched_barrier(0);
    readout_tiles<M + 1, MODE, ADD, PD>(x, st0, st1, S, Sz, cb, wqh, m, s, row, tr, acc, zacc, natl, sc);
  }
}

template <typename T, int MODE, bool CARRY = false>
__global__ __launch_bounds__(256, 2) void k3_readout(const T* __restrict__ x_in, const float* __restrict__ wq,
                                                     const float* __restrict__ S, const float* __restrict__ Sz, int Hq,
                                                     int Hkv, int N, int NB, float floor, float* __restrict__ num,
                                                     float* __restrict__ den, T* __restrict__ out,
                                                     const float* __restrict__ dvl, T* __restrict__ dv,
                                                     const float* __restrict__ cS, const float* __restrict__ cSz,
                                                     int SL, int nseg) {
  __shared__ __attribute__((aligned(16))) float st0[32 * kStRow], st1[32 * kStRow];
  __shared__ float zd[kC];
  __shared__ int16_t natl[kS];
  int hh = 0, ch, u;
  if constexpr (MODE == 0) {
    head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  } else {
    const int total = gridDim.x, id = blockIdx.x;
    const int w = (total & 7) == 0 ? (id & 7) * (total >> 3) + (id >> 3) : id;
    ch = w % NB;
    u = w / NB;
  }
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int m = wv & 1, n = wv >> 1;
  const int tok0 = ch * kC;
  const size_t xbase = MODE == 0 ? (size_t)(b * Hq + h) * N * kD : (size_t)u * N * kD;
  const size_t cb = (size_t)u * NB + ch;
  const float* wqh = MODE == 0 ? wq + (size_t)h * kFP : nullptr;
  const int tok = tok0 + 32 * n + row;
  const bool ok = tok < N;
  float x[kD];
  load_rotated_f32(x_in, xbase + (size_t)(ok ? tok : N - 1) * kD, ok, s, x);
  const SegCarry sc = seg_carry(cS, cSz, u, ch, SL, nseg);
  for (int i = tid; i < kS; i += 256) natl[i] = kSlot3.nat[i];
  __syncthreads();
  constexpr int PD = MODE == 1 ? 2 : 1;
  TileRegs<256> tr[PD];
  load_tile<256, CARRY, MODE == 0>(S, Sz, cb, 0, wqh, natl, tr[0], sc);
  store_tile<256, CARRY, MODE == 0>(st0, tr[0]);
#pragma unroll
  for (int i = 1; i <= PD; ++i) load_tile<256, CARRY, MODE == 0>(S, Sz, cb, i, wqh, natl, tr[i % PD], sc);
  __syncthreads();
  f32x16 acc = f32x16{};
  float zacc = 0.f;
  readout_tiles<0, MODE, CARRY, PD>(x, st0, st1, S, Sz, cb, wqh, m, s, row, tr, acc, zacc, natl, sc);

  if constexpr (MODE == 0) {
    const size_t dbase = (size_t)(b * Hq + h) * N;
    if (m == 0) {
      const float z = zacc + partner(zacc);
      if (s == 0) zd[32 * n + row] = (ok ? den[dbase + tok] : 0.f) + z;
    }
    lds_sync();
    if (ok) {
      const float dd = zd[32 * n + row];
      if (m == 0 && s == 0) den[dbase + tok] = dd;
      const float inv = 1.f / (floor > 0.f ? fmaxf(dd, floor) : dd);
      float* nrow = num + xbase + (size_t)tok * kD + 32 * m + 4 * s;
      T* orow = out + xbase + (size_t)tok * kD + 32 * m + 4 * s;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float4 loc = *reinterpret_cast<const float4*>(nrow + 8 * a);
        const float y[4] = {acc[4 * a] + loc.x, acc[4 * a + 1] + loc.y, acc[4 * a + 2] + loc.z,
                            acc[4 * a + 3] + loc.w};
        *reinterpret_cast<float4*>(nrow + 8 * a) = make_float4(y[0], y[1], y[2], y[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) orow[8 * a + e] = from_f<T>(y[e] * inv);
      }
    }
  } else {
    if (ok) {
      // local part: the unit's query heads in order
      for (int r2 = 0; r2 < R; ++r2) {
        const float* lrow = dvl + ((size_t)(b * Hq + kh * R + r2) * N + tok) * kD + 32 * m + 4 * s;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float4 loc = *reinterpret_cast<const float4*>(lrow + 8 * a);
          acc[4 * a] += loc.x;
          acc[4 * a + 1] += loc.y;
          acc[4 * a + 2] += loc.z;
          acc[4 * a + 3] += loc.w;
        }
      }
      T* drow = dv + xbase + (size_t)tok * kD + 32 * m + 4 * s;
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int e = 0; e < 4; ++e) drow[8 * a + e] = from_f<T>(acc[4 * a + e]);
    }
  }
}

// ---------------------------------------------------------------------------
// Fold: block of 2 waves per (query head, chunk, unit) (MODE 0, dq) or
// (chunk, unit) (MODE 1, dk); wave w owns tokens 32 w + lane % 32. Per
// M-tile: D^T[slot][t] = sum_e S[slot][e] y_t[e] + Sz[slot] y_t[64] (A rows
// in the fold row order, K index = value 32 s + k at step k, the ones column
// as a 33rd step in lane group 0), y = [G, Gz] (MODE 0) or [v, 1] (MODE 1),
// then folded through the rotated row (static registers); the tile rows carry
// the slot weights (MODE 0). The result plus the local part is written as
// dq / dk.
// ---------------------------------------------------------------------------
template <int M>
__device__ __forceinline__ void fold_tile_f32(const float (&x)[kD], float (&dx)[kD], const float (&yv)[32], float yz,
                                              const float* st, int s, int row) {
  const float* ar = st + fold::fold_row(row) * kStRow + 32 * s;
  f32x16 D = f32x16{};
#pragma unroll
  for (int k4 = 0; k4 < 8; ++k4) {
    const float4 a = *reinterpret_cast<const float4*>(ar + 4 * k4);
    D = mfma_f32(a.x, yv[4 * k4], D);
    D = mfma_f32(a.y, yv[4 * k4 + 1], D);
    D = mfma_f32(a.z, yv[4 * k4 + 2], D);
    D = mfma_f32(a.w, yv[4 * k4 + 3], D);
  }
  const float az = s == 0 ? st[fold::fold_row(row) * kStRow + kD] : 0.f;
  D = mfma_f32(az, s == 0 ? yz : 0.f, D);
  float w16[16];
  fold::fold_weights<M, false>(nullptr, s, w16);
  fold::fold_tile<M>(D, x, dx, w16);
}

template <int M, bool ADD, bool W>
__device__ __forceinline__ void fold_tiles(const float (&x)[kD], float (&dx)[kD], const float (&yv)[32], float yz,
                                           float* st0, float* st1, const float* __restrict__ S,
                                           const float* __restrict__ Sz, size_t cb, const float* wqh, int s, int row,
                                           TileRegs<128>& tr, const int16_t* natl, const SegCarry& sc) {
  pin64(dx);
  fold_tile_f32<M>(x, dx, yv, yz, (M & 1) ? st1 : st0, s, row);
  if constexpr (M + 1 < kMT) {
    store_tile<128, ADD, W>((M & 1) ? st0 : st1, tr);
    if constexpr (M + 2 < kMT) load_tile<128, ADD, W>(S, Sz, cb, M + 2, wqh, natl, tr, sc);
    lds_sync();
    __builtin_amdgcn_sched_barrier(0);
    fold_tiles<M + 1, ADD, W>(x, dx, yv, yz, st0, st1, S, Sz, cb, wqh, s, row, tr, natl, sc);
  }
}

template <typename T, int MODE, bool CARRY = false>
__global__ __launch_bounds__(128, 2) void k3_fold(const T* __restrict__ x_in, const float* __restrict__ y_in,
                                                  const T* __restrict__ v_in, const float* __restrict__ yz_in,
                                                  const float* __restrict__ wq, const float* __restrict__ S,
                                                  const float* __restrict__ Sz, const float* __restrict__ local,
                                                  int Hq, int Hkv, int N, int NB, T* __restrict__ dx_out,
                                                  const float* __restrict__ cS, const float* __restrict__ cSz, int SL,
                                                  int nseg) {
  __shared__ __attribute__((aligned(16))) float st0[32 * kStRow], st1[32 * kStRow];
  __shared__ int16_t natl[kS];
  int hh = 0, ch, u;
  if constexpr (MODE == 0) {
    head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  } else {
    const int total = gridDim.x, id = blockIdx.x;
    const int w = (total & 7) == 0 ? (id & 7) * (total >> 3) + (id >> 3) : id;
    ch = w % NB;
    u = w / NB;
  }
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t xbase = MODE == 0 ? (size_t)(b * Hq + h) * N * kD : (size_t)u * N * kD;
  const size_t cb = (size_t)u * NB + ch;
  const float* wqh = MODE == 0 ? wq + (size_t)h * kFP : nullptr;
  const int tok = tok0 + 32 * wv + row;
  const bool ok = tok < N;
  const size_t rowoff = xbase + (size_t)(ok ? tok : N - 1) * kD;
  float x[kD], dx[kD];
  load_rotated_f32(x_in, rowoff, ok, s, x);
  // the lane group's half of y (values 32 s .. 32 s + 31) and the ones column
  float yv[32];
  float yz;
  if constexpr (MODE == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 a = reinterpret_cast<const float4*>(y_in + rowoff + 32 * s)[i];
      yv[4 * i] = ok ? a.x : 0.f;
      yv[4 * i + 1] = ok ? a.y : 0.f;
      yv[4 * i + 2] = ok ? a.z : 0.f;
      yv[4 * i + 3] = ok ? a.w : 0.f;
    }
    yz = ok ? yz_in[(size_t)(b * Hq + h) * N + tok] : 0.f;
  } else {
    float t16[16];
    load16(v_in, rowoff + 32 * s, ok, t16);
#pragma unroll
    for (int i = 0; i < 16; ++i) yv[i] = t16[i];
    load16(v_in, rowoff + 32 * s + 16, ok, t16);
#pragma unroll
    for (int i = 0; i < 16; ++i) yv[16 + i] = t16[i];
    yz = ok ? 1.f : 0.f;
  }
#pragma unroll
  for (int i = 0; i < kD; ++i) dx[i] = 0.f;
  const SegCarry sc = seg_carry(cS, cSz, u, ch, SL, nseg);
  for (int i = tid; i < kS; i += 128) natl[i] = kSlot3.nat[i];
  __syncthreads();
  TileRegs<128> tr;
  load_tile<128, CARRY, MODE == 0>(S, Sz, cb, 0, wqh, natl, tr, sc);
  store_tile<128, CARRY, MODE == 0>(st0, tr);
  load_tile<128, CARRY, MODE == 0>(S, Sz, cb, 1, wqh, natl, tr, sc);
  __syncthreads();
  fold_tiles<0, CARRY, MODE == 0>(x, dx, yv, yz, st0, st1, S, Sz, cb, wqh, s, row, tr, natl, sc);
  float full[32];
  fold::combine_rotation_groups(dx, s, full);
  if (ok) {
    // local part: dq's own head (MODE 0), or the unit's heads in order (MODE 1)
    for (int r2 = 0; r2 < (MODE == 0 ? 1 : R); ++r2) {
      const size_t lo = MODE == 0 ? rowoff + 32 * s : ((size_t)(b * Hq + kh * R + r2) * N + tok) * kD + 32 * s;
      const float4* lf = reinterpret_cast<const float4*>(local + lo);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float4 a = lf[j];
        full[4 * j] += a.x;
        full[4 * j + 1] += a.y;
        full[4 * j + 2] += a.z;
        full[4 * j + 3] += a.w;
      }
    }
    fold::store32(dx_out + rowoff + 32 * s, full);
  }
}

// ---------------------------------------------------------------------------
// Intra-chunk (local) VJP on the matrix cores, one block of three waves per
// (query head, chunk, unit); wave w owns the lower 32 x 32 tile (it, jt) =
// (0,0), (1,0), (1,1) of the (query i, key j) plane. With s_g(i,j) =
// scale sum_{d in g} q_i[d] k_j[d], ds_ij = g_i . v_j + gz_i (j <= i) and
// t_g = sum_h Gam_gh s_h (the fp32 kernels' symmetric-Gam convention):
//   kappa_ij = c0 + sum_g s_g (lam_g + t_g),  X_g = ds scale (lam_g + 2 t_g)
//   dq_i[d] = sum_j X_g(d)[i][j] k_j[d],  dk_j[d] = sum_i X_g(d)[i][j] q_i[d],
//   dv_j[e] = sum_i kappa_ij g_i[e]   (dk, dv per query head: dkl, dvl)
// and the coefficient partials [0] sum ds, [1 + g] sum ds s_g,
// [9 + 8 g + h] sum ds s_g s_h (full symmetric 8 x 8).
// The group sums run over the group-sorted dimensions (k-step k holds sorted
// positions 2k and 2k + 1 in lane groups 0 and 1; a step that straddles two
// groups runs once for each, masked), the tile in both orientations: C[i][j]
// (lane column j) for dk, dv and the partials, C[j][i] (lane column i) for
// dq; the X_g and kappa accumulators then serve as the K-major operand of the
// output products (K index = accumulator row, step k taking register k).
// ---------------------------------------------------------------------------
constexpr int kLRow = kD + 4;

struct LocalCtx {
  const float (*qx)[kLRow];
  const float (*kx)[kLRow];
  const float (*vx)[kLRow];
  const float (*gs)[kLRow];
  const float* gz;
  const int* perm;
  const int* gstart;
  int G;
};

// acc[g] = sum over the group-sorted dims d of g: A[a_row][d] B[b_row][d]
// (A = the lane row's operand, B = the lane column's), scaled by scale.
__device__ __forceinline__ void group_sums_mfma(const float (*A)[kLRow], const float (*B)[kLRow], int a_row,
                                                int b_row, const int* perm, const int* gstart, int G, int s,
                                                float scale, f32x16 (&acc)[8]) {
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    acc[g] = f32x16{};
    if (g < G) {
      const int p0 = gstart[g], p1 = gstart[g + 1];
      for (int kk = p0 >> 1; kk < (p1 + 1) >> 1; ++kk) {
        const int p = 2 * kk + s, d = perm[p];
        const float a = (p >= p0 && p < p1) ? A[a_row][d] : 0.f;
        acc[g] = mfma_f32(a, B[b_row][d], acc[g]);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[g][i] *= scale;
  }
}

// ds over K = values: C[row][col] = sum_e Gr[row][e] Vc[col][e], value 32 s + k at step k.
__device__ __forceinline__ f32x16 dot_rows_mfma(const float (*Ar)[kLRow], const float (*Bc)[kLRow], int a_row,
                                                int b_row, int s) {
  f32x16 acc = f32x16{};
#pragma unroll
  for (int k4 = 0; k4 < 8; ++k4) {
    const float4 a = *reinterpret_cast<const float4*>(&Ar[a_row][32 * s + 4 * k4]);
    const float4 b = *reinterpret_cast<const float4*>(&Bc[b_row][32 * s + 4 * k4]);
    acc = mfma_f32(a.x, b.x, acc);
    acc = mfma_f32(a.y, b.y, acc);
    acc = mfma_f32(a.z, b.z, acc);
    acc = mfma_f32(a.w, b.w, acc);
  }
  return acc;
}

// ---------------------------------------------------------------------------
// Intra-chunk forward on the matrix cores, one block of 3 waves per (query
// head, chunk, unit); wave w owns the lower tile (j-tile, i-tile) = (0,0),
// (0,1), (1,1) in orientation C[j][i] (lane column = query i):
//   kappa(i, j) = c0 + sum_g s_g (lam_g + sum_h Gam_gh s_h),  j <= i,
// with the group sums s_g on the matrix cores over the group-sorted dims, then
//   num^T[e][i] = sum_j V^T[e][j] kappa^T[j][i] (the kappa accumulators as the
//   K-major operand, step k taking register k),  den[i] = sum_j kappa(i, j).
// Writes the intra-chunk num and den, to which k3_readout adds the state part
// (reference: the local terms of grouped_reference.py:214-318 in group-sum form).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(192) void k3_intra_fwd(const T* __restrict__ q, const T* __restrict__ k,
                                                    const T* __restrict__ v, const int32_t* __restrict__ labels,
                                                    const float* __restrict__ c0, const float* __restrict__ lam,
                                                    const float* __restrict__ gam, int Gn, int Hq, int Hkv, int N,
                                                    int NB, float scale, float* __restrict__ num,
                                                    float* __restrict__ den) {
  __shared__ __attribute__((aligned(16))) float qx[kC][kLRow];
  __shared__ __attribute__((aligned(16))) float kx[kC][kLRow];
  __shared__ __attribute__((aligned(16))) float vx[kC][kLRow];
  __shared__ __attribute__((aligned(16))) float xb[kD][33];  // tile (1,0)'s num^T
  __shared__ float xz[32];                                    // and its den
  __shared__ HeadGroups<8> hg;
  int hh, ch, u;
  head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int it = wv == 0 ? 0 : 1, jt = wv == 2 ? 1 : 0;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;
  // staging: 192 threads, 64 rows x 64 dims per operand, 16 consecutive dims each
  for (int idx = tid; idx < 3 * kC * 4; idx += 192) {
    const int op = idx >> 8, rr = (idx >> 2) & 63, q4 = idx & 3, tok = tok0 + rr;
    const bool ok = tok < N;
    float vals[16];
    const size_t off = (op == 0 ? qbase : kbase) + (size_t)(ok ? tok : N - 1) * kD + 16 * q4;
    if (op == 0) load16(q, off, ok, vals);
    else if (op == 1) load16(k, off, ok, vals);
    else load16(v, off, ok, vals);
    float* dst = op == 0 ? &qx[rr][16 * q4] : op == 1 ? &kx[rr][16 * q4] : &vx[rr][16 * q4];
#pragma unroll
    for (int e = 0; e < 16; e += 4)
      *reinterpret_cast<float4*>(dst + e) = make_float4(vals[e], vals[e + 1], vals[e + 2], vals[e + 3]);
  }
  load_head_groups(hg, labels, c0, lam, gam, Gn, h);  // synchronizes the block
  // the head's coefficients, wave-uniform: kept in scalar registers
  auto uni = [](float x) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x))); };
  float lm[8], gm[8][8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    lm[g] = uni(g < Gn ? hg.lam[g] : 0.f);
#pragma unroll
    for (int e = 0; e < 8; ++e) gm[g][e] = uni((g < Gn && e < Gn) ? hg.gam[g * Gn + e] : 0.f);
  }
  const float cz = uni(hg.c0);

  const int jr = 32 * jt + row, ic = 32 * it + row;
  f32x16 S[8];
  group_sums_mfma(kx, qx, jr, ic, hg.perm, hg.gstart, Gn, s, scale, S);
  f32x16 kap;
  float dsum = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const bool valid = 32 * jt + c32_row(r, l) <= ic;
    float kv = cz;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      float inner = lm[g];
#pragma unroll
      for (int e = 0; e < 8; ++e) inner = fmaf(gm[g][e], S[e][r], inner);
      kv = fmaf(S[g][r], inner, kv);
    }
    kap[r] = valid ? kv : 0.f;
    dsum += kap[r];
  }
  dsum += partner(dsum);
  // num^T[e][i] = sum_j V^T[e][j] kappa^T[j][i]; j = 32 jt + c32_row(k, 32 s) at step k
  f32x16 nm[2] = {f32x16{}, f32x16{}};
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    const int e = 32 * dt + row;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) nm[dt] = mfma_f32(vx[32 * jt + c32_row(kk, 32 * s)][e], kap[kk], nm[dt]);
  }
  // i-tile 1 gets tiles (1,0) and (1,1): wave 1 hands its part to wave 2
  if (wv == 1) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) xb[32 * dt + c32_row(r, l)][row] = nm[dt][r];
    if (s == 0) xz[row] = dsum;
  }
  __syncthreads();
  if (wv != 1) {
    const int i = 32 * it + row, tok = tok0 + i;
    if (wv == 2) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) nm[dt][r] = xb[32 * dt + c32_row(r, l)][row] + nm[dt][r];
      dsum = xz[row] + dsum;
    }
    if (tok < N) {
      float* dst = num + qbase + (size_t)tok * kD;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int a = 0; a < 4; ++a)
          *reinterpret_cast<float4*>(dst + 32 * dt + 8 * a + 4 * s) =
              make_float4(nm[dt][4 * a], nm[dt][4 * a + 1], nm[dt][4 * a + 2], nm[dt][4 * a + 3]);
      if (s == 0) den[(size_t)(b * Hq + h) * N + tok] = dsum;
    }
  }
}

template <typename T, int PART>
__global__ __launch_bounds__(192, PART == 0 ? 2 : 1) void k3_local(const T* __restrict__ q, const T* __restrict__ k,
                                                const T* __restrict__ v, const float* __restrict__ G,
                                                const float* __restrict__ Gz, const int32_t* __restrict__ labels,
                                                const float* __restrict__ c0, const float* __restrict__ lam,
                                                const float* __restrict__ gam, int Gn, int Hq, int Hkv, int N,
                                                int NB, float scale, float* __restrict__ dql,
                                                float* __restrict__ dkl, float* __restrict__ dvl,
                                                float* __restrict__ coefl) {
  __shared__ __attribute__((aligned(16))) float qx[kC][kLRow];
  __shared__ __attribute__((aligned(16))) float kx[kC][kLRow];
  __shared__ __attribute__((aligned(16))) float vx[kC][kLRow];
  __shared__ __attribute__((aligned(16))) float gs[kC][kLRow];
  // tile (1,0)'s partial outputs: dq (PART 0), dk and dv (PART 1)
  __shared__ __attribute__((aligned(16))) float xb[PART == 0 ? 1 : 2][kD][33];
  __shared__ float gz[kC];
  __shared__ float cred[PART == 1 ? 3 : 1][45];
  __shared__ HeadGroups<8> hg;
  int hh, ch, u;
  head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int it = wv == 0 ? 0 : 1, jt = wv == 2 ? 1 : 0;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;
  // staging: 192 threads, 64 rows x 64 dims per operand, 16 consecutive dims each
  for (int idx = tid; idx < 4 * kC * 4; idx += 192) {
    const int op = idx >> 8, rr = (idx >> 2) & 63, q4 = idx & 3, tok = tok0 + rr;
    const bool ok = tok < N;
    float vals[16];
    const size_t off = (op == 0 || op == 3 ? qbase : kbase) + (size_t)(ok ? tok : N - 1) * kD + 16 * q4;
    if (op == 0) load16(q, off, ok, vals);
    else if (op == 1) load16(k, off, ok, vals);
    else if (op == 2) load16(v, off, ok, vals);
    else load16(G, off, ok, vals);
    float* dst = op == 0 ? &qx[rr][16 * q4] : op == 1 ? &kx[rr][16 * q4] : op == 2 ? &vx[rr][16 * q4] : &gs[rr][16 * q4];
#pragma unroll
    for (int e = 0; e < 16; e += 4)
      *reinterpret_cast<float4*>(dst + e) = make_float4(vals[e], vals[e + 1], vals[e + 2], vals[e + 3]);
  }
  if (tid < kC) gz[tid] = tok0 + tid < N ? Gz[(size_t)(b * Hq + h) * N + tok0 + tid] : 0.f;
  load_head_groups(hg, labels, c0, lam, gam, Gn, h);  // synchronizes the block
  // the head's coefficients, wave-uniform (scalar registers)
  auto uni = [](float x) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x))); };
  float lm[8], gm[8][8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    lm[g] = uni(g < Gn ? hg.lam[g] : 0.f);
#pragma unroll
    for (int e = 0; e < 8; ++e) gm[g][e] = uni((g < Gn && e < Gn) ? hg.gam[g * Gn + e] : 0.f);
  }
  const float cz = uni(hg.c0);
  // elementwise step on one entry: s (8 group sums) -> X_g (in place) and kappa
  auto entry = [&](float (&sv)[8], float ds, bool valid, float& kap) {
    float tg[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      float t = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) t = fmaf(gm[g][e], sv[e], t);
      tg[g] = t;
    }
    float kv = cz;
#pragma unroll
    for (int g = 0; g < 8; ++g) kv = fmaf(sv[g], lm[g] + tg[g], kv);
    const float dss = ds * scale;
#pragma unroll
    for (int g = 0; g < 8; ++g) sv[g] = valid ? dss * (lm[g] + 2.f * tg[g]) : 0.f;
    kap = valid ? kv : 0.f;
  };

  f32x16 S[8];
  // ---- PART 0, orientation C[j][i] (lane column = query i): dq ----
  if constexpr (PART == 0) {
    const int jr = 32 * jt + row, ic = 32 * it + row;
    group_sums_mfma(kx, qx, jr, ic, hg.perm, hg.gstart, Gn, s, scale, S);
    f32x16 dsT = dot_rows_mfma(vx, gs, jr, ic, s);  // sum_e v_j[e] g_i[e]
    const float gzi = gz[ic];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int jl = c32_row(r, l);
      const bool valid = 32 * jt + jl <= ic;
      float sv[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) sv[g] = S[g][r];
      float kap;
      entry(sv, dsT[r] + gzi, valid, kap);
#pragma unroll
      for (int g = 0; g < 8; ++g) S[g][r] = sv[g];
    }
    // dq^T[d][i] = sum_g sum_j (K o m_g)^T[d][j] X_g^T[j][i]; j = 32 jt + c32_row(k, 32 s) at step k
    f32x16 dq[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int d = 32 * dt + row, gd = hg.lab[d];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        if (g < Gn) {
#pragma unroll
          for (int kk = 0; kk < 16; ++kk) {
            const int j = 32 * jt + c32_row(kk, 32 * s);
            dq[dt] = mfma_f32(gd == g ? kx[j][d] : 0.f, S[g][kk], dq[dt]);
          }
        }
      }
    }
    // i-tile 1 gets tiles (1,0) and (1,1): wave 1 hands its part to wave 2
    if (wv == 1) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) xb[0][32 * dt + c32_row(r, l)][row] = dq[dt][r];
    }
    __syncthreads();
    if (wv != 1) {
      const int i = 32 * it + row, tok = tok0 + i;
      if (wv == 2) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) dq[dt][r] = xb[0][32 * dt + c32_row(r, l)][row] + dq[dt][r];
      }
      if (tok < N) {
        float* dst = dql + qbase + (size_t)tok * kD;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int a = 0; a < 4; ++a)
            *reinterpret_cast<float4*>(dst + 32 * dt + 8 * a + 4 * s) =
                make_float4(dq[dt][4 * a], dq[dt][4 * a + 1], dq[dt][4 * a + 2], dq[dt][4 * a + 3]);
      }
    }
    __syncthreads();
  }
  // ---- PART 1, orientation C[i][j] (lane column = key j): dk, dv, coefficient partials ----
  if constexpr (PART == 1) {
    const int ir = 32 * it + row, jc = 32 * jt + row;
    group_sums_mfma(qx, kx, ir, jc, hg.perm, hg.gstart, Gn, s, scale, S);
    f32x16 ds = dot_rows_mfma(gs, vx, ir, jc, s);  // sum_e g_i[e] v_j[e]
    f32x16 kap16;
    float cacc[45];
#pragma unroll
    for (int e = 0; e < 45; ++e) cacc[e] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * it + c32_row(r, l);
      const bool valid = jc <= i;
      const float dsv = valid ? ds[r] + gz[i] : 0.f;
      float sv[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) sv[g] = S[g][r];
      if (coefl) {
        cacc[0] += dsv;
        int e = 9;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const float pg = dsv * sv[g];
          cacc[1 + g] += pg;
#pragma unroll
          for (int h2 = g; h2 < 8; ++h2) cacc[e++] += pg * sv[h2];
        }
      }
      float kap;
      entry(sv, dsv, valid, kap);
      kap16[r] = kap;
#pragma unroll
      for (int g = 0; g < 8; ++g) S[g][r] = sv[g];
    }
    // dk^T[d][j] = sum_g sum_i (Q o m_g)^T[d][i] X_g[i][j]; dv^T[e][j] = sum_i G^T[e][i] kappa[i][j]
    f32x16 dk[2] = {f32x16{}, f32x16{}}, dv[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int d = 32 * dt + row, gd = hg.lab[d];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        if (g < Gn) {
#pragma unroll
          for (int kk = 0; kk < 16; ++kk) {
            const int i = 32 * it + c32_row(kk, 32 * s);
            dk[dt] = mfma_f32(gd == g ? qx[i][d] : 0.f, S[g][kk], dk[dt]);
          }
        }
      }
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
        const int i = 32 * it + c32_row(kk, 32 * s);
        dv[dt] = mfma_f32(gs[i][d], kap16[kk], dv[dt]);
      }
    }
    // coefficient partials: lane sums (fixed butterfly), then the waves in order
    if (coefl) {
#pragma unroll
      for (int e = 0; e < 45; ++e) {
        float x = cacc[e];
        x += __shfl_xor(x, 1, 64);
        x += __shfl_xor(x, 2, 64);
        x += __shfl_xor(x, 4, 64);
        x += __shfl_xor(x, 8, 64);
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        if (l == 0) cred[wv][e] = x;
      }
    }
    // j-tile 0 gets tiles (0,0) and (1,0): wave 1 hands its part to wave 0
    if (wv == 1) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          xb[0][32 * dt + c32_row(r, l)][row] = dk[dt][r];
          xb[1][32 * dt + c32_row(r, l)][row] = dv[dt][r];
        }
    }
    __syncthreads();
    if (wv != 1) {
      const int j = 32 * jt + row, tok = tok0 + j;
      if (wv == 0) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            dk[dt][r] += xb[0][32 * dt + c32_row(r, l)][row];
            dv[dt][r] += xb[1][32 * dt + c32_row(r, l)][row];
          }
      }
      if (tok < N) {
        float* dkd = dkl + qbase + (size_t)tok * kD;
        float* dvd = dvl + qbase + (size_t)tok * kD;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            *reinterpret_cast<float4*>(dkd + 32 * dt + 8 * a + 4 * s) =
                make_float4(dk[dt][4 * a], dk[dt][4 * a + 1], dk[dt][4 * a + 2], dk[dt][4 * a + 3]);
            *reinterpret_cast<float4*>(dvd + 32 * dt + 8 * a + 4 * s) =
                make_float4(dv[dt][4 * a], dv[dt][4 * a + 1], dv[dt][4 * a + 2], dv[dt][4 * a + 3]);
          }
      }
    }
    if (coefl && tid < 45) {
      const float x = (cred[0][tid] + cred[1][tid]) + cred[2][tid];
      float* out = coefl + ((size_t)(b * Hq + h) * NB + ch) * 73;
      if (tid == 0) {
        out[0] = x;
      } else if (tid <= 8) {
        out[tid] = x;
      } else {
        int rem = tid - 9, g = 0;
        while (rem >= 8 - g) {
          rem -= 8 - g;
          ++g;
        }
        out[9 + 8 * g + g + rem] = x;
        out[9 + 8 * (g + rem) + g] = x;
      }
    }
  }
}

// Per-head sums of the local coefficient partials over (batch, chunk), in a
// fixed order: coefs[h][e].
__global__ __launch_bounds__(256) void k3_coef_reduce(const float* __restrict__ coefl, int B, int Hq, int NB,
                                                      float* __restrict__ coefs) {
  __shared__ float ps[256];
  const int e = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
  float acc = 0.f;
  for (int r = t; r < B * NB; r += 256) {
    const int b = r / NB, ch = r - b * NB;
    acc += coefl[((size_t)(b * Hq + h) * NB + ch) * 73 + e];
  }
  ps[t] = acc;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (t < w) ps[t] += ps[t + w];
    __syncthreads();
  }
  if (t == 0) coefs[(size_t)h * 73 + e] = ps[0];
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <typename T>
void launch_f32_state_fwd(const LaunchGeom& g, const T* k, const T* v, float* carry, float* carry_z, hipStream_t st,
                          const Timer& timed) {
  timed("k3_state_fwd", st, [&] {
    hipLaunchKernelGGL(k3_state_fwd<T>, dim3(kFP / 64, g.U), dim3(256), 0, st, k, v, g.N, g.NB, carry, carry_z);
  });
}

template <typename T>
void launch_f32_intra_fwd(const LaunchGeom& g, const T* q, const T* k, const T* v, const int32_t* labels, const float* c0,
                          const float* lam, const float* gam, int groups, float scale, float* num, float* den,
                          hipStream_t st, const Timer& timed) {
  timed("k3_intra_fwd", st, [&] {
    hipLaunchKernelGGL(k3_intra_fwd<T>, dim3(g.R * g.NB * g.U), dim3(192), 0, st, q, k, v, labels, c0, lam, gam,
                       groups, g.Hq, g.Hkv, g.N, g.NB, scale, num, den);
  });
}

template <typename T>
void launch_f32_readout_fwd(const LaunchGeom& g, const T* q, const float* wq, const float* carry, const float* carry_z,
                            float floor, float* num, float* den, T* out, hipStream_t st, const Timer& timed) {
  timed("k3_readout", st, [&] {
    hipLaunchKernelGGL((k3_readout<T, 0>), dim3(g.R * g.NB * g.U), dim3(256), 0, st, q, wq, carry, carry_z, g.Hq,
                       g.Hkv, g.N, g.NB, floor, num, den, out, nullptr, nullptr, nullptr, nullptr, 1, 1);
  });
}

// One stream (the allocation-free entry point, the profiling mode, a call
// made during a graph capture before the second stream exists): the state
// scan first. This order measured 3.94-3.95 ms per config-2 step on one
// stream, against 4.12 ms with the two-stream order (the intra-chunk kernels
// first) run on one stream.
template <typename T>
void launch_f32_backward_serial(const LaunchGeom& g, const F32BwdArgs<T>& a, hipStream_t st, const Timer& timed) {
  if (a.dk || a.dv || a.dwq_part) {
    timed("k3_state_bwd", st, [&] {
      hipLaunchKernelGGL(k3_state_bwd<T>, dim3(kFP / 64, g.U, a.plan.S), dim3(256), 0, st, a.q, a.G, a.Gz, a.wq, a.P, a.Pz,
                         g.Hq, g.Hkv, g.N, g.NB, a.plan.SL, a.dT, a.dTz, a.segt, a.segtz, a.dwq_part);
    });
    if (a.plan.S > 1 && (a.dk || a.dv)) {
      timed("k3_seg_carry", st, [&] {
        const size_t n = (size_t)g.U * kFP * (kD + 1);
        hipLaunchKernelGGL(k3_seg_carry, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a.segt, a.segtz, g.U,
                           a.plan.S);
      });
    }
  }
  const float* cS = a.plan.S > 1 ? a.segt : nullptr;
  const float* cSz = a.plan.S > 1 ? a.segtz : nullptr;
  timed("k3_local_dq", st, [&] {
    hipLaunchKernelGGL((k3_local<T, 0>), dim3(g.R * g.NB * g.U), dim3(192), 0, st, a.q, a.k, a.v, a.G, a.Gz,
                       a.labels, a.c0, a.lam, a.gam, a.groups, g.Hq, g.Hkv, g.N, g.NB, a.scale, a.dql, a.dkl, a.dvl,
                       a.coefl);
  });
  timed("k3_local_kv", st, [&] {
    hipLaunchKernelGGL((k3_local<T, 1>), dim3(g.R * g.NB * g.U), dim3(192), 0, st, a.q, a.k, a.v, a.G, a.Gz,
                       a.labels, a.c0, a.lam, a.gam, a.groups, g.Hq, g.Hkv, g.N, g.NB, a.scale, a.dql, a.dkl, a.dvl,
                       a.coefl);
  });
  if (a.dq) {
    timed("k3_fold_q", st, [&] {
      hipLaunchKernelGGL((k3_fold<T, 0>), dim3(g.R * g.NB * g.U), dim3(128), 0, st, a.q, a.G, nullptr, a.Gz, a.wq,
                         a.P, a.Pz, a.dql, g.Hq, g.Hkv, g.N, g.NB, a.dq, nullptr, nullptr, 1, 1);
    });
  }
  if (a.dk) {
    timed("k3_fold_k", st, [&] {
      auto* kern = cS ? k3_fold<T, 1, true> : k3_fold<T, 1, false>;
      hipLaunchKernelGGL(kern, dim3(g.NB * g.U), dim3(128), 0, st, a.k, nullptr, a.v, nullptr, nullptr,
                         a.dT, a.dTz, a.dkl, g.Hq, g.Hkv, g.N, g.NB, a.dk, cS, cSz, a.plan.SL, a.plan.S);
    });
  }
  if (a.dv) {
    timed("k3_readout_v", st, [&] {
      auto* kern = cS ? k3_readout<T, 1, true> : k3_readout<T, 1, false>;
      hipLaunchKernelGGL(kern, dim3(g.NB * g.U), dim3(256), 0, st, a.k, nullptr, a.dT, a.dTz, g.Hq,
                         g.Hkv, g.N, g.NB, 0.f, nullptr, nullptr, nullptr, a.dvl, a.dv, cS, cSz, a.plan.SL, a.plan.S);
    });
  }
  if (a.coefl) {
    timed("k3_coef_reduce", st, [&] {
      hipLaunchKernelGGL(k3_coef_reduce, dim3(73, g.Hq), dim3(256), 0, st, a.coefl, g.B, g.Hq, g.NB, a.coefs);
    });
  }
}

template <typename T>
void launch_f32_backward(const LaunchGeom& g, const F32BwdArgs<T>& a, hipStream_t st, hipStream_t aux,
                         const Timer& timed) {
  // Two streams, as on the bf16 path: the intra-chunk VJP and then the
  // query-side fold on the second stream beside the state scan; the dk and dv
  // kernels and the coefficient reduction wait on the caller's stream for the
  // event the second stream records after the dk / dv / coefficient part.
  const bool forked = aux != st;
  if (!forked) {
    launch_f32_backward_serial(g, a, st, timed);
    return;
  }
  stream_wait(aux, st);
  // the two orientations in separate launches: the dq part fits two blocks per
  // CU, the dk / dv / coefficient part one
  timed("k3_local_kv", aux, [&] {
    hipLaunchKernelGGL((k3_local<T, 1>), dim3(g.R * g.NB * g.U), dim3(192), 0, aux, a.q, a.k, a.v, a.G, a.Gz,
                       a.labels, a.c0, a.lam, a.gam, a.groups, g.Hq, g.Hkv, g.N, g.NB, a.scale, a.dql, a.dkl, a.dvl,
                       a.coefl);
  });
  hipEvent_t ev_kv = forked ? record_event(aux) : nullptr;
  timed("k3_local_dq", aux, [&] {
    hipLaunchKernelGGL((k3_local<T, 0>), dim3(g.R * g.NB * g.U), dim3(192), 0, aux, a.q, a.k, a.v, a.G, a.Gz,
                       a.labels, a.c0, a.lam, a.gam, a.groups, g.Hq, g.Hkv, g.N, g.NB, a.scale, a.dql, a.dkl, a.dvl,
                       a.coefl);
  });
  if (a.dq) {
    timed("k3_fold_q", aux, [&] {
      hipLaunchKernelGGL((k3_fold<T, 0>), dim3(g.R * g.NB * g.U), dim3(128), 0, aux, a.q, a.G, nullptr, a.Gz, a.wq,
                         a.P, a.Pz, a.dql, g.Hq, g.Hkv, g.N, g.NB, a.dq, nullptr, nullptr, 1, 1);
    });
  }
  // the scan also forms the state coefficient partials (its per-item products)
  if (a.dk || a.dv || a.dwq_part) {
    timed("k3_state_bwd", st, [&] {
      hipLaunchKernelGGL(k3_state_bwd<T>, dim3(kFP / 64, g.U, a.plan.S), dim3(256), 0, st, a.q, a.G, a.Gz, a.wq, a.P, a.Pz,
                         g.Hq, g.Hkv, g.N, g.NB, a.plan.SL, a.dT, a.dTz, a.segt, a.segtz, a.dwq_part);
    });
    if (a.plan.S > 1 && (a.dk || a.dv)) {
      timed("k3_seg_carry", st, [&] {
        const size_t n = (size_t)g.U * kFP * (kD + 1);
        hipLaunchKernelGGL(k3_seg_carry, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a.segt, a.segtz, g.U,
                           a.plan.S);
      });
    }
  }
  // dT holds each segment's own suffix; the dk and dv kernels add the segment
  // carries (the later segments' totals) as they stage the state
  const float* cS = a.plan.S > 1 ? a.segt : nullptr;
  const float* cSz = a.plan.S > 1 ? a.segtz : nullptr;
  if (forked) wait_event(st, ev_kv);
  if (a.dk) {
    timed("k3_fold_k", st, [&] {
      auto* kern = cS ? k3_fold<T, 1, true> : k3_fold<T, 1, false>;
      hipLaunchKernelGGL(kern, dim3(g.NB * g.U), dim3(128), 0, st, a.k, nullptr, a.v, nullptr, nullptr,
                         a.dT, a.dTz, a.dkl, g.Hq, g.Hkv, g.N, g.NB, a.dk, cS, cSz, a.plan.SL, a.plan.S);
    });
  }
  if (a.dv) {
    timed("k3_readout_v", st, [&] {
      auto* kern = cS ? k3_readout<T, 1, true> : k3_readout<T, 1, false>;
      hipLaunchKernelGGL(kern, dim3(g.NB * g.U), dim3(256), 0, st, a.k, nullptr, a.dT, a.dTz, g.Hq,
                         g.Hkv, g.N, g.NB, 0.f, nullptr, nullptr, nullptr, a.dvl, a.dv, cS, cSz, a.plan.SL, a.plan.S);
    });
  }
  if (a.coefl) {
    timed("k3_coef_reduce", st, [&] {
      hipLaunchKernelGGL(k3_coef_reduce, dim3(73, g.Hq), dim3(256), 0, st, a.coefl, g.B, g.Hq, g.NB, a.coefs);
    });
  }
}

#define OAL_F32MMA_INST(T)                                                                                        \
  template void launch_f32_state_fwd<T>(const LaunchGeom&, const T*, const T*, float*, float*, hipStream_t,        \
                                        const Timer&);                                                            \
  template void launch_f32_intra_fwd<T>(const LaunchGeom&, const T*, const T*, const T*, const int32_t*,         \
                                        const float*, const float*, const float*, int, float, float*, float*,       \
                                        hipStream_t, const Timer&);                                                 \
  template void launch_f32_readout_fwd<T>(const LaunchGeom&, const T*, const float*, const float*, const float*, \
                                          float, float*, float*, T*, hipStream_t, const Timer&);                  \
  template void launch_f32_backward<T>(const LaunchGeom&, const F32BwdArgs<T>&, hipStream_t, hipStream_t,          \
                                       const Timer&);
OAL_F32MMA_INST(float)
OAL_F32MMA_INST(uint16_t)
#undef OAL_F32MMA_INST

}  // namespace oal
