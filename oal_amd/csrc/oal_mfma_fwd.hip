// bf16 matrix-core (MFMA) forward for gfx950.
//
// k2_state_fwd  : per (32-slot tile, unit) sequential chunk scan; the running
//                 state lives in MFMA accumulators; stores the exclusive prefix
//                 P_c in two k-blocked bf16 layouts plus the fp32 denominator
//                 column in natural feature order.
// k2_out_fwd    : per (query head, chunk, unit) one wave: denominator state term
//                 as a 64x64 quadratic form, intra-chunk kernel from MFMA group
//                 sums, state readout phi_Q . P_c with query features generated
//                 in registers, intra term kappa . V, normalize.
//
// Saved layouts (per unit u and chunk c; "tile" = 32 slots, "k-step" = 16 slots):
//   PT [u][c][kKS][64 e][16]        bf16  (readout B operand: slots contiguous)
//   PR [u][c][kS/32][4][32][16 e]   bf16  (backward A operand: values contiguous)
//   PZ [u][c][kFP]                  f32   (denominator column, natural order)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"

namespace oal {

__constant__ SlotTable kSlot = make_slot_table();

// Per-head slot coefficients: wq of natural feature nat(slot), 0 for invalid slots.
__global__ __launch_bounds__(256) void k2_slot_coefficients(const int32_t* __restrict__ labels,
                                                            const float* __restrict__ c0,
                                                            const float* __restrict__ lam,
                                                            const float* __restrict__ gam, int G, float scale,
                                                            float* __restrict__ wqs) {
  const int h = blockIdx.x;
  auto label = [&](int d) {
    int g = labels[h * kD + d];
    return g < 0 ? 0 : (g >= G ? G - 1 : g);
  };
  for (int s = threadIdx.x; s < kS; s += blockDim.x) {
    const int n = kSlot.nat[s];
    const int r = kSlot.ar[s], c = kSlot.ac[s];
    float w = 0.f;
    if (n == 0) {
      w = c0[h];
    } else if (n > 0 && n <= kD) {
      w = scale * lam[(size_t)h * G + label(r)];
    } else if (n > kD) {
      w = (r == c ? 1.f : 2.f) * scale * scale * gam[((size_t)h * G + label(r)) * G + label(c)];
    }
    wqs[(size_t)h * kS + s] = w;
  }
}

template <typename T>
__device__ __forceinline__ float ldf(const T* p, size_t i) {
  return to_f(p[i]);
}

// ---------------------------------------------------------------------------
// Forward state scan. grid (kS/32, U), one wave. Lane row = slot (32 per tile),
// accumulator N-tiles: values 0-31, 32-63, and [den, 0...] (a ones column).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(64) void k2_state_fwd(const T* __restrict__ k, const T* __restrict__ v, int N, int NB,
                                                   uint16_t* __restrict__ PT, uint16_t* __restrict__ PR,
                                                   float* __restrict__ PZ) {
  __shared__ float kT[kRow][kC + 4];            // kT[d][tok], rows 64 = valid flag, 65 = 0
  __shared__ __attribute__((aligned(16))) __bf16 vT[96][kC + 8];  // vT[e][tok], row 64 = valid flag
  __shared__ float stage[32][97];

  const int tile = blockIdx.x, u = blockIdx.y;
  const int l = threadIdx.x, s = l >> 5, row = l & 31;
  const int slot = tile * 32 + row;
  const int ar = kSlot.ar[slot], ac = kSlot.ac[slot];
  const size_t base = (size_t)u * N * kD;

  // constant rows of vT (values rows are rewritten per chunk)
  for (int idx = l; idx < 31 * (kC + 8); idx += 64) vT[65 + idx / (kC + 8)][idx % (kC + 8)] = (__bf16)0.f;

  f32x16 acc[3];
#pragma unroll
  for (int n = 0; n < 3; ++n) acc[n] = f32x16{};

  const size_t chunk_elems = (size_t)kKS * 64 * 16;  // per (u, c) for PT and PR
  for (int ch = 0; ch < NB; ++ch) {
    // 1. exclusive prefix P_c = current accumulators
#pragma unroll
    for (int n = 0; n < 3; ++n) {
#pragma unroll
      for (int i = 0; i < 16; ++i) stage[c32_row(i, l)][32 * n + row] = acc[n][i];
    }
    __syncthreads();
    uint16_t* pt = PT + ((size_t)u * NB + ch) * chunk_elems;
    uint16_t* pr = PR + ((size_t)u * NB + ch) * chunk_elems;
    {
      // PT[t][e][16]: lane -> (k-step half hh = s, e = row and row + 32)
      const int t = 2 * tile + s;
#pragma unroll
      for (int eh = 0; eh < 2; ++eh) {
        const int e = row + 32 * eh;
        uint32_t w[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) w[q] = pack_bf16x2(stage[16 * s + 2 * q][e], stage[16 * s + 2 * q + 1][e]);
        uint4* dst = reinterpret_cast<uint4*>(pt + ((size_t)t * 64 + e) * 16);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
      }
      // PR[tile][kk][32][16]: lane -> (slot row, kk = 2s, 2s+1)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const int kk = 2 * s + kh;
        uint32_t w[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) w[q] = pack_bf16x2(stage[row][16 * kk + 2 * q], stage[row][16 * kk + 2 * q + 1]);
        uint4* dst = reinterpret_cast<uint4*>(pr + (((size_t)tile * 4 + kk) * 32 + row) * 16);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
      }
      if (s == 0) {
        const int n = kSlot.nat[slot];
        if (n >= 0) PZ[((size_t)u * NB + ch) * kFP + n] = stage[row][64];
      }
    }
    // 2. stage chunk c
    __syncthreads();
    const int tok0 = ch * kC;
    for (int idx = l; idx < kC * kD; idx += 64) {
      const int j = idx >> 6, d = idx & 63, tok = tok0 + j;
      const bool ok = tok < N;
      kT[d][j] = ok ? ldf(k, base + (size_t)tok * kD + d) : 0.f;
      vT[d][j] = (__bf16)(ok ? ldf(v, base + (size_t)tok * kD + d) : 0.f);
    }
    {
      const bool ok = tok0 + l < N;
      kT[64][l] = ok ? 1.f : 0.f;
      kT[65][l] = 0.f;
      vT[64][l] = (__bf16)(ok ? 1.f : 0.f);
    }
    __syncthreads();
    // 3. T_c = phi_K^T [V, 1]
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int j0 = 16 * kk + 8 * s;
      float f[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) f[q] = kT[ar][j0 + q] * kT[ac][j0 + q];
      const bf16x8 a = pack8(f);
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(&vT[32 * n + row][j0]);
        acc[n] = mfma32(a, b, acc[n]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Forward readout, one wave per (query head, chunk, unit).
// ---------------------------------------------------------------------------
template <int T>
__device__ __forceinline__ void readout_steps(const float (&qa)[kD], const float (&qb)[kD], const float* wq,
                                              const uint16_t* pt, int lane, f32x16 (&acc)[2][2]) {
  const int s = lane >> 5, row = lane & 31;
  float w[8];
  const float4 w0 = *reinterpret_cast<const float4*>(wq + 16 * T + 8 * s);
  const float4 w1 = *reinterpret_cast<const float4*>(wq + 16 * T + 8 * s + 4);
  w[0] = w0.x; w[1] = w0.y; w[2] = w0.z; w[3] = w0.w;
  w[4] = w1.x; w[5] = w1.y; w[6] = w1.z; w[7] = w1.w;
  const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(pt + ((size_t)T * 64 + row) * 16 + 8 * s);
  const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(pt + ((size_t)T * 64 + 32 + row) * 16 + 8 * s);
  const bf16x8 a0 = feature_fragment<T>(qa, w);
  const bf16x8 a1 = feature_fragment<T>(qb, w);
  acc[0][0] = mfma32(a0, b0, acc[0][0]);
  acc[0][1] = mfma32(a0, b1, acc[0][1]);
  acc[1][0] = mfma32(a1, b0, acc[1][0]);
  acc[1][1] = mfma32(a1, b1, acc[1][1]);
  if constexpr (T + 1 < kKS) readout_steps<T + 1>(qa, qb, wq, pt, lane, acc);
}

// 8 consecutive elements of a row as a bf16 MFMA fragment.
__device__ __forceinline__ bf16x8 load8(const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ bf16x8 load8(const float* p) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return pack8(v);
}

template <typename T>
__global__ __launch_bounds__(64) void k2_out_fwd(const T* __restrict__ q, const T* __restrict__ k,
                                                 const T* __restrict__ v, const float* __restrict__ wqs,
                                                 const uint16_t* __restrict__ PT, const float* __restrict__ PZ,
                                                 const int32_t* __restrict__ labels, const float* __restrict__ c0,
                                                 const float* __restrict__ lam, const float* __restrict__ gam, int G,
                                                 int Hq, int Hkv, int N, int NB, float scale, float floor,
                                                 T* __restrict__ out, float* __restrict__ num,
                                                 float* __restrict__ den) {
  constexpr int LD = kD + 8;  // bf16 row stride (bank spread)
  __shared__ __attribute__((aligned(16))) __bf16 qs[kC][LD];
  __shared__ __attribute__((aligned(16))) __bf16 vT[kD][LD];
  __shared__ __attribute__((aligned(16))) __bf16 km[kC][LD];  // Mz for the quadratic form, then kappa
  __shared__ float bz[kD];
  __shared__ float denS[kC], denL[kC];
  __shared__ int lab[kD];
  __shared__ float lamh[8], gamh[64];

  const int hh = blockIdx.x, ch = blockIdx.y, u = blockIdx.z;
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int l = threadIdx.x, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;
  const float* pz = PZ + ((size_t)u * NB + ch) * kFP;
  const float sc2 = scale * scale;

  // --- stage q and v^T, group tables -----------------------------------------
  for (int idx = l; idx < kC * kD; idx += 64) {
    const int j = idx >> 6, d = idx & 63, tok = tok0 + j;
    const bool ok = tok < N;
    qs[j][d] = (__bf16)(ok ? ldf(q, qbase + (size_t)tok * kD + d) : 0.f);
    vT[d][j] = (__bf16)(ok ? ldf(v, kbase + (size_t)tok * kD + d) : 0.f);
  }
  {
    int g = labels[h * kD + l];
    lab[l] = g < 0 ? 0 : (g >= G ? G - 1 : g);
    if (l < G) lamh[l] = lam[(size_t)h * G + l];
    if (l < G * G) gamh[l] = gam[(size_t)h * G * G + l];
    denL[l] = 0.f;
  }
  __syncthreads();
  const float c0h = c0[h];
  for (int idx = l; idx < kD * kD; idx += 64) {
    const int r = idx >> 6, c = idx & 63;
    const int hi = r > c ? r : c, lo = r > c ? c : r;
    km[r][c] = (__bf16)(sc2 * gamh[lab[r] * G + lab[c]] * pz[1 + kD + pair_index(hi, lo)]);
  }
  bz[l] = scale * lamh[lab[l]] * pz[1 + l];
  const float az = c0h * pz[0];
  __syncthreads();

  // --- denominator state term: den_i = az + q_i . (bz + Mz q_i) -------------
  {
    float part[2] = {0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int md = 0; md < 2; ++md) {
        f32x16 z = f32x16{};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(&km[32 * md + row][16 * kk + 8 * s]);
          const bf16x8 bb = *reinterpret_cast<const bf16x8*>(&qs[32 * nt + row][16 * kk + 8 * s]);
          z = mfma32(a, bb, z);
        }
        const int tok = 32 * nt + row;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int d = 32 * md + c32_row(i, l);
          part[nt] += (float)qs[tok][d] * (z[i] + bz[d]);
        }
      }
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const float tot = part[nt] + __shfl_xor(part[nt], 32, 64);
      if (s == 0) denS[32 * nt + row] = az + tot;
    }
  }
  __syncthreads();  // Mz is dead; km now holds kappa

  // --- intra-chunk kappa via group sums (16x16x32 MFMA) ----------------------
  {
    const int r16 = l & 15, g16 = l >> 4;
    uint32_t mask[8][2][4];
#pragma unroll
    for (int g = 0; g < 8; ++g)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int d = 32 * kk + 8 * g16 + 2 * w;
          mask[g][kk][w] = (lab[d] == g ? 0x0000ffffu : 0u) | (lab[d + 1] == g ? 0xffff0000u : 0u);
        }
    for (int ti = 0; ti < 4; ++ti) {
      for (int tj = 0; tj <= ti; ++tj) {
        f32x4 sg[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) sg[g] = f32x4{};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
          const u32x4 qa = *reinterpret_cast<const u32x4*>(&qs[16 * ti + r16][32 * kk + 8 * g16]);
          const int tokj = tok0 + 16 * tj + r16;
          bf16x8 kb;
          if (tokj < N) {
            kb = load8(k + kbase + (size_t)tokj * kD + 32 * kk + 8 * g16);
          } else {
            kb = bf16x8{};
          }
#pragma unroll
          for (int g = 0; g < 8; ++g) {
            if (g < G) {
              const u32x4 m = {mask[g][kk][0], mask[g][kk][1], mask[g][kk][2], mask[g][kk][3]};
              sg[g] = mfma16(__builtin_bit_cast(bf16x8, qa & m), kb, sg[g]);
            }
          }
        }
        float rs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ii = 16 * ti + c16_row(i, l), jj = 16 * tj + r16;
          float kv = 0.f;
          if (jj <= ii && tok0 + ii < N) {
            kv = c0h;
#pragma unroll
            for (int g = 0; g < 8; ++g) {
              if (g < G) {
                float inner = lamh[g];
#pragma unroll
                for (int g2 = 0; g2 < 8; ++g2)
                  if (g2 < G) inner += gamh[g * G + g2] * (sg[g2][i] * scale);
                kv += (sg[g][i] * scale) * inner;
              }
            }
          }
          const __bf16 kb16 = (__bf16)kv;
          km[ii][jj] = kb16;
          rs[i] = (float)kb16;
        }
        if (tj < ti) {
#pragma unroll
          for (int i = 0; i < 4; ++i) km[16 * tj + c16_row(i, l)][16 * ti + r16] = (__bf16)0.f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = rs[i];
          x += __shfl_xor(x, 1, 64);
          x += __shfl_xor(x, 2, 64);
          x += __shfl_xor(x, 4, 64);
          x += __shfl_xor(x, 8, 64);
          rs[i] = x;
        }
        if (r16 == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) denL[16 * ti + c16_row(i, l)] += rs[i];
        }
      }
    }
  }
  __syncthreads();

  // --- state readout -------------------------------------------------------
  f32x16 acc[2][2];
  {
    float qa[kD], qb[kD];
#pragma unroll
    for (int m = 0; m < kD; ++m) {
      qa[m] = (float)qs[row][(m + 32 * s) & 63];
      qb[m] = (float)qs[32 + row][(m + 32 * s) & 63];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    const uint16_t* pt = PT + ((size_t)u * NB + ch) * ((size_t)kKS * 64 * 16);
    readout_steps<0>(qa, qb, wqs + (size_t)h * kS, pt, l, acc);
  }
  // --- intra term kappa . V --------------------------------------------------
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk < 2 * (mt + 1)) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(&km[32 * mt + row][16 * kk + 8 * s]);
          const bf16x8 bb = *reinterpret_cast<const bf16x8*>(&vT[32 * nt + row][16 * kk + 8 * s]);
          acc[mt][nt] = mfma32(a, bb, acc[mt][nt]);
        }
      }
  // --- normalize and write (accumulator layout: 32 consecutive columns per row)
  const size_t dbase = (size_t)(b * Hq + h) * N;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int j = 32 * mt + c32_row(i, l), tok = tok0 + j;
      if (tok < N) {
        const float dd = denS[j] + denL[j];
        const float inv = 1.f / (floor > 0.f ? fmaxf(dd, floor) : dd);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const size_t o = qbase + (size_t)tok * kD + 32 * nt + row;
          num[o] = acc[mt][nt][i];
          out[o] = from_f<T>(acc[mt][nt][i] * inv);
        }
        if (row == 0) den[dbase + tok] = dd;
      }
    }
}

// ---------------------------------------------------------------------------
// MFMA layout self-test: checks the accumulator layouts assumed above.
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
  atomicAdd(errors, bad);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
size_t mfma_saved_bytes(int Hq, int U, int NB) {
  const size_t chunk = (size_t)kKS * 64 * 16 * sizeof(uint16_t);
  return align256(sizeof(float) * (size_t)Hq * kS) + 2 * align256(chunk * U * NB) +
         align256(sizeof(float) * (size_t)U * NB * kFP);
}

MfmaSaved mfma_saved_view(void* base, int Hq, int U, int NB) {
  char* p = static_cast<char*>(base);
  const size_t chunk = (size_t)kKS * 64 * 16 * sizeof(uint16_t);
  MfmaSaved v;
  v.wqs = reinterpret_cast<float*>(p);
  p += align256(sizeof(float) * (size_t)Hq * kS);
  v.PT = reinterpret_cast<uint16_t*>(p);
  p += align256(chunk * U * NB);
  v.PR = reinterpret_cast<uint16_t*>(p);
  p += align256(chunk * U * NB);
  v.PZ = reinterpret_cast<float*>(p);
  return v;
}

template <typename T>
void launch_mfma_forward(const LaunchGeom& g, const void* q, const void* k, const void* v, const int32_t* labels,
                         const float* c0, const float* lam, const float* gam, int groups, float scale, float floor,
                         void* out, float* num, float* den, void* saved, hipStream_t st, const Timer& timed) {
  MfmaSaved sv = mfma_saved_view(saved, g.Hq, g.U, g.NB);
  const T* qt = static_cast<const T*>(q);
  const T* kt = static_cast<const T*>(k);
  const T* vt = static_cast<const T*>(v);
  timed("k2_slot_coefficients", st, [&] {
    hipLaunchKernelGGL(k2_slot_coefficients, dim3(g.Hq), dim3(256), 0, st, labels, c0, lam, gam, groups, scale,
                       sv.wqs);
  });
  timed("k2_state_fwd", st, [&] {
    hipLaunchKernelGGL(k2_state_fwd<T>, dim3(kS / 32, g.U), dim3(64), 0, st, kt, vt, g.N, g.NB, sv.PT, sv.PR, sv.PZ);
  });
  timed("k2_out_fwd", st, [&] {
    hipLaunchKernelGGL(k2_out_fwd<T>, dim3(g.R, g.NB, g.U), dim3(64), 0, st, qt, kt, vt, sv.wqs, sv.PT, sv.PZ,
                       labels, c0, lam, gam, groups, g.Hq, g.Hkv, g.N, g.NB, scale, floor, static_cast<T*>(out), num,
                       den);
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
