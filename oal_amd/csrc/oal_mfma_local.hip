// Intra-chunk (local) VJP of the bf16 matrix-core backward for gfx950.
//
// For one chunk, with s_g(i,j) = scale * sum_{d in g} q_i[d] k_j[d] and
// ds(i,j) = g_i . v_j + gz_i  (j <= i; g, gz from the normalization VJP):
//   dq_i[d] += scale lam_g(d) sum_j ds k_j[d] + 2 scale sum_h Gam_g(d)h sum_j ds s_h k_j[d]
//   dk_j[d] += the same with q_i in place of k_j (summed over the query heads)
//   dv_j    += sum_i kappa(i,j) g_i
//   dc0 += sum ds,  dlam_g += sum ds s_g,  dGam_gh += sum ds s_g s_h
// (reference: closed-form state VJP grouped_reference.py:214-318 and the local
// score terms of hd_block_gemm_backward_wave.py:253-477, here in group-sum form).
// The 64x64 chunk is covered by three lower 32x32 tiles (key tile jt, query
// tile it) = (0,0), (0,1), (1,1). Group sums and ds come from
// v_mfma_f32_32x32x16_bf16 on row-major operands; their accumulators are fed
// straight back into the MFMA as the K-major operand of the dq / dk / dv
// products, whose other operand is the transposed bf16 copy of K, q or G.
//
// k2_local_dq    one block per (query head, chunk): dq local part and the state
//                part of the denominator's dq (gz_i (bz + 2 Mz q_i)). With the
//                coefficient gradients requested it also writes the per-(head,
//                chunk) coefficient partials from the same group sums.
// k2_local_dk    one block per (unit, chunk): dk local part summed over the
//                unit's query heads in registers (group sums one at a time).
// k2_local_dv    one block per (unit, chunk): the dv local part from the
//                forward's saved kappa, summed over the unit's query heads.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"

namespace oal {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

__device__ __forceinline__ int clamp_label(int g, int G) { return g < 0 ? 0 : (g >= G ? G - 1 : g); }

// Group mask table for fragments covering dims d, d + 1 with
// d = 16 kk + 8 ss + 2 w: entry [kk][g][ss][w]; 256 entries, one per thread.
__device__ __forceinline__ void build_masks(uint32_t (*mk)[8][2][4], const int32_t* __restrict__ labels, int h,
                                            int G, int t0) {
  for (int t = t0; t < 256; t += blockDim.x) {
    const int kk = t >> 6, g = (t >> 3) & 7, ss = (t >> 2) & 1, w = t & 3;
    const int d = 16 * kk + 8 * ss + 2 * w;
    const int g0 = clamp_label(labels[h * kD + d], G), g1 = clamp_label(labels[h * kD + d + 1], G);
    mk[kk][g][ss][w] = (g0 == g ? 0x0000ffffu : 0u) | (g1 == g ? 0xffff0000u : 0u);
  }
}

__device__ __forceinline__ bf16x8 masked(bf16x8 f, const uint32_t* m) {
  const u32x4 mm = *reinterpret_cast<const u32x4*>(m);
  return __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, f) & mm);
}

// Tile pair tp -> (key tile jt, query tile it).
__device__ __forceinline__ int tile_jt(int tp) { return tp == 2 ? 1 : 0; }
__device__ __forceinline__ int tile_it(int tp) { return tp == 0 ? 0 : 1; }

}  // namespace

// ---------------------------------------------------------------------------
// dq local part + denominator-state dq, one block per (query head, chunk),
// grid R * NB * U (XCD-ordered), 3 waves = tile pairs 0..2 (orientation
// C[j][i] for the group sums; dq accumulators C[i][d], lane = d):
//   dq[i][d] = sum_h coef_h(d) sum_j X_h[i][j] K[j][d], X_h = ds o s'_h, X_8 = ds
// with s'_h the unscaled group sum (s_h = scale s'_h), computed one group at a
// time, coef_h(d) = 2 scale^2 Gam[g(d)][h], coef_8(d) = scale lam[g(d)];
// waves 0 and 1 (query tiles 0, 1) add
// gz_i (bz_d + 2 (Mz q_i)_d), Mz = gm o PZm, and write dqf.
// COEF: the eight group sums are kept (two waves per SIMD instead of three),
// the block also writes the coefficient partials from them (with ds[i][j] =
// g_i . v_j + gz_i on live entries: [0] sum ds, [1 + g] sum ds s_g,
// [9 + 8 g + h] sum ds s_g s_h in the full symmetric 8 x 8 layout, each a
// fixed-order sum over the block's 192 lanes), and the dq products take s_h
// from those registers.
// ---------------------------------------------------------------------------
template <typename T, bool COEF>
__global__ __launch_bounds__(192, COEF ? 2 : 3) void k2_local_dq(const T* __restrict__ q, const T* __restrict__ k,
                                                   const T* __restrict__ v, const uint16_t* __restrict__ G16,
                                                   const float* __restrict__ Gz, const uint16_t* __restrict__ KT16,
                                                   const float* __restrict__ PZ, const float* __restrict__ PZm,
                                                   const int32_t* __restrict__ labels, const float* __restrict__ lam,
                                                   const float* __restrict__ gam, const float* __restrict__ gm,
                                                   const float* __restrict__ lb, int G, int Hq, int Hkv, int N,
                                                   int NB, float scale, float* __restrict__ dqf,
                                                   float* __restrict__ coefl) {
  constexpr int LD = kD + 8;
  __shared__ __attribute__((aligned(16))) uint32_t mk[4][8][2][4];
  __shared__ __attribute__((aligned(16))) __bf16 Mz[kD][LD];
  __shared__ __attribute__((aligned(16))) uint16_t kts[kD][LD];  // k^T of the chunk
  __shared__ float cft[9][kD];  // coef_h(d), h = 0..8
  __shared__ float bz[kD];
  __shared__ float gzs[kC];
  __shared__ float red[2][16][64];  // wave 2's dq (query tile 1)
  __shared__ float cp[COEF ? 3 * 64 : 1][45];  // per-lane coefficient partials
  __shared__ float cred[COEF ? 4 * 45 : 1];

  int hh, ch, u;
  head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;
  const size_t cbase = (size_t)u * NB + ch;
  const size_t np = (size_t)NB * kC;

  // The prologue's global loads are issued together, labels first (the
  // coefficient rows depend on them), and the lane's operand rows right after
  // the Mz stores: two round trips in all instead of one per loop. Loads and
  // LDS stores are unconditional: a thread past an item count wraps onto an
  // item another thread also holds and stores the same value there.
  // masks: thread t = tid & 31 covers dims d, d + 1, d = 16 kk + 8 ss + 2 w
  const int mt = tid & 31, mkk = mt >> 3, mss = (mt >> 2) & 1, mw = mt & 3;
  const int md = 16 * mkk + 8 * mss + 2 * mw;
  const int ml0 = labels[h * kD + md], ml1 = labels[h * kD + md + 1];
  const int cd = tid & 63;  // dim of the coefficient table, bz and token of gzs
  const int cl = clamp_label(labels[h * kD + cd], G);
  // Mz = gm o PZm (bf16): items e = tid, tid + 192 (< 256): row e / 4, columns 16 (e % 4) .. + 15
  float4 mg[2][4], mz[2][4];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int e = (tid + 192 * x) & 255, r = e >> 2, qq = e & 3;
    const float4* gp = reinterpret_cast<const float4*>(gm + ((size_t)h * kD + r) * kD + 16 * qq);
    const float4* zp = reinterpret_cast<const float4*>(PZm + (cbase * kD + r) * kD + 16 * qq);
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      mg[x][y] = gp[y];
      mz[x][y] = zp[y];
    }
  }
  const float lbv = lb[(size_t)h * kD + cd], pzv = PZ[cbase * kFP + 1 + cd];
  const float gzv = Gz[(size_t)(b * Hq + h) * N + min(tok0 + cd, N - 1)];
  // k^T of the chunk: 512 pieces of 8 tokens, pieces tid, tid + 192, tid + 384 (< 512)
  bf16x8 ktv[3];
#pragma unroll
  for (int x = 0; x < 3; ++x) {
    const int pc = (tid + 192 * x) & 511, d = pc >> 3, c = 8 * (pc & 7);
    ktv[x] = *reinterpret_cast<const bf16x8*>(KT16 + ((size_t)u * kD + d) * np + tok0 + c);
  }
  // coefficient rows of dim cd: gam[g(cd)][0..7], lam[g(cd)] (group index clamped)
  float cg[9];
#pragma unroll
  for (int h2 = 0; h2 < 8; ++h2) cg[h2] = gam[((size_t)h * G + cl) * G + min(h2, G - 1)];
  cg[8] = lam[(size_t)h * G + cl];

  {
    const int g0 = clamp_label(ml0, G), g1 = clamp_label(ml1, G);
#pragma unroll
    for (int g = 0; g < 8; ++g) mk[mkk][g][mss][mw] = (g0 == g ? 0x0000ffffu : 0u) | (g1 == g ? 0xffff0000u : 0u);
  }
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int e = (tid + 192 * x) & 255, r = e >> 2, qq = e & 3;
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2) {
      const float4 g0 = mg[x][2 * i2], g1 = mg[x][2 * i2 + 1], z0 = mz[x][2 * i2], z1 = mz[x][2 * i2 + 1];
      float y[8] = {g0.x * z0.x, g0.y * z0.y, g0.z * z0.z, g0.w * z0.w,
                    g1.x * z1.x, g1.y * z1.y, g1.z * z1.z, g1.w * z1.w};
      *reinterpret_cast<bf16x8*>(&Mz[r][16 * qq + 8 * i2]) = pack8(y);
    }
  }
  const int tp = wv, jt = tile_jt(tp), it = tile_it(tp);
  const int jr = tok0 + 32 * jt + row, ir = tok0 + 32 * it + row;  // this lane's operand rows
  const bool jok = jr < N, iok = ir < N;
  const size_t jo = (size_t)(jok ? jr : N - 1) * kD, io = (size_t)(iok ? ir : N - 1) * kD;
  bf16x8 kf[4], qf[4], vf[4], gf[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int c = 16 * kk + 8 * s;
    kf[kk] = row8(k + kbase + jo + c, jok);
    qf[kk] = row8(q + qbase + io + c, iok);
    vf[kk] = row8(v + kbase + jo + c, jok);
    gf[kk] = row8(G16 + qbase + io + c, iok);
  }
#pragma unroll
  for (int x = 0; x < 3; ++x) {
    const int pc = (tid + 192 * x) & 511;
    *reinterpret_cast<bf16x8*>(&kts[pc >> 3][8 * (pc & 7)]) = ktv[x];
  }
  bz[cd] = lbv * pzv;
  gzs[cd] = tok0 + cd < N ? gzv : 0.f;
#pragma unroll
  for (int h2 = 0; h2 < 8; ++h2) cft[h2][cd] = h2 < G ? 2.f * scale * scale * cg[h2] : 0.f;
  cft[8][cd] = scale * cg[8];
  lds_sync();

  f32x16 ds = f32x16{};
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) ds = mfma32(vf[kk], gf[kk], ds);
  // lane column i = 32 it + row; register rows j = 32 jt + c32_row(r)
  const int i = 32 * it + row;
  const float gzi = gzs[i];  // zero past N
  float dsv[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int j = 32 * jt + c32_row(r, l);
    dsv[r] = j <= i ? ds[r] + gzi : 0.f;
  }
  f32x16 sgs[COEF ? 8 : 1];
  if constexpr (COEF) {
    // all eight group sums, then the partials [0] sum ds, [1 + g] sum ds s_g,
    // [9 + packed (g <= h)] sum ds s_g s_h over this lane's 16 entries
#pragma unroll
    for (int g = 0; g < 8; ++g) sgs[g] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int g = 0; g < 8; ++g) sgs[g] = mfma32(masked(kf[kk], &mk[kk][g][s][0]), qf[kk], sgs[g]);
    float ca[45];
#pragma unroll
    for (int e = 0; e < 45; ++e) ca[e] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float sv[8], tv[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        sv[g] = sgs[g][r];  // unscaled; the sums are scaled once below
        tv[g] = dsv[r] * sv[g];
      }
      ca[0] += dsv[r];
      int e = 9;
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        ca[1 + g] += tv[g];
#pragma unroll
        for (int h2 = g; h2 < 8; ++h2) {
          ca[e] = fmaf(tv[g], sv[h2], ca[e]);
          ++e;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 45; ++e) cp[tid][e] = ca[e] * (e == 0 ? 1.f : e < 9 ? scale : scale * scale);
  }
  bf16x8 kt[2][2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int t = 0; t < 2; ++t)
      kt[dt][t] = *reinterpret_cast<const bf16x8*>(&kts[32 * dt + row][32 * jt + 16 * t + 8 * s]);
  // this lane's query row again for the den-state term: the prologue's copy
  // would stay live across the partials and spill. The pointer goes through an
  // empty asm so that the compiler cannot fold the reload into the first load.
  const T* qre = q;
  asm volatile("" : "+s"(qre));
  bf16x8 qz[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) qz[kk] = row8(qre + qbase + io + 16 * kk + 8 * s, iok);
  f32x16 dq[2] = {f32x16{}, f32x16{}};
#pragma unroll
  for (int h2 = 0; h2 < 9; ++h2) {
    float x[16];
    if (h2 < 8) {
      f32x16 sh;
      if constexpr (COEF) {
        sh = sgs[h2];
      } else {
        sh = f32x16{};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) sh = mfma32(masked(kf[kk], &mk[kk][h2][s][0]), qf[kk], sh);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = dsv[r] * sh[r];  // the scale of s_h is in cft
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = dsv[r];
    }
    const bf16x8 f0 = acc_kfrag(x, 0, s), f1 = acc_kfrag(x, 1, s);
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      f32x16 p = mfma32(f0, kt[dt][0], f32x16{});
      p = mfma32(f1, kt[dt][1], p);
      const float cf = cft[h2][32 * dt + row];
#pragma unroll
      for (int r = 0; r < 16; ++r) dq[dt][r] = fmaf(cf, p[r], dq[dt][r]);
    }
  }
  if (wv == 2) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[dt][r][l] = dq[dt][r];
  } else {
    // den-state dq of query tile it = wv: gz_i (bz_d + 2 Z[i][d]), Z = q Mz; the
    // query fragments qz are this lane's row i = 32 it + row
    float gzr[16];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) gzr[4 * a + vv] = gzs[32 * it + 8 * a + 4 * s + vv];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      f32x16 z = f32x16{};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        z = mfma32(qz[kk], *reinterpret_cast<const bf16x8*>(&Mz[32 * dt + row][16 * kk + 8 * s]), z);
      const float bzd = bz[32 * dt + row];
#pragma unroll
      for (int r = 0; r < 16; ++r) dq[dt][r] = fmaf(gzr[r], bzd + 2.f * z[r], dq[dt][r]);
    }
  }
  __syncthreads();
  if (wv < 2) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = dq[dt][r];
        if (wv == 1) x += red[dt][r][l];
        const int tok = tok0 + 32 * wv + c32_row(r, l);
        if (tok < N) dqf[qbase + (size_t)tok * kD + 32 * dt + row] = x;
      }
  }
  if constexpr (COEF) {
    // column sums over the 192 lanes (4 interleaved partial sums per column,
    // then their sum), expanded to the symmetric [1 + 8 + 8 x 8] layout
    if (tid < 180) {
      const int e = tid % 45, part = tid / 45;
      float x = 0.f;
      for (int r = part; r < 192; r += 4) x += cp[r][e];
      cred[tid] = x;
    }
    __syncthreads();
    if (tid < 73) {
      int e = tid;
      if (tid >= 9) {
        int g = (tid - 9) >> 3, h2 = (tid - 9) & 7;
        if (h2 < g) {
          const int t2 = g;
          g = h2;
          h2 = t2;
        }
        e = 9 + g * 8 - g * (g - 1) / 2 + (h2 - g);
      }
      const size_t bn = (size_t)(gridDim.x / (R * NB) / Hkv) * NB;
      coefl[((size_t)h * 73 + tid) * bn + (size_t)b * NB + ch] =
          (cred[e] + cred[45 + e]) + (cred[90 + e] + cred[135 + e]);
    }
  }
}

// ---------------------------------------------------------------------------
// dk and dv local parts, one block per (unit, chunk), 3 waves (tile pairs),
// summed over the unit's query heads in registers (orientation C[i][j],
// lane = key token j). Outputs dkl / dvl [U][N][64] (f32).
// ---------------------------------------------------------------------------
struct LocalTile {
  int tp, jt, it, j, ir, jr;
  bool iok, jok;
  size_t io, jo;
};

__device__ __forceinline__ LocalTile local_tile(int tp, int tok0, int N, int row) {
  LocalTile t;
  t.tp = tp;
  t.jt = tile_jt(tp);
  t.it = tile_it(tp);
  t.j = 32 * t.jt + row;
  t.ir = tok0 + 32 * t.it + row;
  t.jr = tok0 + 32 * t.jt + row;
  t.iok = t.ir < N;
  t.jok = t.jr < N;
  t.io = (size_t)(t.iok ? t.ir : N - 1) * kD;
  t.jo = (size_t)(t.jok ? t.jr : N - 1) * kD;
  return t;
}

__device__ __forceinline__ int unit_chunk_block(int NB, int& ch) {
  const int total = gridDim.x, id = blockIdx.x;
  const int wid = (total & 7) == 0 ? (id & 7) * (total >> 3) + (id >> 3) : id;
  ch = wid % NB;
  return wid / NB;
}

// Combine tile pair 1 into tile pair 0 (both key tile 0) and write out[j][e].
__device__ __forceinline__ void local_write(float (*red)[16][64], const f32x16 (&acc)[2], const LocalTile& t,
                                           int l, int row, int tok0, int N, size_t kbase, float* __restrict__ out) {
  if (t.tp == 1) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[n][r][l] = acc[n][r];
  }
  __syncthreads();
  if (t.tp != 1) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = acc[n][r];
        if (t.tp == 0) x += red[n][r][l];
        const int tok = tok0 + 32 * t.jt + c32_row(r, l);
        if (tok < N) out[kbase + (size_t)tok * kD + 32 * n + row] = x;
      }
  }
}

// dk[j][d] += sum_h coef_h(d) sum_i X_h[i][j] q_i[d], X_h = ds o s'_h, X_8 = ds,
// with s'_h the unscaled group sum computed one group at a time and the
// coefficients of k2_local_dq (the scale folded into coef_h).
template <typename T>
__global__ __launch_bounds__(192) void k2_local_dk(const T* __restrict__ q, const T* __restrict__ k,
                                                   const T* __restrict__ v, const uint16_t* __restrict__ G16,
                                                   const float* __restrict__ Gz, const uint16_t* __restrict__ QT16,
                                                   const int32_t* __restrict__ labels, const float* __restrict__ lam,
                                                   const float* __restrict__ gam, int G, int Hq, int Hkv, int N,
                                                   int NB, float scale, float* __restrict__ dkl) {
  // group masks and per-dimension coefficients of all the unit's query heads
  // (up to 8), built once: no dependent label -> coefficient loads per head
  __shared__ __attribute__((aligned(16))) uint32_t mk[8][4][8][2][4];
  __shared__ float cfl[8][9][kD];
  __shared__ float red[2][16][64];
  int ch;
  const int u = unit_chunk_block(NB, ch);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t kbase = (size_t)u * N * kD;
  const size_t np = (size_t)NB * kC;
  const LocalTile t = local_tile(wv, tok0, N, row);
  f32x16 acc[2] = {f32x16{}, f32x16{}};

  for (int hh = 0; hh < R; ++hh) build_masks(mk[hh], labels, kh * R + hh, G, tid);
  {
    // the coefficient table with every load of a thread in flight together:
    // entries past R * 9 * 64 clamped (in bounds, unstored), the group index of
    // gam clamped and masked afterwards
    constexpr int kIt = (8 * 9 * kD + 191) / 192;
    const int ne = R * 9 * kD;
    int gd[kIt];
#pragma unroll
    for (int j = 0; j < kIt; ++j) {
      const int e = min(tid + 192 * j, ne - 1);
      const int hh = e / (9 * kD), d = e % kD;
      gd[j] = clamp_label(labels[(kh * R + hh) * kD + d], G);
    }
    float cv[kIt];
#pragma unroll
    for (int j = 0; j < kIt; ++j) {
      const int e = min(tid + 192 * j, ne - 1);
      const int hh = e / (9 * kD), h2 = (e / kD) % 9, h = kh * R + hh;
      cv[j] = h2 == 8 ? lam[(size_t)h * G + gd[j]] : gam[((size_t)h * G + gd[j]) * G + min(h2, G - 1)];
    }
#pragma unroll
    for (int j = 0; j < kIt; ++j) {
      const int e = tid + 192 * j;
      if (e < ne) {
        const int hh = e / (9 * kD), h2 = (e / kD) % 9, d = e % kD;
        cfl[hh][h2][d] = h2 == 8 ? scale * cv[j] : (h2 < G ? 2.f * scale * scale * cv[j] : 0.f);
      }
    }
  }
  __syncthreads();
  for (int hh = 0; hh < R; ++hh) {
    const int h = kh * R + hh, mb = hh;
    const size_t qbase = (size_t)(b * Hq + h) * N * kD;
    // ds[i][j] = g_i . v_j + gz_i on live (j <= i, i < N) entries
    f32x16 ds = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      ds = mfma32(row8(G16 + qbase + t.io + 16 * kk + 8 * s, t.iok), row8(v + kbase + t.jo + 16 * kk + 8 * s, t.jok),
                  ds);
    float dsv[16];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int i0 = 32 * t.it + 8 * a + 4 * s;
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) {
        const int i = i0 + vv;
        const float gzi = tok0 + i < N ? Gz[(size_t)(b * Hq + h) * N + tok0 + i] : 0.f;
        dsv[4 * a + vv] = (t.j <= i && tok0 + i < N) ? ds[4 * a + vv] + gzi : 0.f;
      }
    }
    bf16x8 qt[2][2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        qt[dt][tt] = *reinterpret_cast<const bf16x8*>(QT16 + ((size_t)(b * Hq + h) * (kD + 2) + 32 * dt + row) * np +
                                                       tok0 + 32 * t.it + 16 * tt + 8 * s);
    float cf[9][2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int h2 = 0; h2 < 9; ++h2) cf[h2][dt] = cfl[hh][h2][32 * dt + row];
#pragma unroll
    for (int h2 = 0; h2 < 9; ++h2) {
      float x[16];
      if (h2 < 8) {
        f32x16 sh = f32x16{};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          sh = mfma32(masked(row8(q + qbase + t.io + 16 * kk + 8 * s, t.iok), &mk[mb][kk][h2][s][0]),
                      row8(k + kbase + t.jo + 16 * kk + 8 * s, t.jok), sh);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = dsv[r] * sh[r];  // the scale of s_h is in cf
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = dsv[r];
      }
      const bf16x8 f0 = acc_kfrag(x, 0, s), f1 = acc_kfrag(x, 1, s);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        f32x16 p = mfma32(f0, qt[dt][0], f32x16{});
        p = mfma32(f1, qt[dt][1], p);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] = fmaf(cf[h2][dt], p[r], acc[dt][r]);
      }
    }
  }
  local_write(red, acc, t, l, row, tok0, N, kbase, dkl);
}

// dv[j][e] += sum_i kappa[i][j] g_i[e], summed over the unit's query heads in
// registers. kappa comes from the forward (k2_intra_fwd saves each tile pair's
// bf16 kappa as this product's K-major A fragments, 32 bytes per lane), so a
// head costs two fragment loads, four G^T loads and four matrix products.
__global__ __launch_bounds__(192, 2) void k2_local_dv(const uint16_t* __restrict__ kapf,
                                                   const uint16_t* __restrict__ GT16, int Hq, int Hkv, int N, int NB,
                                                   float* __restrict__ dvl) {
  __shared__ float red[2][16][64];
  int ch;
  const int u = unit_chunk_block(NB, ch);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const int tok0 = ch * kC;
  const size_t kbase = (size_t)u * N * kD;
  const size_t np = (size_t)NB * kC;
  const LocalTile t = local_tile(wv, tok0, N, row);
  f32x16 acc[2] = {f32x16{}, f32x16{}};
#pragma unroll 2
  for (int hh = 0; hh < R; ++hh) {
    const int h = kh * R + hh;
    const uint16_t* kp = kapf + ((((size_t)(b * Hq + h) * NB + ch) * 3 + wv) * 64 + l) * 16;
    const bf16x8 f0 = *reinterpret_cast<const bf16x8*>(kp), f1 = *reinterpret_cast<const bf16x8*>(kp + 8);
#pragma unroll
    for (int et = 0; et < 2; ++et) {
      const uint16_t* gt = GT16 + ((size_t)(b * Hq + h) * (kD + 2) + 32 * et + row) * np + tok0 + 32 * t.it + 8 * s;
      acc[et] = mfma32(f0, *reinterpret_cast<const bf16x8*>(gt), acc[et]);
      acc[et] = mfma32(f1, *reinterpret_cast<const bf16x8*>(gt + 16), acc[et]);
    }
  }
  local_write(red, acc, t, l, row, tok0, N, kbase, dvl);
}

template <typename T>
void launch_local_bwd(const LaunchGeom& g, const T* q, const T* k, const T* v, const LocalBwdArgs& a, bool need_dq,
                      bool need_dkv, unsigned parts, hipStream_t st, const Timer& timed) {
  // The coefficient partials come from the dq kernel's group sums, also when
  // dq itself is not requested (its dq then goes to the workspace unused), so
  // that every requested gradient is bit-identical whatever else is requested.
  // parts: kLocalDq (with the per-pair path's whole local VJP), kLocalDkv.
  if (a.pairwise && (parts & kLocalDq)) {
    launch_pair_local_bwd<T>(g, q, k, v, a, need_dq, need_dkv, st, timed);
  }
  const bool coef = a.coefl != nullptr;
  if (!a.pairwise && (need_dq || coef) && (parts & kLocalDq)) {
    timed("k2_local_dq", st, [&] {
      if (coef)
        hipLaunchKernelGGL((k2_local_dq<T, true>), dim3(g.R * g.NB * g.U), dim3(192), 0, st, q, k, v, a.G16, a.Gz,
                           a.KT16, a.PZ, a.PZm, a.labels, a.lam, a.gam, a.gm, a.lb, a.groups, g.Hq, g.Hkv, g.N, g.NB,
                           a.scale, a.dqf, a.coefl);
      else
        hipLaunchKernelGGL((k2_local_dq<T, false>), dim3(g.R * g.NB * g.U), dim3(192), 0, st, q, k, v, a.G16, a.Gz,
                           a.KT16, a.PZ, a.PZm, a.labels, a.lam, a.gam, a.gm, a.lb, a.groups, g.Hq, g.Hkv, g.N, g.NB,
                           a.scale, a.dqf, nullptr);
    });
  }
  if (!a.pairwise && need_dkv && (parts & kLocalDkv)) {
    timed("k2_local_dk", st, [&] {
      hipLaunchKernelGGL(k2_local_dk<T>, dim3(g.NB * g.U), dim3(192), 0, st, q, k, v, a.G16, a.Gz, a.QT16,
                         a.labels, a.lam, a.gam, a.groups, g.Hq, g.Hkv, g.N, g.NB, a.scale, a.dkl);
    });
  }
  if (need_dkv && (parts & kLocalDkv)) {
    timed("k2_local_dv", st, [&] {
      hipLaunchKernelGGL(k2_local_dv, dim3(g.NB * g.U), dim3(192), 0, st, a.KAP, a.GT16, g.Hq, g.Hkv, g.N, g.NB,
                         a.dvl);
    });
  }
}

template void launch_local_bwd<float>(const LaunchGeom&, const float*, const float*, const float*,
                                      const LocalBwdArgs&, bool, bool, unsigned, hipStream_t, const Timer&);
template void launch_local_bwd<uint16_t>(const LaunchGeom&, const uint16_t*, const uint16_t*, const uint16_t*,
                                         const LocalBwdArgs&, bool, bool, unsigned, hipStream_t, const Timer&);

}  // namespace oal
