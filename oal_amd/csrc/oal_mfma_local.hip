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
// k2_local_dk and k2_local_dv cover the 64x64 chunk with three lower 32x32
// tiles (key tile jt, query tile it) = (0,0), (0,1), (1,1); k2_local_dq covers
// its causal triangle with ten 16x16 sub-tiles. Group sums and ds come from
// the MFMA on row-major operands; their accumulators are fed straight back
// into the MFMA as the K-major operand of the dq / dk / dv products, whose
// other operand is the transposed bf16 copy of K, q or G.
//
// k2_local_dq    one block of two waves per (query head, chunk): dq local part
//                and the state part of the denominator's dq (gz_i (bz + 2 Mz
//                q_i)). With the coefficient gradients requested it also writes
//                the per-(head, chunk) coefficient partials from the same group
//                sums.
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
// dq local part + denominator-state dq on 16 x 16 sub-tiles, one block of two
// waves per (query head, chunk), grid R * NB * U (XCD-ordered). The chunk's
// causal lower triangle is 10 sub-tiles (key block jb <= query block ib, 16
// tokens each); wave 0 owns query blocks 3 and 0, wave 1 blocks 2 and 1 (five
// sub-tiles each), so each query row's dq is formed by one wave. Per sub-tile,
// on v_mfma_f32_16x16x32_bf16 (lane column = query i, rows = key j):
//   ds^T = V G^T (+ gz_i, j <= i), the eight group sums s'^T_g from masked key
//   fragments, the coefficient partials over the lane's four entries, and
//   dq[i][d] += coef_h(d) sum_j X_h[i][j] k_j[d], X_h = ds o s'_h (X_8 = ds),
//   on v_mfma_f32_16x16x16_bf16 with the 16 x 16 accumulator tile X_h as the
//   A operand as it stands (no exchange between lanes).
// Then, per query block, gz_i (bz_d + 2 (Mz q_i)_d), Mz = gm o PZm, and the
// dq rows. Against the 32 x 32 form: 10 sub-tiles instead of 12, and eight
// group-sum registers per lane instead of 128, so three blocks' worth of
// waves per SIMD fit. COEF: the partials ([0] sum ds, [1 + g] sum ds s_g,
// [9 + packed (g <= h)] sum ds s_g s_h), summed over each 16-lane row by DPP
// (fixed order), then over the block's eight rows in order.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}

template <typename T, bool COEF>
__global__ __launch_bounds__(128, 3) void k2_local_dq(const T* __restrict__ q, const T* __restrict__ k,
                                                       const T* __restrict__ v, const uint16_t* __restrict__ G16,
                                                       const float* __restrict__ Gz, const uint16_t* __restrict__ KT16,
                                                       const float* __restrict__ PZ, const float* __restrict__ PZm,
                                                       const int32_t* __restrict__ labels, const float* __restrict__ lam,
                                                       const float* __restrict__ gam, const float* __restrict__ gm,
                                                       const float* __restrict__ lb, int G, int Hq, int Hkv, int N,
                                                       int NB, float scale, float* __restrict__ dqf,
                                                       float* __restrict__ coefl) {
  constexpr int LD = kD + 8;
  // masks of the key fragments: [k-step][group][lane group][word], word w of
  // lane group lg covers dims 32 ks + 8 lg + 2 w, + 1
  __shared__ __attribute__((aligned(16))) uint32_t mk[2][8][4][4];
  __shared__ __attribute__((aligned(16))) uint16_t kts[kD][LD];  // k^T of the chunk
  __shared__ __attribute__((aligned(16))) __bf16 Mz[kD][LD];
  __shared__ float cft[9][kD];  // coef_h(d)
  __shared__ float bz[kD];
  __shared__ float gzs[kC];
  __shared__ float cp[COEF ? 8 : 1][45];  // row sums of the partials

  int hh, ch, u;
  head_chunk_unit(Hq / Hkv, NB, (int)(gridDim.x / ((Hq / Hkv) * NB)), hh, ch, u);
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv, h = kh * R + hh;
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, lr = l & 15, lg = l >> 4;
  const int tok0 = ch * kC;
  const size_t qbase = (size_t)(b * Hq + h) * N * kD;
  const size_t kbase = (size_t)u * N * kD;
  const size_t cbase = (size_t)u * NB + ch;
  const size_t np = (size_t)NB * kC;

  for (int e = tid; e < 256; e += 128) {
    const int ks = e >> 7, g = (e >> 4) & 7, lgm = (e >> 2) & 3, w = e & 3;
    const int d = 32 * ks + 8 * lgm + 2 * w;
    const int g0 = clamp_label(labels[h * kD + d], G), g1 = clamp_label(labels[h * kD + d + 1], G);
    mk[ks][g][lgm][w] = (g0 == g ? 0x0000ffffu : 0u) | (g1 == g ? 0xffff0000u : 0u);
  }
  for (int pc = tid; pc < 512; pc += 128) {
    const int d = pc >> 3, c = 8 * (pc & 7);
    *reinterpret_cast<bf16x8*>(&kts[d][c]) =
        *reinterpret_cast<const bf16x8*>(KT16 + ((size_t)u * kD + d) * np + tok0 + c);
    const float4* gp = reinterpret_cast<const float4*>(gm + ((size_t)h * kD + d) * kD + c);
    const float4* zp = reinterpret_cast<const float4*>(PZm + (cbase * kD + d) * kD + c);
    const float4 g0 = gp[0], g1 = gp[1], z0 = zp[0], z1 = zp[1];
    float y[8] = {g0.x * z0.x, g0.y * z0.y, g0.z * z0.z, g0.w * z0.w,
                  g1.x * z1.x, g1.y * z1.y, g1.z * z1.z, g1.w * z1.w};
    *reinterpret_cast<bf16x8*>(&Mz[d][c]) = pack8(y);
  }
  {
    const int d = l;
    const int cl = clamp_label(labels[h * kD + d], G);
    if (wv == 0) {
#pragma unroll
      for (int h2 = 0; h2 < 8; ++h2)
        cft[h2][d] = h2 < G ? 2.f * scale * scale * gam[((size_t)h * G + cl) * G + min(h2, G - 1)] : 0.f;
    } else {
      cft[8][d] = scale * lam[(size_t)h * G + cl];
      bz[d] = lb[(size_t)h * kD + d] * PZ[cbase * kFP + 1 + d];
      gzs[d] = tok0 + d < N ? Gz[(size_t)(b * Hq + h) * N + tok0 + d] : 0.f;
    }
  }
  __syncthreads();

  float ca[COEF ? 45 : 1];
#pragma unroll
  for (int e = 0; e < (COEF ? 45 : 1); ++e) ca[e] = 0.f;
#pragma unroll 1
  for (int bi = 0; bi < 2; ++bi) {
    const int ib = wv == 0 ? (bi == 0 ? 3 : 0) : (bi == 0 ? 2 : 1);
    const int il = 16 * ib + lr;  // this lane's query column (and its operand row)
    const int ir = tok0 + il;
    const bool iok = ir < N;
    const size_t io = (size_t)(iok ? ir : N - 1) * kD;
    bf16x8 qf[2], gf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qf[ks] = row8(q + qbase + io + 32 * ks + 8 * lg, iok);
      gf[ks] = row8(G16 + qbase + io + 32 * ks + 8 * lg, iok);
    }
    const float gzi = gzs[il];  // zero past N
    f32x4 dq[4] = {f32x4{}, f32x4{}, f32x4{}, f32x4{}};
#pragma unroll 1
    for (int jb = 0; jb <= ib; ++jb) {
      const int jr = tok0 + 16 * jb + lr;
      const bool jok = jr < N;
      const size_t jo = (size_t)(jok ? jr : N - 1) * kD;
      bf16x8 kf[2], vf[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        kf[ks] = row8(k + kbase + jo + 32 * ks + 8 * lg, jok);
        vf[ks] = row8(v + kbase + jo + 32 * ks + 8 * lg, jok);
      }
      // ds^T[j][i], j = 16 jb + 4 lg + r, i = il
      f32x4 ds = f32x4{};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) ds = mfma16(vf[ks], gf[ks], ds);
      float dsv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) dsv[r] = 16 * jb + 4 * lg + r <= il ? ds[r] + gzi : 0.f;
      f32x4 sg[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        sg[g] = f32x4{};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) sg[g] = mfma16(masked(kf[ks], &mk[ks][g][lg][0]), qf[ks], sg[g]);
      }
      if constexpr (COEF) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float tv[8];
#pragma unroll
          for (int g = 0; g < 8; ++g) tv[g] = dsv[r] * sg[g][r];
          ca[0] += dsv[r];
          int e = 9;
#pragma unroll
          for (int g = 0; g < 8; ++g) {
            ca[1 + g] += tv[g];
#pragma unroll
            for (int h2 = g; h2 < 8; ++h2) {
              ca[e] = fmaf(tv[g], sg[h2][r], ca[e]);
              ++e;
            }
          }
        }
      }
      // B operands k[j][d], j = 16 jb + 4 lg + (0..3), d = 16 db + lr
      s16x4 kb[4];
#pragma unroll
      for (int db = 0; db < 4; ++db) kb[db] = *reinterpret_cast<const s16x4*>(&kts[16 * db + lr][16 * jb + 4 * lg]);
#pragma unroll
      for (int h2 = 0; h2 < 9; ++h2) {
        float x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = h2 < 8 ? dsv[r] * sg[h2][r] : dsv[r];
        const s16x4 xa = pack4(x);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const f32x4 p = mfma16k16(xa, kb[db], f32x4{});
          const float cf = cft[h2][16 * db + lr];
#pragma unroll
          for (int r = 0; r < 4; ++r) dq[db][r] = fmaf(cf, p[r], dq[db][r]);
        }
        // one group's four products in flight at a time (the scheduler would
        // otherwise issue all 36 first and hold their results)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // denominator state: Z[i][d] = sum_e q_i[e] Mz[d][e], i = 16 ib + 4 lg + r
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      f32x4 z = f32x4{};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        z = mfma16(qf[ks], *reinterpret_cast<const bf16x8*>(&Mz[16 * db + lr][32 * ks + 8 * lg]), z);
      const float bzd = bz[16 * db + lr];
#pragma unroll
      for (int r = 0; r < 4; ++r) dq[db][r] = fmaf(gzs[16 * ib + 4 * lg + r], bzd + 2.f * z[r], dq[db][r]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = tok0 + 16 * ib + 4 * lg + r;
      if (tok < N) {
#pragma unroll
        for (int db = 0; db < 4; ++db) dqf[qbase + (size_t)tok * kD + 16 * db + lr] = dq[db][r];
      }
    }
  }
  if constexpr (COEF) {
    // sums over each 16-lane row (quad pairs, then quads, then half rows)
#pragma unroll
    for (int e = 0; e < 45; ++e) {
      float x = ca[e];
      x = dpp_add<0xB1>(x);   // quad_perm [1, 0, 3, 2]
      x = dpp_add<0x4E>(x);   // quad_perm [2, 3, 0, 1]
      x = dpp_add<0x124>(x);  // row_ror:4
      x = dpp_add<0x128>(x);  // row_ror:8
      ca[e] = x;
    }
    if (lr == 0) {
#pragma unroll
      for (int e = 0; e < 45; ++e) cp[4 * wv + lg][e] = ca[e];
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
      float x = 0.f;
#pragma unroll
      for (int rw = 0; rw < 8; ++rw) x += cp[rw][e];
      const float sc = e == 0 ? 1.f : e < 9 ? scale : scale * scale;
      const size_t bn = (size_t)(gridDim.x / (R * NB) / Hkv) * NB;
      coefl[((size_t)h * 73 + tid) * bn + (size_t)b * NB + ch] = x * sc;
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
bool launch_local_bwd(const LaunchGeom& g, const T* q, const T* k, const T* v, const LocalBwdArgs& a, bool need_dq,
                      bool need_dkv, unsigned parts, hipStream_t st, const Timer& timed, hipEvent_t stop) {
  // The coefficient partials come from the dq kernel's group sums, also when
  // dq itself is not requested (its dq then goes to the workspace unused), so
  // that every requested gradient is bit-identical whatever else is requested.
  // parts: kLocalDq (with the per-pair path's whole local VJP), kLocalDk,
  // kLocalDv.
  if (a.pairwise && (parts & kLocalDq)) {
    launch_pair_local_bwd<T>(g, q, k, v, a, need_dq, need_dkv, st, timed);
  }
  const bool coef = a.coefl != nullptr;
  // the one kernel of a single-part call records stop
  hipEvent_t stop_dq = parts == kLocalDq ? stop : nullptr, stop_dk = parts == kLocalDk ? stop : nullptr,
             stop_dv = parts == kLocalDv ? stop : nullptr;
  bool signalled = false;
  if (!a.pairwise && (need_dq || coef) && (parts & kLocalDq)) {
    timed("k2_local_dq", st, [&] {
      if (coef)
        launch_signal(k2_local_dq<T, true>, dim3(g.R * g.NB * g.U), dim3(128), st, stop_dq, q, k, v, a.G16, a.Gz,
                      a.KT16, a.PZ, a.PZm, a.labels, a.lam, a.gam, a.gm, a.lb, a.groups, g.Hq, g.Hkv, g.N, g.NB,
                      a.scale, a.dqf, a.coefl);
      else
        launch_signal(k2_local_dq<T, false>, dim3(g.R * g.NB * g.U), dim3(128), st, stop_dq, q, k, v, a.G16, a.Gz,
                      a.KT16, a.PZ, a.PZm, a.labels, a.lam, a.gam, a.gm, a.lb, a.groups, g.Hq, g.Hkv, g.N, g.NB,
                      a.scale, a.dqf, static_cast<float*>(nullptr));
    });
    signalled = stop_dq != nullptr;
  }
  if (!a.pairwise && need_dkv && (parts & kLocalDk)) {
    timed("k2_local_dk", st, [&] {
      launch_signal(k2_local_dk<T>, dim3(g.NB * g.U), dim3(192), st, stop_dk, q, k, v, a.G16, a.Gz, a.QT16,
                    a.labels, a.lam, a.gam, a.groups, g.Hq, g.Hkv, g.N, g.NB, a.scale, a.dkl);
    });
    signalled = stop_dk != nullptr;
  }
  if (need_dkv && (parts & kLocalDv)) {
    timed("k2_local_dv", st, [&] {
      launch_signal(k2_local_dv, dim3(g.NB * g.U), dim3(192), st, stop_dv, a.KAP, a.GT16, g.Hq, g.Hkv, g.N, g.NB,
                    a.dvl);
    });
    signalled = stop_dv != nullptr;
  }
  return signalled;
}

template bool launch_local_bwd<float>(const LaunchGeom&, const float*, const float*, const float*,
                                      const LocalBwdArgs&, bool, bool, unsigned, hipStream_t, const Timer&,
                                      hipEvent_t);
template bool launch_local_bwd<uint16_t>(const LaunchGeom&, const uint16_t*, const uint16_t*, const uint16_t*,
                                         const LocalBwdArgs&, bool, bool, unsigned, hipStream_t, const Timer&,
                                         hipEvent_t);

}  // namespace oal
