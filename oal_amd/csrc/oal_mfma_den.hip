// Denominator state of the chunked scan in pair-matrix form: the forward
// prefix of the per-chunk totals k2_fwd_prep leaves (K^T K, sum k, token
// count), the backward per-chunk totals over the query heads of a unit with
// their coefficient partials, and the backward suffix. Kept apart from the
// state scans: the denominator column is a symmetric 64 x 64 matrix per chunk,
// formed and scanned here directly instead of as a 65th value column of the
// 2208-slot state.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"

namespace oal {

// ---------------------------------------------------------------------------
// Denominator state in pair-matrix form. Chunk totals Zt / dCt [U][NB][kZt]:
// [r * 64 + c] the pair entry (r, c) of a symmetric 64 x 64 matrix, [4096 + d]
// the linear entry d, [4160] the constant entry (backward only; the forward's
// constant total of a chunk before the last is its 64 tokens).
// k2_den_scan<FWD>: the forward writes the exclusive prefix PZ [U][NB][kFP]
// (natural feature order) and PZm [U][NB][64][64] (the pair matrix), the
// backward the exclusive suffix dTz [U][NB][kFP]. The summation order is fixed
// (per 64-chunk tile: four 16-chunk row sums, then the walk), so results do
// not depend on the launch.
// ---------------------------------------------------------------------------
// Entry e of a chunk total: its natural feature index (-1 for a pair entry
// above the diagonal, which the natural order does not hold).
__device__ __forceinline__ int den_entry_nat(int e) {
  if (e < kD * kD) {
    const int r = e >> 6, c = e & 63;
    return r >= c ? 1 + kD + pair_index(r, c) : -1;
  }
  return e < kD * kD + kD ? 1 + (e - kD * kD) : 0;
}

// Block (64 entries, unit), 256 threads: tiles of 64 chunks x 64 entries are
// loaded into LDS with coalesced row loads; each wave then walks 16 of the
// tile's chunks in order from the running sum plus the earlier waves' row
// sums, one thread per entry, each chunk's stores coalesced across the wave.
template <bool FWD>
__global__ __launch_bounds__(256) void k2_den_scan(const float* __restrict__ tot, int NB, float* __restrict__ outZ,
                                                   float* __restrict__ outZm) {
  constexpr int kEntries = kD * kD + kD + 1;
  __shared__ float tile[64][65];
  __shared__ float psum[4][64];
  const int u = blockIdx.y, e0 = blockIdx.x * 64, tid = threadIdx.x;
  const int e = e0 + (tid & 63);  // every wave: the same 64 entries
  const int nat = den_entry_nat(e);
  float run = 0.f;
  for (int t0 = 0; t0 < NB; t0 += 64) {
    const int nt = min(64, NB - t0);
    __syncthreads();
    // row i of the tile = the i-th chunk in scan order; all 16 loads of a
    // thread in flight together (rows past the tile reload its last row, unread;
    // entries past kEntries read the padding of the row, unread)
    float x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = min((tid >> 6) + 4 * j, nt - 1);
      const int ch = FWD ? t0 + i : NB - 1 - (t0 + i);
      x[j] = tot[((size_t)u * NB + ch) * kZt + min(e, kZt - 1)];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) tile[(tid >> 6) + 4 * j][tid & 63] = x[j];
    __syncthreads();
    // two-level prefix over the tile: wave q walks tile rows 16 q .. 16 q + 15
    // from run plus the row sums of the waves before it
    const int q = tid >> 6, lane = tid & 63;
    const bool cnst = FWD && nat == 0;  // the forward's constant: 64 tokens per chunk
    float wsum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) wsum += (16 * q + i < nt) ? (cnst ? (float)kC : tile[16 * q + i][lane]) : 0.f;
    psum[q][lane] = wsum;
    __syncthreads();
    float start = run;
    for (int p2 = 0; p2 < q; ++p2) start += psum[p2][lane];
    if (e < kEntries) {
      for (int i = 16 * q; i < min(16 * q + 16, nt); ++i) {
        const int ch = FWD ? t0 + i : NB - 1 - (t0 + i);
        const size_t cb = (size_t)u * NB + ch;
        if (nat >= 0) outZ[cb * kFP + nat] = start;
        if constexpr (FWD) {
          if (e < kD * kD) outZm[cb * kD * kD + e] = start;
        }
        start += cnst ? (float)kC : tile[i][lane];
      }
    }
    run += (psum[0][lane] + psum[1][lane]) + (psum[2][lane] + psum[3][lane]);
  }
}

// ---------------------------------------------------------------------------
// Backward denominator state, one block per (unit, chunk), 4 waves. Per query
// head h of the unit: H_h = sum_j gz_j [1, q_j] [1, q_j]^T over the chunk
// (waves 0-2: the pair blocks (0,0), (1,0), (1,1) of Q^T diag(gz) Q on the
// matrix cores; wave 3: the linear entries sum_j gz_j q_j[d] and the constant
// sum_j gz_j, as products with the gz row). The chunk total
//   dCt[entry] = sum_h wq_h[entry] H_h[entry]
// (wq of a pair = (r == c ? 1 : 2) gm[r][c], of a linear entry lb[d], of the
// constant c0) feeds k2_den_scan<false>; the per-head coefficient partial
//   dwz[u][c][h][nat] = PZ_c[nat] H_h[nat]
// (natural order, every nat < kFeat) is summed over (batch, chunk) by
// k2_dwq_reduce (dwz == nullptr: not formed). QT16 / GT16 are the transposed bf16 operands of the backward
// scan ([q^T; 1; 0] and [G^T; Gz; 0], tokens >= N zero).
// ---------------------------------------------------------------------------
constexpr int kDenHeads = 8;  // query heads staged in LDS per batch

__global__ __launch_bounds__(256, 2) void k2_den_bwd(const uint16_t* __restrict__ QT16, const uint16_t* __restrict__ GT16,
                                                  int trows, const float* __restrict__ gm, const float* __restrict__ lb,
                                                  const float* __restrict__ ic, int kic, const float* __restrict__ PZ,
                                                  const float* __restrict__ PZm, int Hq, int Hkv, int NB,
                                                  float* __restrict__ dCt, float* __restrict__ dwz) {
  // q^T rows 0..63 of the chunk per staged head, 128-byte rows of eight
  // 16-byte token slots, slot (k8 ^ (row & 7)) holding tokens 8 k8 ..; the gz
  // rows of the staged heads unswizzled
  __shared__ __align__(16) uint16_t qs[kDenHeads][kD][kC];
  __shared__ __align__(16) uint16_t gs[kDenHeads][kC];
  const int u = blockIdx.x / NB, ch = blockIdx.x % NB;
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  const size_t np = (size_t)NB * kC;
  const size_t cb = (size_t)u * NB + ch;
  const int mr = w == 0 ? 0 : 1, mc = w == 2 ? 1 : 0;
  // waves 0-2: dCt of the wave's pair block; wave 3: linear d = row, 32 + row
  // and the constant (lanes with s = 0)
  f32x16 dc = f32x16{};
  float dl1 = 0.f, dl2 = 0.f;
  float pz[16];
  if (w < 3) {
#pragma unroll
    for (int i = 0; i < 16; ++i) pz[i] = PZm[cb * kD * kD + (32 * mr + c32_row(i, l)) * kD + 32 * mc + row];
  } else {
    // register n of lane (row, s = 0): linear d = 32 n + row (n < 2), constant (n = 2, row 0)
#pragma unroll
    for (int n = 0; n < 3; ++n) pz[n] = n < 2 ? PZ[cb * kFP + 1 + 32 * n + row] : PZ[cb * kFP];
  }
  // weights of query head h: pair gm of the wave's block (wave 3: of block
  // (1, 0), unused), linear lb of d = row, 32 + row and the constant c0, loaded
  // by every wave without branches (a branch would put the arrays on the stack)
  auto load_w = [&](int h, float (&wv)[16], float (&wl)[3]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 32 * mr + c32_row(i, l), c = 32 * mc + row;
      wv[i] = gm[((size_t)h * kD + r) * kD + c];
    }
    wl[0] = lb[(size_t)h * kD + row];
    wl[1] = lb[(size_t)h * kD + 32 + row];
    wl[2] = ic[(size_t)h * kic];
  };
  // LDS byte offset of q^T row r, tokens 16 kk + 8 s .. of staged head hl
  auto qoff = [&](int hl, int r, int kk) { return ((hl * kD + r) * 8 + ((2 * kk + s) ^ (r & 7))) * 16; };
  const char* qsb = reinterpret_cast<const char*>(&qs[0][0][0]);
  for (int h0 = 0; h0 < R; h0 += kDenHeads) {
    const int nb = min(kDenHeads, R - h0);
    float wcur[16], lcur[3];
    load_w(kh * R + h0, wcur, lcur);
    __syncthreads();
    // each wave copies 8 rows (1 KiB) per call: lane l -> row 8 j + l / 8, slot
    // l % 8 = k8 ^ (l / 8); heads past the batch reload its last head (never read)
#pragma unroll
    for (int j = 0; j < kDenHeads * kD / 8 / 4; ++j) {
      const int jj = 4 * j + w, hl = min(jj >> 3, nb - 1), r = 8 * (jj & 7) + (l >> 3);
      const int k8 = (l & 7) ^ (l >> 3);
      const uint16_t* src = QT16 + ((size_t)(b * Hq + kh * R + h0 + hl) * trows + r) * np + (size_t)ch * kC + 8 * k8;
      copy16_to_lds(src, &qs[jj >> 3][8 * (jj & 7)][0]);
    }
    if (w == 0) {
      const int hl = min(l >> 3, nb - 1);
      const uint16_t* src = GT16 + ((size_t)(b * Hq + kh * R + h0 + hl) * trows + kD) * np + (size_t)ch * kC + 8 * (l & 7);
      copy16_to_lds(src, &gs[0][0]);
    }
    wait_vmcnt<0>();
    __syncthreads();
#pragma unroll 1
    for (int hl = 0; hl < nb; ++hl) {
      const int hh = h0 + hl, h = kh * R + hh;
      float wnext[16], lnext[3];
      load_w(kh * R + h0 + min(hl + 1, nb - 1), wnext, lnext);
      float* part = dwz + (cb * R + hh) * kFP;  // offsets below are unsigned 32-bit
      if (w < 3) {
        f32x16 H = f32x16{};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(qsb + qoff(hl, 32 * mr + row, kk));
          const bf16x8 qc = *reinterpret_cast<const bf16x8*>(qsb + qoff(hl, 32 * mc + row, kk));
          const bf16x8 gz = *reinterpret_cast<const bf16x8*>(&gs[hl][16 * kk + 8 * s]);
          float y[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = (float)qc[j] * (float)gz[j];
          H = mfma32(a, pack8(y), H);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = 32 * mr + c32_row(i, l), c = 32 * mc + row;
          dc[i] = fmaf((r == c ? 1.f : 2.f) * wcur[i], H[i], dc[i]);
          if (dwz && r >= c) part[(unsigned)(1 + kD + pair_index(r, c))] = pz[i] * H[i];
        }
      } else {
        // A row 0 = gz (other rows zero); B = q^T rows 32 n + row (n < 2) or,
        // for n = 2, ones in column 0 (gz is zero past the sequence end)
        f32x16 L[3];
#pragma unroll
        for (int n = 0; n < 3; ++n) L[n] = f32x16{};
        bf16x8 ones;
#pragma unroll
        for (int j = 0; j < 8; ++j) ones[j] = row == 0 ? (__bf16)1.f : (__bf16)0.f;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 gz = *reinterpret_cast<const bf16x8*>(&gs[hl][16 * kk + 8 * s]);
          const bf16x8 a = row == 0 ? gz : bf16x8{};
#pragma unroll
          for (int n = 0; n < 2; ++n)
            L[n] = mfma32(a, *reinterpret_cast<const bf16x8*>(qsb + qoff(hl, 32 * n + row, kk)), L[n]);
          L[2] = mfma32(a, ones, L[2]);
        }
        if (s == 0) {
          if (dwz) {
#pragma unroll
            for (int n = 0; n < 2; ++n) part[1 + 32 * n + row] = pz[n] * L[n][0];
          }
          dc[0] = fmaf(lcur[0], L[0][0], dc[0]);
          dl1 = fmaf(lcur[1], L[1][0], dl1);
          if (row == 0) {
            dl2 = fmaf(lcur[2], L[2][0], dl2);
            if (dwz) part[0] = pz[2] * L[2][0];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) wcur[i] = wnext[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) lcur[i] = lnext[i];
      (void)h;
    }
  }
  float* z = dCt + cb * kZt;
  if (w < 3) {
#pragma unroll
    for (int i = 0; i < 16; ++i) z[(32 * mr + c32_row(i, l)) * kD + 32 * mc + row] = dc[i];
  } else if (s == 0) {
    z[kD * kD + row] = dc[0];
    z[kD * kD + 32 + row] = dl1;
    if (row == 0) z[kD * kD + kD] = dl2;
  }
}

void launch_den_scan(bool fwd, const LaunchGeom& g, const float* tot, float* outZ, float* outZm, hipStream_t st,
                     const Timer& timed) {
  const dim3 grid((kD * kD + kD + 1 + 63) / 64, g.U);
  timed(fwd ? "k2_den_fwd_scan" : "k2_den_bwd_scan", st, [&] {
    if (fwd)
      hipLaunchKernelGGL(k2_den_scan<true>, grid, dim3(256), 0, st, tot, g.NB, outZ, outZm);
    else
      hipLaunchKernelGGL(k2_den_scan<false>, grid, dim3(256), 0, st, tot, g.NB, outZ, nullptr);
  });
}

void launch_den_bwd(const LaunchGeom& g, const uint16_t* QT16, const uint16_t* GT16, int trows, const float* gm,
                    const float* lb, const float* ic, int kic, const float* PZ, const float* PZm, float* dCt,
                    float* dwz, hipStream_t st, const Timer& timed) {
  timed("k2_den_bwd", st, [&] {
    hipLaunchKernelGGL(k2_den_bwd, dim3(g.U * g.NB), dim3(256), 0, st, QT16, GT16, trows, gm, lb, ic, kic, PZ, PZm,
                       g.Hq, g.Hkv, g.NB, dCt, dwz);
  });
}

}  // namespace oal
