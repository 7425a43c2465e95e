// Chunk-state scans on the gfx950 matrix cores, forward and backward.
//
// Forward (reference hd_block_gemm_runtime.py:271-320: block totals, exclusive
// cumsum), per unit u = (batch, kv head):
//   T_c = raw(K_c)^T V_c,        P_c = sum_{c' < c} T_c'
// Backward (reference hd_block_gemm_backward.py:764-908: _query_dcarry and the
// exclusive right scan), per unit:
//   dCarry_c = sum_h wq_h o raw(Q_h,c)^T G_h,c,   dT_c = sum_{c' > c} dCarry_c'
// and the per-slot coefficient partial of each query head
//   dwq_h[slot] += sum_c <P_c[slot], (raw(Q_h,c)^T G_h,c)[slot]>.
// The denominator column (the value-side row of ones / of Gz) is not in these
// scans: its feature-space state is the 64 x 64 pair matrix of the k2_den_*
// kernels below, formed with one small product per chunk instead of a
// 1/32-useful matrix-core column per k-step.
//
// k2_scan<FWD, MODE, TPW, NW>: a block of NW waves, each owning TPW 32-slot
// tiles, of one unit and one segment of consecutive chunks; the state of a
// tile lives in MFMA accumulators laid out value x slot (lane column = slot).
// The value side of an item is read from LDS once per wave and feeds all of
// the wave's tiles (TPW = 2 halves those reads per tile; the backward totals
// keep TPW = 1 for the registers of the per-head products). An item is one
// (chunk, query head) pair in the backward and one chunk in the forward; its
// operands (the feature side q^T / k^T and the value side G^T / V^T, 64
// tokens each) are staged once per block into a double-buffered LDS pair,
// fetched into registers two items ahead. Raw features are products of two
// fp32 rows of the staged feature side, packed to bf16 as the MFMA B operand.
//   MODE 0: segment totals (backward: plus coefficient partials); no state out.
//   MODE 1: replay from the carry of the other segments (the sum of their totals,
//           nearest segment first, formed by each block for its own tiles),
//           emitting every chunk's state; the backward weights the features by
//           wq_h so that every head accumulates into the one state.
//   MODE 2: one segment: MODE 1's output plus MODE 0's partials.
//   MODE 3 (backward): one pass per segment from a zero carry: emits each
//           chunk's segment-local suffix state, forms MODE 0's partials and
//           writes the segment total. The state a consumer needs is that local
//           state plus the segment's carry (MODE 4); the only consumer of the
//           backward state, k2_kv_fold, adds the carry with matrix products of
//           its own, so the backward contracts every item once.
//   MODE 4 (backward): the carry of each segment, the sum of the totals of the
//           segments after it, emitted once per (unit, segment); no items. A block walks its tiles' segments from the last
//           one backwards with a running sum, so each total is read once.
// PART (backward, MODE 0 and 2): form the coefficient partials; without them
// (no coefficient gradient requested) the forward state is not read. The
// per-head products stay apart either way, so that the state -- and every
// gradient -- is bit-identical whichever gradients are requested.
// Emitted layout per (unit, chunk), identical in both directions:
//   R [kS/32][4][32][16 values] bf16. Readers that contract over the slots
//   stage a k-step's four 512-byte pieces and read their fragments transposed
//   (ds_read_b64_tr_b16), so no second, slot-contiguous copy is written.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>

#include "oal_internal.hpp"
#include "oal_mfma_common.hpp"
#include "oal_slot_coef.hpp"

namespace oal {

static __constant__ SlotTable kSlot = make_slot_table();

namespace {

// tile groups of a scan whose NW waves own TPW tiles each
constexpr int scan_tile_groups(int tpw, int nw) { return (kS / 32 + nw * tpw - 1) / (nw * tpw); }
constexpr int kFRow = kC + 4;                              // fp32 LDS row stride, feature side
constexpr int kVRow = kC + 8;                              // bf16 LDS row stride, value side
constexpr int kOpRows = kD + 2;                            // feature side rows 64 (one), 65 (zero)
constexpr size_t kChunkElems = (size_t)kKS * 64 * 16;

}  // namespace

template <bool FWD, int MODE, int TPW, int NW, bool PART>
__global__ __launch_bounds__(64 * NW, (NW + 1) / 2) void k2_scan(const uint16_t* __restrict__ F, int frows,
                                               const uint16_t* __restrict__ V, int vrows,
                                               const float* __restrict__ wqs, const uint16_t* __restrict__ PRin,
                                               const float* __restrict__ carry, int Hq, int Hkv, int N, int NB, int SL,
                                               int Sg, uint16_t* __restrict__ outR,
                                               float* __restrict__ segtot, float* __restrict__ dwqs) {
  constexpr bool EMIT = MODE == 1 || MODE == 2 || MODE == 3;
  // per-head products kept apart (needed for the partials)
  constexpr bool SPLIT = !FWD && (MODE == 0 || MODE == 2 || MODE == 3);
  constexpr bool PARTIALS = SPLIT && PART;
  static_assert(!SPLIT || TPW == 1, "the per-head products fit registers for one tile per wave");
  constexpr int TG = scan_tile_groups(TPW, NW);
  constexpr int kSTiles = NW;                // slot tiles (waves) per block
  constexpr int kNT = 64 * NW;               // threads per block
  constexpr int kFPT = kD * 8 / kNT;         // 16-byte operand chunks per thread and side
  static_assert(kFPT * kNT == kD * 8, "a block stages whole operand rows");
  // (MODE 4 stages no operands)
  __shared__ __attribute__((aligned(16))) float Fs[MODE == 4 ? 1 : 2][MODE == 4 ? 1 : kOpRows * kFRow];
  __shared__ __attribute__((aligned(16))) __bf16 Vs[MODE == 4 ? 1 : 2][MODE == 4 ? 1 : kD * kVRow];
  __shared__ float dwl[PARTIALS ? 8 : 1][kSTiles * 32];
  // backward: the slot weight wq_h of every query head of the unit (up to 8)
  // for the block's slots, [head][wave][tile][slot row]
  __shared__ float wsl[FWD ? 1 : 8][kSTiles * TPW * 32];

  int u, seg, tgi;
  {
    const int total = gridDim.x, id = blockIdx.x;
    const int w = (total & 7) == 0 ? (id & 7) * (total >> 3) + (id >> 3) : id;
    const int sg = MODE == 4 ? 1 : Sg;  // MODE 4: one block walks every segment
    tgi = w % TG;
    seg = (w / TG) % sg;
    u = w / (TG * sg);
  }
  const int R = Hq / Hkv, b = u / Hkv, kh = u % Hkv;
  const int RI = FWD ? 1 : R;  // items per chunk
  const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31;
  // this wave's tiles (TPW consecutive), their slots and slot rows
  int tile[TPW], slot[TPW], ar[TPW], ac[TPW];
  bool live[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    tile[t] = (kSTiles * tgi + wv) * TPW + t;
    live[t] = tile[t] < kS / 32;
    slot[t] = live[t] ? tile[t] * 32 + row : 0;
    ar[t] = kSlot.ar[slot[t]];
    ac[t] = kSlot.ac[slot[t]];
  }
  const bool any_live = live[0];
  const int c_lo = seg * SL, c_hi = min(NB, c_lo + SL);
  const int NI = c_hi > c_lo ? (c_hi - c_lo) * RI : 0;
  const size_t np = (size_t)NB * kC;

  // constant rows of the feature side: 64 = 1 (the value side is zero for
  // tokens >= N), 65 = 0
  if constexpr (MODE != 4) {
    for (int i = tid; i < 2 * kC; i += kNT) {
      const int bi = i / kC, j = i % kC;
      Fs[bi][kD * kFRow + j] = 1.f;
      Fs[bi][(kD + 1) * kFRow + j] = 0.f;
    }
  }
  if constexpr (PARTIALS) {
    for (int i = tid; i < 8 * kSTiles * 32; i += kNT) dwl[i / (kSTiles * 32)][i % (kSTiles * 32)] = 0.f;
  }

  // acc[t][n]: values 32 n .. 32 n + 31 of tile t
  f32x16 acc[TPW][2];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int n = 0; n < 2; ++n) acc[t][n] = f32x16{};
  if constexpr (MODE == 1) {
    // carry = sum of the totals of the segments before (forward) or after
    // (backward) this one, in a fixed order: nearest segment first
    // (the accumulator registers 4 a .. 4 a + 3 of a lane hold four consecutive
    // values of its slot, read as one 16-byte load; all loads of a segment are
    // issued before they are added)
    const int n_other = FWD ? seg : Sg - 1 - seg;
    for (int o = 0; o < n_other; ++o) {
      const int so = FWD ? seg - 1 - o : seg + 1 + o;
      float4 tv[TPW][2][4];
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float* cr = carry + (((size_t)u * Sg + so) * kS + slot[t]) * kD;
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
          for (int a = 0; a < 4; ++a)
            tv[t][n][a] = *reinterpret_cast<const float4*>(cr + 32 * n + c32_row(4 * a, l));
      }
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        if (live[t]) {
#pragma unroll
          for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
              acc[t][n][4 * a] += tv[t][n][a].x;
              acc[t][n][4 * a + 1] += tv[t][n][a].y;
              acc[t][n][4 * a + 2] += tv[t][n][a].z;
              acc[t][n][4 * a + 3] += tv[t][n][a].w;
            }
        }
      }
    }
  }

  // it / RI as a multiply-high by ceil(2^32 / RI) (exact for RI in 2..8 and
  // it < 2^20, far above any item count), instead of a runtime division
  const uint32_t rmagic = RI > 1 ? 0xFFFFFFFFu / (uint32_t)RI + 1u : 0u;
  auto item_chunk = [&](int it, int& ch, int& hh) {
    const int ci = RI > 1 ? (int)__umulhi((uint32_t)it, rmagic) : it;
    hh = it - ci * RI;
    ch = FWD ? c_lo + ci : c_hi - 1 - ci;
  };
  struct Stage {
    uint4 f[kFPT], v[kFPT];
  };
  // thread tid stages 16-byte chunks tid + kNT i (row chunk >> 3, column 8 (chunk & 7))
  auto uoff = [&](int i) { return (size_t)((tid + kNT * i) >> 3) * np + 8 * (tid & 7); };
  // Every thread issues the same loads on every call (items past the end are
  // clamped to the last one, the row-64 unit to an in-range column): the
  // compiler then counts the loads in flight exactly and waits for an item's
  // loads only where they are stored, keeping the next item's loads in flight.
  auto load = [&](Stage& st, int it) {
    int ch, hh;
    item_chunk(it < NI ? it : NI - 1, ch, hh);
    const int x = FWD ? u : b * Hq + kh * R + hh;
    const uint16_t* fb = F + (size_t)x * frows * np + (size_t)ch * kC;
    const uint16_t* vb = V + (size_t)x * vrows * np + (size_t)ch * kC;
#pragma unroll
    for (int i = 0; i < kFPT; ++i) {
      st.f[i] = *reinterpret_cast<const uint4*>(fb + uoff(i));
      st.v[i] = *reinterpret_cast<const uint4*>(vb + uoff(i));
    }
  };
  auto put = [&](int bi, int idx, const uint4& f) {
    float4* d = reinterpret_cast<float4*>(&Fs[bi][(idx >> 3) * kFRow + 8 * (idx & 7)]);
    d[0] = make_float4(__uint_as_float(f.x << 16), __uint_as_float(f.x & 0xffff0000u), __uint_as_float(f.y << 16),
                       __uint_as_float(f.y & 0xffff0000u));
    d[1] = make_float4(__uint_as_float(f.z << 16), __uint_as_float(f.z & 0xffff0000u), __uint_as_float(f.w << 16),
                       __uint_as_float(f.w & 0xffff0000u));
  };
  auto store = [&](int bi, const Stage& st) {
#pragma unroll
    for (int i = 0; i < kFPT; ++i) {
      const int idx = tid + kNT * i;
      put(bi, idx, st.f[i]);
      *reinterpret_cast<uint4*>(&Vs[bi][(idx >> 3) * kVRow + 8 * (idx & 7)]) = st.v[i];
    }
  };

  // Emission of tile t's state into state block cb (unit u and chunk ch: the
  // exclusive prefix / suffix before ch, cb = u * NB + ch; MODE 4: the carry of
  // segment seg, cb = u * Sg + seg).
  // A lane holds 4-value words at positions 4 s (word "even") and 8 + 4 s
  // (word "odd") of a 16-position row; swapping the odd words of lane group 0
  // with the even words of lane group 1 gives lane group s positions
  // 8 s .. 8 s + 7, stored as one 16-byte piece (the 64 lanes then write 32
  // consecutive rows, 1 KiB).
  auto store_row16 = [&](uint16_t* rowp, uint2 ev, uint2 od) {
    const auto x = __builtin_amdgcn_permlane32_swap(ev.x, od.x, false, false);
    const auto y = __builtin_amdgcn_permlane32_swap(ev.y, od.y, false, false);
    // lanes 0-31: (own even, group 1's even); lanes 32-63: (group 0's odd, own odd)
    *reinterpret_cast<uint4*>(rowp + 8 * s) = make_uint4(x[0], y[0], x[1], y[1]);
  };
  auto emit = [&](int t, size_t cb) {
    // R layout straight from the accumulators: lane = slot, 4 values a word pair
    uint32_t wd[2][4][2];
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        wd[n][a][0] = pack_bf16x2(acc[t][n][4 * a], acc[t][n][4 * a + 1]);
        wd[n][a][1] = pack_bf16x2(acc[t][n][4 * a + 2], acc[t][n][4 * a + 3]);
      }
    uint16_t* tr = outR + cb * kChunkElems + (size_t)tile[t] * 4 * 32 * 16;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int a = 0; a < 4; a += 2) {
        const int kk = 2 * n + (a >> 1);
        store_row16(tr + ((size_t)kk * 32 + row) * 16, make_uint2(wd[n][a][0], wd[n][a][1]),
                    make_uint2(wd[n][a + 1][0], wd[n][a + 1][1]));
      }
  };

  if constexpr (MODE == 4) {
    // carry of segment so = running sum of the totals of segments > so (added
    // from the last segment backwards); the next total's loads are issued
    // before the current carry is emitted
    float4 tv[TPW][2][4];
    auto load_total = [&](int so) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float* cr = carry + (((size_t)u * Sg + so) * kS + slot[t]) * kD;
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
          for (int a = 0; a < 4; ++a)
            tv[t][n][a] = *reinterpret_cast<const float4*>(cr + 32 * n + c32_row(4 * a, l));
      }
    };
    load_total(Sg - 1);
    for (int so = Sg - 1; so >= 0; --so) {
#pragma unroll
      for (int t = 0; t < TPW; ++t)
        if (live[t]) emit(t, (size_t)u * Sg + so);
      if (so == 0) break;
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            acc[t][n][4 * a] += tv[t][n][a].x;
            acc[t][n][4 * a + 1] += tv[t][n][a].y;
            acc[t][n][4 * a + 2] += tv[t][n][a].z;
            acc[t][n][4 * a + 3] += tv[t][n][a].w;
          }
      load_total(so - 1);
    }
    return;
  }

  // Coefficient partials: the P_c rows of this lane's slot (values
  // e = 32 n + 8 a + 4 s + v) for the chunk being processed (pf) and, still
  // packed, for the next chunk (pfn): the next chunk's loads are issued a whole
  // chunk of items before their use.
  float pf[2][16];
  uint2 pfn[2][4];
  auto fetch_partial_rows = [&](int ch) {
    const size_t cb = (size_t)u * NB + ch;
    const uint16_t* pr = PRin + cb * kChunkElems + (size_t)tile[0] * 4 * 32 * 16;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int kk = 2 * n + (a >> 1), pos = 8 * (a & 1) + 4 * s;
        pfn[n][a] = *reinterpret_cast<const uint2*>(pr + ((size_t)kk * 32 + row) * 16 + pos);
      }
  };
  if constexpr (PARTIALS) {
    if (NI > 0 && any_live) fetch_partial_rows(c_hi - 1);
  }
  // One item from LDS buffer bi.
  auto process = [&](int it, int bi) {
    int ch, hh;
    item_chunk(it, ch, hh);
    if (!any_live) return;
    float w[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) w[t] = FWD ? 1.f : wsl[FWD ? 0 : hh][(wv * TPW + t) * 32 + row];
    if (hh == 0) {
      if constexpr (PARTIALS) {
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            const uint2 q = pfn[n][a];
            pf[n][4 * a] = __uint_as_float(q.x << 16);
            pf[n][4 * a + 1] = __uint_as_float(q.x & 0xffff0000u);
            pf[n][4 * a + 2] = __uint_as_float(q.y << 16);
            pf[n][4 * a + 3] = __uint_as_float(q.y & 0xffff0000u);
          }
        // the backward runs chunks in descending order; the segment's first
        // chunk refetches itself (an in-range address, never used)
        fetch_partial_rows(ch > c_lo ? ch - 1 : ch);
      }
    }
    const float* fs = Fs[bi];
    const __bf16* vs = Vs[bi];
    f32x16 hT[2];
    if constexpr (SPLIT) {
#pragma unroll
      for (int n = 0; n < 2; ++n) hT[n] = f32x16{};
    }
    // Operands of one k-block (16 tokens): the value side (shared by the wave's
    // tiles) and the two fp32 feature rows of each tile's slot. The block kk + 1 is read from LDS before
    // block kk is computed, so that the read latency overlaps the products.
    struct KOps {
      bf16x8 va[2];
      float4 a0[TPW], a1[TPW], c0[TPW], c1[TPW];
    };
    auto read_ops = [&](int kk, KOps& o) {
#pragma unroll
      for (int n = 0; n < 2; ++n)
        o.va[n] = *reinterpret_cast<const bf16x8*>(vs + (32 * n + row) * kVRow + 16 * kk + 8 * s);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float4* pa = reinterpret_cast<const float4*>(fs + ar[t] * kFRow + 16 * kk + 8 * s);
        const float4* pc = reinterpret_cast<const float4*>(fs + ac[t] * kFRow + 16 * kk + 8 * s);
        o.a0[t] = pa[0];
        o.a1[t] = pa[1];
        o.c0[t] = pc[0];
        o.c1[t] = pc[1];
      }
    };
    auto compute = [&](const KOps& o) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float4 a0 = o.a0[t], a1 = o.a1[t], c0v = o.c0[t], c1v = o.c1[t];
        float f[8] = {a0.x * c0v.x, a0.y * c0v.y, a0.z * c0v.z, a0.w * c0v.w,
                      a1.x * c1v.x, a1.y * c1v.y, a1.z * c1v.z, a1.w * c1v.w};
        if constexpr (!FWD && !SPLIT) {
#pragma unroll
          for (int j = 0; j < 8; ++j) f[j] *= w[t];
        }
        const bf16x8 bq = pack8(f);
        if constexpr (SPLIT) {
          hT[0] = mfma32(o.va[0], bq, hT[0]);
          hT[1] = mfma32(o.va[1], bq, hT[1]);
        } else {
          acc[t][0] = mfma32(o.va[0], bq, acc[t][0]);
          acc[t][1] = mfma32(o.va[1], bq, acc[t][1]);
        }
      }
    };
    KOps ops[2];
    read_ops(0, ops[0]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk + 1 < 4) read_ops(kk + 1, ops[(kk + 1) & 1]);
      compute(ops[kk & 1]);
    }
    if constexpr (SPLIT) {
      const float wt = w[0];
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[0][n][i] = fmaf(wt, hT[n][i], acc[0][n][i]);
    }
    if constexpr (PARTIALS) {
      // four independent partial sums (a fixed order), not one 32-long chain
      float dp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) dp[i & 3] = fmaf(pf[n][i], hT[n][i], dp[i & 3]);
      const float d = (dp[0] + dp[1]) + (dp[2] + dp[3]);
      // both lane groups hold value rows of the same slot
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(d), __float_as_uint(d), false, false);
      if (s == 0) dwl[hh][wv * 32 + row] += d + __uint_as_float(r[1]);
    }
  };

  // State emission before item it when it starts a chunk. It runs at the end
  // of the previous item, after that item's staging store: the stores then
  // trail the staging loads in flight (vmcnt retires loads and stores in
  // order), so the next waits for staging loads do not wait for them.
  auto emit_before = [&](int it) {
    if constexpr (EMIT) {
      int ch, hh;
      item_chunk(it, ch, hh);
      if (it < NI && any_live && hh == 0) {
#pragma unroll
        for (int t = 0; t < TPW; ++t)
          if (live[t]) emit(t, (size_t)u * NB + ch);
      }
    }
  };

  // Pipeline: items it and it + 1 alternate between the register stages sa and
  // sb; the loads of item it + 2 are issued when item it starts and land in
  // LDS when item it + 1 ends. The stores are unconditional (past the last
  // item they store the clamped last item into the idle buffer): a skipped
  // store would leave its registers' loads possibly pending at the loop head,
  // where the compiler would then wait for every load in flight.
  Stage sa, sb;
  if constexpr (!FWD) {
    // weights of dead tiles (slot clamped to 0) multiply products that are
    // never stored
    for (int i = tid; i < R * kSTiles * TPW * 32; i += kNT) {
      const int hh = i / (kSTiles * TPW * 32), j = i % (kSTiles * TPW * 32);
      const int tl = kSTiles * TPW * tgi + j / 32;
      wsl[hh][j] = wqs[(size_t)(kh * R + hh) * kS + (tl < kS / 32 ? tl * 32 + j % 32 : 0)];
    }
  }
  if (NI > 0) {
    load(sa, 0);
    load(sb, 1);
    store(0, sa);
  }
  emit_before(0);
  lds_sync();
  int bi = 0;
  for (int it = 0; it < NI; it += 2) {
    {
      load(sa, it + 2);
      process(it, bi);
      store(bi ^ 1, sb);
      emit_before(it + 1);
      lds_sync();
      bi ^= 1;
    }
    if (it + 1 < NI) {
      load(sb, it + 3);
      process(it + 1, bi);
      store(bi ^ 1, sa);
      emit_before(it + 2);
      lds_sync();
      bi ^= 1;
    }
  }

  if constexpr (MODE == 0 || MODE == 3) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      if (live[t]) {
        float* st = segtot + (((size_t)u * Sg + seg) * kS + slot[t]) * kD;
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
          for (int a = 0; a < 4; ++a)
            *reinterpret_cast<float4*>(st + 32 * n + c32_row(4 * a, l)) =
                make_float4(acc[t][n][4 * a], acc[t][n][4 * a + 1], acc[t][n][4 * a + 2], acc[t][n][4 * a + 3]);
      }
    }
  }
  if constexpr (PARTIALS) {
    const int B = (int)(gridDim.x / (TG * Sg)) / Hkv;
    if (live[0] && s == 0) {
      for (int hh = 0; hh < R; ++hh)
        dwqs[(((size_t)seg * B + b) * Hq + kh * R + hh) * kS + slot[0]] = dwl[hh][wv * 32 + row];
    }
  }
}

// Forward operands per (unit, chunk): KT16 [U][64][NB * 64] = k^T and
// VT16 [U][65][NB * 64] = [v^T; 1 (token < N)], bf16, tokens >= N zero; and
// the chunk's denominator-state totals Zt [U][NB][kZt]: [r * 64 + c] =
// sum_j k_jr k_jc (matrix cores, wave w owns the 32 x 32 block (w / 2, w % 2)),
// [4096 + d] = sum_j k_jd.
template <typename T>
__global__ __launch_bounds__(256) void k2_fwd_prep(const T* __restrict__ k, const T* __restrict__ v, int N, int NB,
                                                   int nprep, uint16_t* __restrict__ KT16,
                                                   uint16_t* __restrict__ VT16, float* __restrict__ Zt,
                                                   SlotCoefArgs sc) {
  // blocks nprep .. nprep + 8 Hq - 1: the slot coefficients (query head, part)
  if ((int)blockIdx.x >= nprep) {
    const int i = (int)blockIdx.x - nprep;
    slot_coefficients_part(kSlot, sc, i >> 3, i & 7);
    return;
  }
  __shared__ __attribute__((aligned(16))) __bf16 kT[kD][kC + 8];
  __shared__ __attribute__((aligned(16))) __bf16 vT[kD + 1][kC + 8];
  const int u = blockIdx.x / NB, ch = blockIdx.x % NB;
  const int tid = threadIdx.x, j = tid >> 2, qq = tid & 3;
  const int tok = ch * kC + j;
  const bool ok = tok < N;
  const size_t off = ((size_t)u * N + (ok ? tok : N - 1)) * kD + 16 * qq;
  // 16 consecutive elements per thread as 16-byte vector loads, issued before
  // any use (the row index is clamped, so every load is in bounds)
  float kv[16], vv[16];
  if constexpr (sizeof(T) == 2) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 kw[2], vw[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      kw[i] = reinterpret_cast<const u32x4*>(k + off)[i];
      vw[i] = reinterpret_cast<const u32x4*>(v + off)[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kv[8 * i + 2 * e] = __uint_as_float(kw[i][e] << 16);
        kv[8 * i + 2 * e + 1] = __uint_as_float(kw[i][e] & 0xffff0000u);
        vv[8 * i + 2 * e] = __uint_as_float(vw[i][e] << 16);
        vv[8 * i + 2 * e + 1] = __uint_as_float(vw[i][e] & 0xffff0000u);
      }
  } else {
    float4 kf[4], vf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kf[i] = reinterpret_cast<const float4*>(k + off)[i];
      vf[i] = reinterpret_cast<const float4*>(v + off)[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv[4 * i] = kf[i].x, kv[4 * i + 1] = kf[i].y, kv[4 * i + 2] = kf[i].z, kv[4 * i + 3] = kf[i].w;
      vv[4 * i] = vf[i].x, vv[4 * i + 1] = vf[i].y, vv[4 * i + 2] = vf[i].z, vv[4 * i + 3] = vf[i].w;
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    kv[e] = ok ? kv[e] : 0.f;
    vv[e] = ok ? vv[e] : 0.f;
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    kT[16 * qq + e][j] = (__bf16)kv[e];
    vT[16 * qq + e][j] = (__bf16)vv[e];
  }
  if (qq == 0) vT[kD][j] = (__bf16)(ok ? 1.f : 0.f);
  __syncthreads();
  const size_t np = (size_t)NB * kC;
  for (int idx = tid; idx < (2 * kD + 1) * 8; idx += 256) {
    const int r = idx >> 3, c8 = idx & 7;
    if (r < kD) {
      *reinterpret_cast<bf16x8*>(KT16 + ((size_t)u * kD + r) * np + (size_t)ch * kC + 8 * c8) =
          *reinterpret_cast<const bf16x8*>(&kT[r][8 * c8]);
    } else {
      const int rv = r - kD;
      *reinterpret_cast<bf16x8*>(VT16 + ((size_t)u * (kD + 1) + rv) * np + (size_t)ch * kC + 8 * c8) =
          *reinterpret_cast<const bf16x8*>(&vT[rv][8 * c8]);
    }
  }
  {
    const int w = tid >> 6, l = tid & 63, s = l >> 5, row = l & 31, mr = w >> 1, mc = w & 1;
    f32x16 acc = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      acc = mfma32(*reinterpret_cast<const bf16x8*>(&kT[32 * mr + row][16 * kk + 8 * s]),
                   *reinterpret_cast<const bf16x8*>(&kT[32 * mc + row][16 * kk + 8 * s]), acc);
    float* z = Zt + ((size_t)u * NB + ch) * kZt;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[(32 * mr + c32_row(i, l)) * kD + 32 * mc + row] = acc[i];
    // sum_j k_jd: thread (d, quarter) sums 16 tokens, then the quarters in a fixed order
    __shared__ float ksum[4][kD];
    {
      const int d = tid & 63, qt = tid >> 6;
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) sum += (float)kT[d][16 * qt + i];
      ksum[qt][d] = sum;
    }
    __syncthreads();
    if (tid < kD) z[kD * kD + tid] = (ksum[0][tid] + ksum[1][tid]) + (ksum[2][tid] + ksum[3][tid]);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Tiles per wave of the scan kernels (modes 0-4): two wherever the per-head
// products are not kept apart (MODE 4: one, for one wave per tile).
constexpr int scan_tpw(bool fwd, int mode) { return mode == 4 ? 1 : (fwd || mode == 1) ? 2 : 1; }
// waves per block of the scan kernels
constexpr int scan_nw(bool fwd, int mode) { return mode == 4 ? 1 : 4; }

ScanPlan scan_plan(int U, int NB, size_t scratch_bytes, bool fwd) {
  // Segment count from a model of block rounds on MI355X's 256 CUs: each
  // kernel runs two blocks per CU, a block's time is proportional to its
  // chunks, and a partial last round costs a full one; each segment adds a
  // little carry traffic (a replay block reads the totals of the segments on
  // one side of its own). A function of the geometry alone, so that a size
  // query and the launch it sizes always agree.
  constexpr double kSlots = 2.0 * 256;
  const size_t seg_bytes = sizeof(float) * (size_t)U * kS * kD;
  int cap = NB;
  if (scratch_bytes != (size_t)-1) cap = (int)std::min<size_t>((size_t)NB, scratch_bytes / seg_bytes);
  if (cap < 1) cap = 1;
  auto rounds = [&](int mode, int S) {
    return std::ceil(scan_tile_groups(scan_tpw(fwd, mode), scan_nw(fwd, mode)) * (double)U * S / kSlots);
  };
  int best_S = 1;
  double best = 0.0;
  for (int want = 1; want <= cap; ++want) {
    const int SL = (NB + want - 1) / want, S = (NB + SL - 1) / SL;
    const double est = S == 1 ? rounds(2, 1) * SL : (rounds(0, S) + rounds(1, S)) * SL + 0.1 * S;
    if (want == 1 || est < best) {
      best = est;
      best_S = S;
    }
  }
  ScanPlan p;
  p.SL = (NB + best_S - 1) / best_S;
  p.S = (NB + p.SL - 1) / p.SL;
  p.seg_bytes = p.S > 1 ? seg_bytes * p.S : 0;
  return p;
}

ScanPlan bwd_scan_plan(int U, int NB, int R) {
  // One local pass per segment (MODE 3, two blocks per CU), so the time is
  // about rounds x (items per segment + a pipeline start of two items); each
  // segment adds its totals and carry traffic. A function of the geometry
  // alone.
  constexpr double kSlots = 2.0 * 256;
  const int tg = scan_tile_groups(scan_tpw(false, 3), scan_nw(false, 3));
  int best_S = 1;
  double best = 0.0;
  for (int want = 1; want <= NB; ++want) {
    const int SL = (NB + want - 1) / want, S = (NB + SL - 1) / SL;
    const double est = std::ceil(tg * (double)U * S / kSlots) * (SL * R + 2.0) + (S > 1 ? 0.25 * S : 0.0);
    if (want == 1 || est < best) {
      best = est;
      best_S = S;
    }
  }
  ScanPlan p;
  p.SL = (NB + best_S - 1) / best_S;
  p.S = (NB + p.SL - 1) / p.SL;
  p.seg_bytes = p.S > 1 ? sizeof(float) * (size_t)U * kS * kD * p.S : 0;
  return p;
}

template <bool FWD, bool PART>
static void launch_scan_impl(const ScanPlan& p, const ScanArgs& a, hipStream_t st, const Timer& timed) {
  constexpr int T0 = scan_tpw(FWD, 0), T1 = scan_tpw(FWD, 1), T2 = scan_tpw(FWD, 2);
  constexpr int W0 = scan_nw(FWD, 0), W1 = scan_nw(FWD, 1), W2 = scan_nw(FWD, 2);
  auto grid = [&](int tpw, int nw) { return dim3((unsigned)(scan_tile_groups(tpw, nw) * a.U * p.S)); };
  const char* name = FWD ? "k2_state_fwd" : "k2_state_bwd";
  if (p.S == 1) {
    timed(name, st, [&] {
      hipLaunchKernelGGL((k2_scan<FWD, 2, T2, W2, PART>), grid(T2, W2), dim3(64 * W2), 0, st, a.F, a.frows, a.V,
                         a.vrows, a.wqs, a.PR, nullptr, a.Hq, a.Hkv, a.N, a.NB, p.SL, p.S, a.outR, nullptr, a.dwqs);
    });
    return;
  }
  if constexpr (!FWD) {
    // one local pass per segment, then the segments' carries
    constexpr int T3 = scan_tpw(false, 3), W3 = scan_nw(false, 3);
    constexpr int T4 = scan_tpw(false, 4), W4 = scan_nw(false, 4);
    timed(name, st, [&] {
      hipLaunchKernelGGL((k2_scan<false, 3, T3, W3, PART>), grid(T3, W3), dim3(64 * W3), 0, st, a.F, a.frows, a.V,
                         a.vrows, a.wqs, a.PR, nullptr, a.Hq, a.Hkv, a.N, a.NB, p.SL, p.S, a.outR, a.segtot, a.dwqs);
    });
    timed("k2_state_bwd_carry", st, [&] {
      const dim3 g4((unsigned)(scan_tile_groups(T4, W4) * a.U));  // one block per (unit, tile group)
      hipLaunchKernelGGL((k2_scan<false, 4, T4, W4, false>), g4, dim3(64 * W4), 0, st, a.F, a.frows,
                         a.V, a.vrows, a.wqs, a.PR, a.segtot, a.Hq, a.Hkv, a.N, a.NB, p.SL, p.S, a.carryR,
                         nullptr, nullptr);
    });
    return;
  }
  if constexpr (FWD) {
    // segment totals, then each segment's replay from the totals before it
    timed("k2_state_fwd_totals", st, [&] {
      hipLaunchKernelGGL((k2_scan<true, 0, T0, W0, false>), grid(T0, W0), dim3(64 * W0), 0, st, a.F, a.frows, a.V,
                         a.vrows, a.wqs, a.PR, nullptr, a.Hq, a.Hkv, a.N, a.NB, p.SL, p.S, nullptr, a.segtot,
                         nullptr);
    });
    timed(name, st, [&] {
      hipLaunchKernelGGL((k2_scan<true, 1, T1, W1, false>), grid(T1, W1), dim3(64 * W1), 0, st, a.F, a.frows, a.V,
                         a.vrows, a.wqs, a.PR, a.segtot, a.Hq, a.Hkv, a.N, a.NB, p.SL, p.S, a.outR, nullptr,
                         nullptr);
    });
  }
}

template <bool FWD>
void launch_scan(const ScanPlan& p, const ScanArgs& a, hipStream_t st, const Timer& timed) {
  // the backward forms the coefficient partials only when dwqs is given
  if (!FWD && a.dwqs != nullptr)
    launch_scan_impl<FWD, true>(p, a, st, timed);
  else
    launch_scan_impl<FWD, false>(p, a, st, timed);
}

template void launch_scan<true>(const ScanPlan&, const ScanArgs&, hipStream_t, const Timer&);
template void launch_scan<false>(const ScanPlan&, const ScanArgs&, hipStream_t, const Timer&);

template <typename T>
void launch_fwd_prep(const LaunchGeom& g, const T* k, const T* v, uint16_t* KT16, uint16_t* VT16, float* Zt,
                     const SlotCoefArgs& sc, hipStream_t st, const Timer& timed) {
  const int nprep = g.U * g.NB;
  timed("k2_fwd_prep", st, [&] {
    hipLaunchKernelGGL(k2_fwd_prep<T>, dim3(nprep + 8 * g.Hq), dim3(256), 0, st, k, v, g.N, g.NB, nprep, KT16, VT16,
                       Zt, sc);
  });
}
template void launch_fwd_prep<float>(const LaunchGeom&, const float*, const float*, uint16_t*, uint16_t*, float*,
                                     const SlotCoefArgs&, hipStream_t, const Timer&);
template void launch_fwd_prep<uint16_t>(const LaunchGeom&, const uint16_t*, const uint16_t*, uint16_t*, uint16_t*,
                                        float*, const SlotCoefArgs&, hipStream_t, const Timer&);

}  // namespace oal
