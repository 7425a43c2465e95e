// MFMA fragment types and the rotated feature-slot order used by the bf16
// (matrix-core) kernels on gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "oal_common.hpp"

namespace oal {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// v_mfma_f32_32x32x16_bf16: lane l supplies A[l%32][8*(l/32) + j] and
// B[8*(l/32) + j][l%32] (j < 8); accumulator register i of lane l holds
// C[8*(i/4) + 4*(l/32) + i%4][l%32].
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8*(l/16) + j],
// B[8*(l/16) + j][l%16]; register i holds C[4*(l/16) + i][l%16].
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// v_mfma_f32_16x16x16_bf16: lane l supplies A[l%16][4*(l/16) + j],
// B[4*(l/16) + j][l%16] (j < 4); register i holds C[4*(l/16) + i][l%16], so a
// 16x16 accumulator tile is, lane for lane, the A operand of a product whose K
// index is the tile's row.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 mfma16k16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ constexpr int c32_row(int i, int lane) { return 8 * (i / 4) + 4 * (lane / 32) + (i % 4); }
__device__ __forceinline__ constexpr int c16_row(int i, int lane) { return 4 * (lane / 16) + i; }

// ---------------------------------------------------------------------------
// Rotated slot order.
// The 32x32x16 MFMA splits K into two lane groups (s = lane/32) of 8 slots.
// Lane group s keeps its token's row rotated by 32*s: xrot[m] = x[(m + 32 s) % 64]
// (xrot[64] = 1, xrot[65] = 0). A base (rb, cb) evaluated on xrot is the
// feature x[(rb+32s)%64] * x[(cb+32s)%64]: one static register pair serves
// both lane groups. Slot sigma = 16 t + 8 s + j belongs to k-step t, lane
// group s and base 8 t + j. Bases: 32 linear (d, one), 1 constant (one, one),
// 1056 pair orbits under the +32 rotation, then padding (zero, zero).
// Slots whose rotated pair repeats the s = 0 pair (pairs {r, r+32}) and the
// constant's s = 1 slot are invalid: their state rows are zero.
// ---------------------------------------------------------------------------
constexpr int kS = 2208;         // slots (138 k-steps of 16, 69 tiles of 32)
constexpr int kBases = kS / 2;   // 1104
constexpr int kKS = kS / 16;     // 138

struct SlotTable {
  uint8_t rb[kBases];
  uint8_t cb[kBases];
  uint8_t ar[kS];   // actual row index (64 = one, 65 = zero)
  uint8_t ac[kS];   // actual column index
  int16_t nat[kS];  // natural feature index (grouped_reference pair order), -1 if invalid
};

constexpr int pair_index(int r, int c) { return r * (r + 1) / 2 + c; }

constexpr SlotTable make_slot_table() {
  SlotTable t{};
  bool assigned[kD * (kD + 1) / 2] = {};
  int b = 0;
  for (int d = 0; d < kD / 2; ++d) {
    t.rb[b] = static_cast<uint8_t>(d);
    t.cb[b] = 64;
    ++b;
  }
  t.rb[b] = 64;
  t.cb[b] = 64;
  ++b;
  for (int r = 0; r < kD; ++r) {
    for (int c = 0; c <= r; ++c) {
      if (assigned[pair_index(r, c)]) continue;
      t.rb[b] = static_cast<uint8_t>(r);
      t.cb[b] = static_cast<uint8_t>(c);
      ++b;
      assigned[pair_index(r, c)] = true;
      const int r2 = (r + 32) % 64, c2 = (c + 32) % 64;
      const int hi = r2 > c2 ? r2 : c2, lo = r2 > c2 ? c2 : r2;
      assigned[pair_index(hi, lo)] = true;
    }
  }
  for (; b < kBases; ++b) {
    t.rb[b] = 65;
    t.cb[b] = 65;
  }
  for (int sg = 0; sg < kS; ++sg) {
    const int tt = sg / 16, s = (sg % 16) / 8, j = sg % 8, base = 8 * tt + j;
    const int rb = t.rb[base], cb = t.cb[base];
    int nat = -1, ar = 65, ac = 65;
    if (rb == 64) {
      if (s == 0) {
        nat = 0;
        ar = 64;
        ac = 64;
      }
    } else if (rb < 64 && cb == 64) {
      const int d = (rb + 32 * s) % 64;
      nat = 1 + d;
      ar = d;
      ac = 64;
    } else if (rb < 64) {
      const int r = (rb + 32 * s) % 64, c = (cb + 32 * s) % 64;
      const int hi = r > c ? r : c, lo = r > c ? c : r;
      const bool dup = s == 1 && hi == (rb > cb ? rb : cb) && lo == (rb > cb ? cb : rb);
      if (!dup) {
        nat = 1 + kD + pair_index(hi, lo);
        ar = hi;
        ac = lo;
      }
    }
    t.nat[sg] = static_cast<int16_t>(nat);
    t.ar[sg] = static_cast<uint8_t>(ar);
    t.ac[sg] = static_cast<uint8_t>(ac);
  }
  return t;
}

constexpr SlotTable kSlotHost = make_slot_table();

constexpr bool slot_table_is_a_permutation() {
  bool seen[kFeat] = {};
  int valid = 0;
  for (int s = 0; s < kS; ++s) {
    const int n = kSlotHost.nat[s];
    if (n < 0) continue;
    if (n >= kFeat || seen[n]) return false;
    seen[n] = true;
    ++valid;
  }
  return valid == kFeat;
}
static_assert(slot_table_is_a_permutation(), "every feature must occupy exactly one valid slot");

// Value of base B on a rotated row (static register indices).
template <int B>
__device__ __forceinline__ float base_value(const float (&x)[kD]) {
  constexpr int rb = kSlotHost.rb[B], cb = kSlotHost.cb[B];
  if constexpr (rb == 65) {
    return 0.f;
  } else if constexpr (rb == 64) {
    return 1.f;
  } else if constexpr (cb == 64) {
    return x[rb];
  } else {
    return x[rb] * x[cb];
  }
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ s16x4 pack4(const float (&v)[4]) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  u32x2 u = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  return __builtin_bit_cast(s16x4, u);
}

__device__ __forceinline__ bf16x8 pack8(const float (&v)[8]) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 u = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
  return __builtin_bit_cast(bf16x8, u);
}

// A fragment of k-step T: features of bases 8T..8T+7 on the rotated row,
// scaled by the lane group's slot coefficients w[0..7].
template <int T, int... J>
__device__ __forceinline__ bf16x8 feature_fragment_impl(const float (&x)[kD], const float (&w)[8],
                                                        std::integer_sequence<int, J...>) {
  float v[8] = {(base_value<8 * T + J>(x) * w[J])...};
  return pack8(v);
}
template <int T>
__device__ __forceinline__ bf16x8 feature_fragment(const float (&x)[kD], const float (&w)[8]) {
  return feature_fragment_impl<T>(x, w, std::make_integer_sequence<int, 8>{});
}
// Lane J of this lane's 16-lane row (DPP row_newbcast:J). Used as an operand
// of a VALU instruction it folds into that instruction's DPP source, so a
// per-slot weight reaches the lanes that need it without its own instruction:
// one register can hold the 16 weights a row of lanes uses in turn, in place
// of an LDS read of every weight by every lane.
template <int J>
__device__ __forceinline__ float row_bcast(float w) {
  static_assert(J >= 0 && J < 16, "a row has 16 lanes");
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(w), 0x150 + J, 0xf, 0xf, true));
}
// Weighted feature of base B with the weight wb applied to the first factor:
// the instruction that reads the broadcast weight then reads no register
// written by the VALU just before it (a DPP read of such a register needs two
// wait states).
template <int B>
__device__ __forceinline__ float weighted_base(const float (&x)[kD], float wb) {
  constexpr int rb = kSlotHost.rb[B], cb = kSlotHost.cb[B];
  if constexpr (rb == 65) {
    return 0.f * wb;
  } else if constexpr (rb == 64) {
    return wb;
  } else if constexpr (cb == 64) {
    return x[rb] * wb;
  } else {
    return (x[rb] * wb) * x[cb];
  }
}
// feature_fragment with the weights in one register: lane OFF + j of each row
// holds the weight of slot 8 s + j of k-step T (j < 8; s = the row's lane
// group; OFF = 0 or 8, so that a register can serve two k-steps).
template <int T, int OFF, int... J>
__device__ __forceinline__ bf16x8 feature_fragment_row_impl(const float (&x)[kD], float wrow,
                                                            std::integer_sequence<int, J...>) {
  float v[8] = {weighted_base<8 * T + J>(x, row_bcast<OFF + J>(wrow))...};
  return pack8(v);
}
template <int T, int OFF = 0>
__device__ __forceinline__ bf16x8 feature_fragment_row(const float (&x)[kD], float wrow) {
  return feature_fragment_row_impl<T, OFF>(x, wrow, std::make_integer_sequence<int, 8>{});
}
template <int T, int... J>
__device__ __forceinline__ bf16x8 raw_fragment_impl(const float (&x)[kD], std::integer_sequence<int, J...>) {
  float v[8] = {base_value<8 * T + J>(x)...};
  return pack8(v);
}
template <int T>
__device__ __forceinline__ bf16x8 raw_fragment(const float (&x)[kD]) {
  return raw_fragment_impl<T>(x, std::make_integer_sequence<int, 8>{});
}

__device__ __forceinline__ float bf16_to_f(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }

}  // namespace oal

namespace oal {

// ---------------------------------------------------------------------------
// R-layout k-step tiles. The chunk state in the R layout is [69 tiles][4 value
// blocks][32 slots][16 values] bf16; a k-step (16 slots) staged in LDS is
// [4 value blocks][16 slots][16 values], the four 512-byte pieces of its tile.
// ---------------------------------------------------------------------------
// Element offset in the chunk's R state of piece p (value block) of k-step t,
// for the 32 lanes r of a 512-byte copy:
__device__ __forceinline__ size_t rpiece(int t, int p, int r) {
  return (size_t)(t >> 1) * 2048 + p * 512 + (t & 1) * 256 + r * 8;
}

// B fragment of value half n of a staged k-step tile: lane l supplies slots
// 8 (l / 32) .. + 7 of value 32 n + l % 32. ds_read_b64_tr_b16 hands lane i of
// each 16-lane group column i of the 4 x 16 block whose row j the group's lanes
// 4 j .. 4 j + 3 address (four values each), so the 16-lane group g reads rows =
// slots 8 (g / 2) + 0..3, then + 4..7, of value block 2 n + g % 2.
typedef short trv4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8 tr_fragment(const __bf16* tile, int lane, int n) {
  const int g = lane >> 4, i = lane & 15;
  const __bf16* p = tile + (2 * n + (g & 1)) * 256 + (8 * (g >> 1) + (i >> 2)) * 16 + 4 * (i & 3);
  typedef __attribute__((address_space(3))) trv4 lds_trv4;
  const trv4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_trv4*)(p));
  const trv4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_trv4*)(p + 4 * 16));
  typedef short trv8 __attribute__((ext_vector_type(8)));
  const trv8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// Work item of a 1-D grid over (query head in group, chunk, unit), ordered so
// that the query heads of one (chunk, unit) run on one XCD and share its L2:
// workgroups are dispatched round-robin over the 8 XCDs, so workgroup id goes
// to XCD id % 8; item w = (id % 8) * (total / 8) + id / 8 gives each XCD a
// contiguous range of items (head fastest). Falls back to w = id when the
// item count is not a multiple of 8.
__device__ __forceinline__ void head_chunk_unit(int R, int NB, int U, int& hh, int& ch, int& u) {
  const int total = R * NB * U;
  const int id = blockIdx.x;
  const int w = (total & 7) == 0 ? (id & 7) * (total >> 3) + (id >> 3) : id;
  hh = w % R;
  ch = (w / R) % NB;
  u = w / (R * NB);
}

}  // namespace oal

namespace oal {

// Asynchronous global -> LDS copy (global_load_lds_dwordx4): every lane of the
// wave moves 16 bytes from its own global address to lds_base + 16 * lane,
// where lds_base is wave-uniform. Completion is tracked by vmcnt.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;
__device__ __forceinline__ void copy16_to_lds(const void* gsrc, void* lds_base) {
  __builtin_amdgcn_global_load_lds((gbl_void_t*)gsrc, (lds_void_t*)lds_base, 16, 0, 0);
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left free).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Marks the 64 registers of a per-lane array as read and written at this
// point (no instruction is emitted): arithmetic that updates them cannot be
// moved past it. Code generation for a fully unrolled pipeline sees one basic
// block and may otherwise defer whole stages of register arithmetic to the
// end, holding (and spilling) the operands of every stage in between.
__device__ __forceinline__ void pin64(float (&a)[64]) {
#pragma unroll
  for (int i = 0; i < 64; i += 16)
    asm volatile(""
                 : "+v"(a[i]), "+v"(a[i + 1]), "+v"(a[i + 2]), "+v"(a[i + 3]), "+v"(a[i + 4]), "+v"(a[i + 5]),
                   "+v"(a[i + 6]), "+v"(a[i + 7]), "+v"(a[i + 8]), "+v"(a[i + 9]), "+v"(a[i + 10]),
                   "+v"(a[i + 11]), "+v"(a[i + 12]), "+v"(a[i + 13]), "+v"(a[i + 14]), "+v"(a[i + 15]));
}

// NS LDS stages of an asynchronous copy ring. The stages are distinct
// __shared__ objects: the compiler then tells a read of one stage from the
// copies still in flight into the others, where a single array would make it
// wait for every copy in flight (vmcnt(0)) before each read.
template <int NS>
struct LdsRing {
  __bf16* st[NS];
};

// Ring barrier: this wave's copies older than the newest N have landed in LDS
// (vmcnt(N)), its own LDS reads and writes are done (lgkmcnt(0)), then the
// workgroup barrier. Unlike __syncthreads() it carries no release fence, which
// would wait for every asynchronous copy in flight (vmcnt(0)) and empty the
// ring; the empty asm statements keep the compiler from moving memory accesses
// across it, the scheduling barriers keep each stage's arithmetic between its
// two ring barriers (so that products of later stages are not hoisted and
// spilled).
template <int N>
__device__ __forceinline__ void ring_sync() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

// Copies N4 float4 from global memory to LDS over NT threads with every load
// of a thread issued before its first store (a strided loop waits for each
// load before issuing the next). Items t + NT x past the end are clamped onto
// the last item, which its own thread also copies: the same value to the same
// place.
template <int NT, int N4>
__device__ __forceinline__ void stage_f4(float4* dst, const float4* __restrict__ src, int t) {
  constexpr int kIt = (N4 + NT - 1) / NT;
  float4 v[kIt];
#pragma unroll
  for (int x = 0; x < kIt; ++x) v[x] = src[min(t + NT * x, N4 - 1)];
#pragma unroll
  for (int x = 0; x < kIt; ++x) dst[min(t + NT * x, N4 - 1)] = v[x];
}

// Workgroup barrier over LDS only: this wave's LDS reads and writes are done
// (lgkmcnt(0)), then s_barrier. Unlike __syncthreads() it does not wait for
// outstanding global loads and stores (vmcnt counts both on gfx950), so
// register prefetches and state stores stay in flight across it; a use of a
// loaded register still waits for its own load.
__device__ __forceinline__ void lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((63 & 15) | ((63 >> 4) << 14) | (7 << 4));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace oal

