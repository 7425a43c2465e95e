// Declarations shared by the translation units of liboal_amd.so.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <functional>
#include <tuple>

namespace oal {

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct LaunchGeom {
  int B, Hq, Hkv, N, NB, U, R;
};

// Runs `launch`, bracketed by HIP events on `stream` when profiling is on.
using Timer = std::function<void(const char*, hipStream_t, const std::function<void()>&)>;

// Per-head coefficient pack of the intra-chunk kernels: c0, scale * lam[g]
// (g < 8, zero padded), scale^2 * Gam[g][h] (8 x 8, zero padded).
constexpr int kIC = 80;
// Denominator-state entries per (unit, chunk) in pair-matrix form: the 64 x 64
// pair matrix, the 64 linear entries, the constant, padded.
constexpr int kZt = 64 * 64 + 64 + 64;
constexpr int kIcLam = 1;
constexpr int kIcGam = 9;

struct MfmaSaved {
  float* wqs;     // [Hq][kS] slot coefficients
  float* ic;      // [Hq][kIC] intra-chunk coefficient pack
  float* gm;      // [Hq][64][64] scale^2 Gam[g(r)][g(c)]
  float* lb;      // [Hq][64] scale lam[g(d)]
  uint16_t* PR;   // [U][NB][kS/32][4][32][16] bf16 (the readouts' and the backward's state)
  float* PZ;      // [U][NB][kFP] denominator column, natural order
  float* PZm;     // [U][NB][64][64] denominator column as a symmetric pair matrix
  uint16_t* KT16; // [U][64][NB * 64] bf16 k^T (tokens >= N zero)
  uint16_t* VT16; // [U][65][NB * 64] bf16 [v^T; 1 (token < N)]
  uint16_t* KAP;  // [B][Hq][NB][3][64][16] bf16 intra-chunk kappa, k2_local_dv's operand fragments
  float* Zt;      // [U][NB][kZt] per-chunk denominator-state totals (forward scratch)
  size_t bytes;
};

// R = query heads per KV head (B * Hq = U * R)
size_t mfma_saved_bytes(int Hq, int U, int NB, int R);
MfmaSaved mfma_saved_view(void* base, int Hq, int U, int NB, int R);

template <typename T>
void launch_mfma_forward(const LaunchGeom& g, const void* q, const void* k, const void* v, const int32_t* labels,
                         const float* c0, const float* lam, const float* gam, int groups, float scale, float floor,
                         void* out, float* num, float* den, void* saved, hipStream_t st, const Timer& timed);

struct MfmaWork {
  uint16_t* G16;  // [B][Hq][N][64] bf16 normalization VJP
  float* Gz;      // [B][Hq][N]
  uint16_t* GT16; // [B][Hq][66][NB * 64] bf16: G^T, Gz, 0
  uint16_t* QT16; // [B][Hq][66][NB * 64] bf16: q^T, 1 (token < N), 0
  uint16_t* dTR;  // [U][NB][kS/32][4][32][16] bf16
  float* dTz;     // [U][NB][kFP] exclusive suffix of the denominator state (natural order)
  float* dCt;     // [U][NB][kZt] per-chunk denominator dCarry (pair-matrix form)
  float* dwz;     // [U][NB][R][kFP] per-(chunk, head) denominator coefficient partials
  float* dwqz;    // [Hq][kFP] their sums over (batch, chunk)
  float* dwqs;    // [S][B][Hq][kS] slot-coefficient gradients (state part) per segment
  float* dwq;     // [Hq][kS] their sum
  float* segtot;  // [U][S][kS][65] per-segment dCarry totals, then (in place) their carries
  float* dqf;     // [B][Hq][N][64] local dq
  float* dkl;     // [U][N][64] local dk, summed over the unit's query heads
  float* dvl;     // [U][N][64] local dv, summed over the unit's query heads
  float* coefl;   // [Hq][73][B * NB] local (dc0, dlam[8], dgam[8][8]) per chunk
  float* coefs;   // [Hq][73] their sums over the chunks
  float* dkp;     // per-pair path: [B][Hq][N][64] local dk per query head
  float* dwql;    // per-pair path: [Hq][B * NB * 2][kS] local slot-coefficient partials
  uint16_t* dCR;  // [U][S][kS/32][4][32][16] bf16, R layout
  int S, SL;      // segments of the backward state scan and chunks per segment
  size_t bytes;
};
// pairwise: more than 8 groups (the per-pair path's local buffers)
MfmaWork mfma_work_view(void* base, int B, int Hq, int U, int N, int NB, bool pairwise);

// Independent kernels of one entry point may run on a second stream of the
// device: aux_stream(st) is that stream (default priority, created once per
// device), or st itself when per-kernel timing is on (timed kernels never
// overlap) or the stream cannot be had; stream_wait(w, s) makes stream w wait
// for the work enqueued on s so far (a fork or a join; both are captured into
// a graph like any stream dependency).
hipStream_t aux_stream(hipStream_t st);
void stream_wait(hipStream_t waiter, hipStream_t signaller);
// An event of the device's ring recorded on s now, and a wait for it enqueued
// on waiter later (stream_wait is the two at once).
hipEvent_t record_event(hipStream_t s);
void wait_event(hipStream_t waiter, hipEvent_t ev);
// The next event of the device's ring, not recorded: a launch_signal stop
// event. capturing(s): s is capturing a graph (or its state is unknown).
hipEvent_t next_event();
bool capturing(hipStream_t s);
// Launch of kernel k on s; with stop given, the launch itself records stop
// when the kernel completes (hipExtLaunchKernel's stop event), instead of a
// marker of its own behind it on s, which leaves s idle for several
// microseconds before its next kernel.
// If that launch is refused, the kernel is launched as usual and stop
// recorded behind it.
template <typename... KA, typename... A>
void launch_signal(void (*k)(KA...), dim3 grid, dim3 block, hipStream_t s, hipEvent_t stop, A... args) {
  static_assert(sizeof...(KA) == sizeof...(A), "one argument per kernel parameter");
  if (!stop) {
    hipLaunchKernelGGL(k, grid, block, 0, s, args...);
    return;
  }
  std::tuple<KA...> t{static_cast<KA>(args)...};
  void* ptrs[sizeof...(KA)];
  std::apply([&](auto&... e) {
    int i = 0;
    ((ptrs[i++] = static_cast<void*>(&e)), ...);
  }, t);
  if (hipExtLaunchKernel(reinterpret_cast<const void*>(k), grid, block, ptrs, 0, s, nullptr, stop, 0) != hipSuccess) {
    (void)hipGetLastError();
    hipLaunchKernelGGL(k, grid, block, 0, s, args...);
    (void)hipEventRecord(stop, s);
  }
}

// aux: a second stream for the kernels that do not depend on each other (the
// intra-chunk VJP beside the state scan, the key-side fold beside the query
// side), or st to run every kernel on st.
template <typename T>
int launch_mfma_backward(const LaunchGeom& g, const void* q, const void* k, const void* v, const int32_t* labels,
                         const float* c0, const float* lam, const float* gam, int groups, float scale, float floor,
                         const float* num, const float* den, const void* saved, const void* dout, const float* dnum,
                         const float* dden, void* dq, void* dk, void* dv, float* dc0, float* dlam, float* dgam,
                         void* workspace, hipStream_t st, hipStream_t aux, const Timer& timed);

struct LocalBwdArgs {
  const uint16_t* G16;
  const float* Gz;
  const uint16_t* QT16;
  const uint16_t* GT16;
  const uint16_t* KT16;
  const uint16_t* KAP;
  const float* PZ;
  const float* PZm;
  const int32_t* labels;
  const float* lam;
  const float* gam;
  const float* ic;
  const float* gm;
  const float* lb;
  int groups;
  float scale;
  float* dqf;
  float* dkl;
  float* dvl;
  float* coefl;  // nullptr when the coefficient gradients are not requested
  // per-pair coefficients (more than 8 groups): feature-form local VJP
  bool pairwise;
  const float* wqs;  // [Hq][kS] slot coefficients
  float* dkp;        // [B][Hq][N][64] local dk per query head, summed over the heads into dkl
  float* dwql;       // [Hq][B * NB * 2][kS] local slot-coefficient partials (nullptr: not requested)
};

// Feature-form local VJP of the per-pair path (oal_mfma_pair.hip).
template <typename T>
void launch_pair_local_bwd(const LaunchGeom& g, const T* q, const T* k, const T* v, const LocalBwdArgs& a,
                           bool need_dq, bool need_dkv, hipStream_t st, const Timer& timed);
void launch_pair_coef_grad(const LaunchGeom& g, const float* dwq, const float* dwqz, const int32_t* labels, int G,
                           float scale, float* dc0, float* dlam, float* dgam, hipStream_t st, const Timer& timed);

// Parts of the intra-chunk VJP that one call of launch_local_bwd launches:
// the dq kernel (which also forms the coefficient partials), the dk and dv kernels.
// With stop given and parts naming one kernel of the group-sum path, that
// kernel's launch records stop (launch_signal); the return value says whether
// it did (if not, the caller records its own event).
constexpr unsigned kLocalDq = 1, kLocalDk = 2, kLocalDv = 4, kLocalDkv = kLocalDk | kLocalDv;
template <typename T>
bool launch_local_bwd(const LaunchGeom& g, const T* q, const T* k, const T* v, const LocalBwdArgs& a, bool need_dq,
                      bool need_dkv, unsigned parts, hipStream_t st, const Timer& timed, hipEvent_t stop = nullptr);

// Segmentation of a chunk-state scan: S segments of SL chunks, a function of
// the geometry alone. The forward runs more than one segment as totals, carry,
// replay; the backward as one local pass per segment plus the segments'
// carries. Either needs seg_bytes of segment totals; scratch_bytes caps S
// ((size_t)-1: no cap).
struct ScanPlan {
  int S, SL;
  size_t seg_bytes;
};
ScanPlan scan_plan(int U, int NB, size_t scratch_bytes, bool fwd);
ScanPlan bwd_scan_plan(int U, int NB, int R);

// Operands and outputs of one chunk-state scan (oal_mfma_scan.hip).
// Matrix-core fp32 route (oal_f32_mma.hip, up to 8 groups): natural-order
// fp32 states as the scalar fp32 kernels keep them.
template <typename T>
void launch_f32_state_fwd(const LaunchGeom& g, const T* k, const T* v, float* carry, float* carry_z, hipStream_t st,
                          const Timer& timed);
template <typename T>
void launch_f32_intra_fwd(const LaunchGeom& g, const T* q, const T* k, const T* v, const int32_t* labels, const float* c0,
                          const float* lam, const float* gam, int groups, float scale, float* num, float* den,
                          hipStream_t st, const Timer& timed);
template <typename T>
void launch_f32_readout_fwd(const LaunchGeom& g, const T* q, const float* wq, const float* carry, const float* carry_z,
                            float floor, float* num, float* den, T* out, hipStream_t st, const Timer& timed);
// Chunk segments of the fp32 backward state scan, a function of the geometry
// alone (the workspace holds the segment totals): each (64-feature slice,
// unit, segment) block walks its segment's chunks and the unit's R heads.
// Model: four resident blocks per CU on a 256-CU MI355X, a block's time
// proportional to its items (plus a start of two), a partial last round costing
// a full one, and the carry pass (suffix of the segment totals, added to every
// chunk's state) about 40 items plus one per segment.
struct F32ScanPlan {
  int S, SL;
};
inline F32ScanPlan f32_bwd_plan(int U, int NB, int R) {
  constexpr int kSlices = 2176 / 64, kResident = 4 * 256;
  F32ScanPlan best{1, NB};
  double best_t = 0.0;
  for (int want = 1; want <= NB && want <= 64; ++want) {
    const int SL = (NB + want - 1) / want, S = (NB + SL - 1) / SL;
    const int blocks = kSlices * U * S;
    const double rounds = (double)((blocks + kResident - 1) / kResident);
    const double t = rounds * (SL * R + 2.0) + (S > 1 ? 40.0 + S : 0.0);
    if (want == 1 || t < best_t) {
      best_t = t;
      best = F32ScanPlan{S, SL};
    }
  }
  return best;
}

template <typename T>
struct F32BwdArgs {
  const T *q, *k, *v;
  const float *G, *Gz, *wq, *P, *Pz;
  const int32_t* labels;
  const float *c0, *lam, *gam;
  int groups;
  float scale;
  float *dT, *dTz;    // [U][NB][kFP][64], [U][NB][kFP]
  F32ScanPlan plan;   // f32_bwd_plan of the geometry
  float *segt, *segtz;  // segment totals, then carries: [U][S][kFP][64], [U][S][kFP] (S > 1)
  float* dwq_part;    // state coefficient partials [B][Hq][NB][kFP] (nullptr: not requested)
  float *dql, *dkl, *dvl;  // local parts, [B][Hq][N][64] per query head
  float* coefl;       // local coefficient partials [B][Hq][NB][73] (nullptr: not requested)
  float* coefs;       // their per-head sums [Hq][73]
  T *dq, *dk, *dv;
};
template <typename T>
void launch_f32_backward(const LaunchGeom& g, const F32BwdArgs<T>& a, hipStream_t st, hipStream_t aux,
                         const Timer& timed);

struct ScanArgs {
  const uint16_t* F;  // feature side, [X][frows][NB * 64] bf16 (rows 0..63 used)
  int frows;
  const uint16_t* V;  // value side, [X][vrows][NB * 64] bf16 (rows 0..63 used)
  int vrows;
  const float* wqs;   // backward: [Hq][kS] slot coefficients
  const uint16_t* PR; // backward: forward state (R layout), for the coefficient partials
  int U, Hq, Hkv, N, NB;
  uint16_t* outR;     // emitted state, R layout
  float* segtot;      // [U][S][kS][64] scratch when S > 1
  float* dwqs;        // backward: [S][B][Hq][kS] coefficient partials
  uint16_t* carryR;   // backward with S > 1: [U][S] segment carries, R layout
};
template <bool FWD>
void launch_scan(const ScanPlan& p, const ScanArgs& a, hipStream_t st, const Timer& timed);
// Inputs and outputs of the per-head slot coefficients (wqs, ic, gm, lb of the
// saved state), formed in blocks of k2_fwd_prep's launch.
struct SlotCoefArgs {
  const int32_t* labels;
  const float* c0;
  const float* lam;
  const float* gam;
  int G;
  float scale;
  float* wqs;
  float* ic;
  float* gm;
  float* lb;
};
template <typename T>
void launch_fwd_prep(const LaunchGeom& g, const T* k, const T* v, uint16_t* KT16, uint16_t* VT16, float* Zt,
                     const SlotCoefArgs& sc, hipStream_t st, const Timer& timed);
// Denominator state in pair-matrix form (oal_mfma_scan.hip): the chunk prefix
// (forward: PZ natural order and PZm) or suffix (backward: dTz) of per-chunk
// totals, and the backward's per-chunk totals and coefficient partials.
void launch_den_scan(bool fwd, const LaunchGeom& g, const float* tot, float* outZ, float* outZm, hipStream_t st,
                     const Timer& timed);
void launch_den_bwd(const LaunchGeom& g, const uint16_t* QT16, const uint16_t* GT16, int trows, const float* gm,
                    const float* lb, const float* ic, int kic, const float* PZ, const float* PZm, float* dCt,
                    float* dwz, hipStream_t st, const Timer& timed);

int run_mfma_selftest(int* dev_errors, hipStream_t st);

// FP64 route (oal_f64.hip): pairwise evaluation over 32-token tiles.
struct F64Geom {
  int B, Hq, Hkv, N;
};
size_t f64_workspace_bytes(int B, int Hq, int N);
void launch_f64_forward(const F64Geom& g, const double* q, const double* k, const double* v, const int32_t* labels,
                        const double* c0, const double* lam, const double* gam, int G, double scale, double* out,
                        double* num, double* den, hipStream_t st, const Timer& timed);
void launch_f64_backward(const F64Geom& g, const double* q, const double* k, const double* v,
                         const int32_t* labels, const double* c0, const double* lam, const double* gam, int G,
                         double scale, const double* num, const double* den, const double* dout,
                         const double* dnum, const double* dden, double* dq, double* dk, double* dv, double* dc0,
                         double* dlam, double* dgam, void* workspace, hipStream_t st, const Timer& timed);

}  // namespace oal
