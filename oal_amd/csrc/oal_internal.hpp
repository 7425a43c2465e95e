// Declarations shared by the translation units of liboal_amd.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <functional>

namespace oal {

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct LaunchGeom {
  int B, Hq, Hkv, N, NB, U, R;
};

// Runs `launch`, bracketed by HIP events on `stream` when profiling is on.
using Timer = std::function<void(const char*, hipStream_t, const std::function<void()>&)>;

struct MfmaSaved {
  float* wqs;     // [Hq][kS] slot coefficients
  uint16_t* PT;   // [U][NB][kKS][64][16] bf16
  uint16_t* PR;   // [U][NB][kS/32][4][32][16] bf16
  float* PZ;      // [U][NB][kFP] denominator column, natural order
};

size_t mfma_saved_bytes(int Hq, int U, int NB);
MfmaSaved mfma_saved_view(void* base, int Hq, int U, int NB);

template <typename T>
void launch_mfma_forward(const LaunchGeom& g, const void* q, const void* k, const void* v, const int32_t* labels,
                         const float* c0, const float* lam, const float* gam, int groups, float scale, float floor,
                         void* out, float* num, float* den, void* saved, hipStream_t st, const Timer& timed);

int run_mfma_selftest(int* dev_errors, hipStream_t st);

}  // namespace oal
