// Shared device and host helpers for the ASRN HIP library (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/asrn_hip.h"

namespace asrn {

constexpr int kWave = 64;

// ---- error reporting (thread-local last message; every entry point returns 0 on success) -------------------------
int fail(const char* fmt, ...);
int check_launch(const char* what);

#define ASRN_REQUIRE(cond, ...)            \
  do {                                     \
    if (!(cond)) return ::asrn::fail(__VA_ARGS__); \
  } while (0)

// ---- wave helpers ---------------------------------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
// sum over each aligned group of 32 lanes (the result is in every lane of the group)
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ int readlane_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// lanes of the wave that hold the same `nbits`-bit key as this lane (only meaningful for lanes with valid = true)
__device__ __forceinline__ uint64_t match_key(int key, int nbits, bool valid) {
  uint64_t m = __ballot(valid);
  for (int j = 0; j < nbits; ++j) {
    const int bit = (key >> j) & 1;
    const uint64_t bj = __ballot(bit);
    m &= bit ? bj : ~bj;
  }
  return m;
}

// ---- suffix match: number of leading equal previous signatures (NaN never equal) ---------------------------------
// Pf[t][j] = sig[t-1-j], NaN when t-1-j < 0 (reference nucleo:167-172, nucleo:98-108).
__device__ __forceinline__ int suffix_match(const float* __restrict__ sigb, int64_t q, int64_t k, int K) {
  int ell = 0;
  for (int j = 0; j < K; ++j) {
    const int64_t iq = q - 1 - j, ik = k - 1 - j;
    if (iq < 0 || ik < 0) break;
    if (!(sigb[iq] == sigb[ik])) break;
    ++ell;
  }
  return ell;
}

}  // namespace asrn
