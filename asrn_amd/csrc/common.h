// Shared device and host helpers for the ASRN HIP library (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "asrn_hip.h"

namespace asrn {

constexpr int kWave = 64;

// ---- error reporting (thread-local last message; every entry point returns 0 on success) -------------------------
int fail(const char* fmt, ...);
int check_launch(const char* what);
// out[c] = sum over g of partial[g * cols + c] (per-workgroup partial rows of parameter gradients), in a fixed order,
// one launch on `stream`
int group_sums(const float* partial, int groups, int cols, float* out, hipStream_t stream);

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

// ---- workgroup placement ----------------------------------------------------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup i runs on XCD i % 8), each with its own L2. For a
// 1-D grid of xcd_grid(rows, chunks) workgroups, the (chunk, row) of this workgroup such that every chunk of a row runs
// on XCD row % 8: a later kernel with the same map reads what an earlier one wrote for the row from that XCD's L2.
// The rows past `rows` in the last group of 8 come out >= rows; their workgroups have nothing to do.
constexpr int kXcdCount = 8;
inline unsigned xcd_grid(int64_t rows, int chunks) {
  return (unsigned)((rows + kXcdCount - 1) / kXcdCount * kXcdCount * chunks);
}
__device__ __forceinline__ void xcd_chunk_row(int chunks, int* chunk, int64_t* row) {
  const int64_t i = blockIdx.x, rest = i / kXcdCount;
  *chunk = (int)(rest % chunks);
  *row = i % kXcdCount + kXcdCount * (rest / chunks);
}

// ---- DPP reductions (no LDS traffic): rotate within each 16-lane row, then combine the four rows ---------------------
// DPP control words of GFX9-family ISAs: row_ror:n = 0x120 + n.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// every lane of each 16-lane row ends with the row's sum / max
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp<0x128>(v);
  v += dpp<0x124>(v);
  v += dpp<0x122>(v);
  v += dpp<0x121>(v);
  return v;
}
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp<0x128>(v));
  v = fmaxf(v, dpp<0x124>(v));
  v = fmaxf(v, dpp<0x122>(v));
  v = fmaxf(v, dpp<0x121>(v));
  return v;
}
// wave-uniform totals, combined in a fixed order (deterministic)
__device__ __forceinline__ float wave_sum_u(float v) {
  v = row_sum16(v);
  return ((readlane_f(v, 0) + readlane_f(v, 16)) + readlane_f(v, 32)) + readlane_f(v, 48);
}
__device__ __forceinline__ float wave_max_u(float v) {
  v = row_max16(v);
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
// the two 32-lane halves' sums
__device__ __forceinline__ void half_sums_u(float v, float* h0, float* h1) {
  v = row_sum16(v);
  *h0 = readlane_f(v, 0) + readlane_f(v, 16);
  *h1 = readlane_f(v, 32) + readlane_f(v, 48);
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
