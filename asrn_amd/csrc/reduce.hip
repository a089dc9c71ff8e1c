// Column sums of a row-major matrix (the bias gradients of the layer's projections, the per-token partials of the
// candidate backward, the slab partials of the weight gradients), in a fixed order: deterministic and free of the
// cleared semaphores a generic multi-workgroup reduction needs.
//
// A workgroup of 256 threads covers `cw` lanes of VEC adjacent columns by 256 / cw row lanes. Each thread sums its
// rows of one slab of R rows (row lane r takes rows r, r + 256 / cw, ...), then the row lanes combine in an LDS tree
// of fixed shape. With more than one slab, the slab sums land in a workspace and a second launch sums them the same
// way, as one slab. Everything accumulates in fp32; bf16 input is widened on load.
#include "common.h"

namespace asrn {

constexpr int kColThreads = 256;

// Parameter gradients from per-workgroup partial rows (groups x cols, row-major), one launch: a workgroup of 1024
// threads takes 64 adjacent columns by 16 row lanes, so each wave reads 256 contiguous bytes of one row. Row lane r
// sums rows r, r + 16, ... in increasing order, 32 loads in flight, then the row lanes combine in order in LDS.
constexpr int kGsCols = 64, kGsLanes = 16, kGsBatch = 32;
__global__ __launch_bounds__(kGsCols * kGsLanes) void k_group_sums(const float* __restrict__ partial, int groups,
                                                                   int cols, float* __restrict__ out) {
  __shared__ float red[kGsLanes][kGsCols];
  const int cl = threadIdx.x % kGsCols, rl = threadIdx.x / kGsCols;
  const int c = blockIdx.x * kGsCols + cl;
  float acc = 0.f;
  if (c < cols) {
    for (int g0 = rl; g0 < groups; g0 += kGsLanes * kGsBatch) {
      float v[kGsBatch];
#pragma unroll
      for (int j = 0; j < kGsBatch; ++j) {
        const int g = g0 + j * kGsLanes;
        v[j] = g < groups ? partial[(int64_t)g * cols + c] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < kGsBatch; ++j) acc += v[j];
    }
  }
  red[rl][cl] = acc;
  __syncthreads();
  if (rl == 0 && c < cols) {
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < kGsLanes; ++r) s += red[r][cl];
    out[c] = s;
  }
}

int group_sums(const float* partial, int groups, int cols, float* out, hipStream_t stream) {
  if (cols <= 0) return 0;
  hipLaunchKernelGGL(k_group_sums, dim3((unsigned)((cols + kGsCols - 1) / kGsCols)), dim3(kGsCols * kGsLanes), 0,
                     stream, partial, groups, cols, out);
  return check_launch("group_sums");
}

__device__ __forceinline__ float bf16_to_f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

template <int VEC>
__device__ __forceinline__ void load_cols(const float* p, float (&v)[VEC]) {
  if constexpr (VEC == 4) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    v[0] = *p;
  }
}
template <int VEC>
__device__ __forceinline__ void load_cols(const uint16_t* p, float (&v)[VEC]) {
  if constexpr (VEC == 4) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16_to_f(u.x & 0xffffu); v[1] = bf16_to_f(u.x >> 16);
    v[2] = bf16_to_f(u.y & 0xffffu); v[3] = bf16_to_f(u.y >> 16);
  } else {
    v[0] = bf16_to_f(*p);
  }
}

// out[blockIdx.y][c] = sum of x[r][c] over the rows r of slab blockIdx.y (rows [R y, R (y + 1)) within `rows`)
template <typename T, int VEC>
__global__ __launch_bounds__(kColThreads) void k_colsum(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                        int64_t ld, int64_t R, int cw, float* __restrict__ out) {
  __shared__ float red[kColThreads * VEC];
  const int tid = threadIdx.x, cl = tid % cw, rl = tid / cw, nrl = kColThreads / cw;
  const int64_t c0 = ((int64_t)blockIdx.x * cw + cl) * VEC;
  const int64_t r0 = (int64_t)blockIdx.y * R;
  const int64_t r1 = r0 + R < rows ? r0 + R : rows;
  const bool live = c0 < cols;   // VEC = 4 only when cols % 4 == 0, so a live lane's VEC columns are all in range
  float acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
  if (live) {
    const T* p = x + c0;
    int64_t r = r0 + rl;
    // eight rows in flight per thread, then the remainder, always in increasing row order
    for (; r + 7 * nrl < r1; r += 8 * nrl) {
      float v8[8][VEC];
#pragma unroll
      for (int j = 0; j < 8; ++j) load_cols<VEC>(p + (r + j * nrl) * ld, v8[j]);
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] += v8[j][v];
    }
    for (; r < r1; r += nrl) {
      float v1[VEC];
      load_cols<VEC>(p + r * ld, v1);
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] += v1[v];
    }
  }
  if (nrl > 1) {   // row lanes combine in a fixed tree: lane r takes r + s for s = nrl / 2, nrl / 4, ..., 1
#pragma unroll
    for (int v = 0; v < VEC; ++v) red[v * kColThreads + tid] = acc[v];
    __syncthreads();
    for (int s = nrl >> 1; s > 0; s >>= 1) {
      if (rl < s) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          acc[v] += red[v * kColThreads + tid + s * cw];
          red[v * kColThreads + tid] = acc[v];
        }
      }
      __syncthreads();
    }
  }
  if (rl == 0 && live) {
    float* o = out + (int64_t)blockIdx.y * cols + c0;
#pragma unroll
    for (int v = 0; v < VEC; ++v) o[v] = acc[v];
  }
}

// lanes along the columns: the smallest power of two covering the column groups, at most `cap`
static int col_lanes(int64_t groups, int cap) {
  int cw = 1;
  while (cw < groups && cw < cap) cw <<= 1;
  return cw;
}

// the first launch's slab count: enough workgroups to fill the chip, at least 16 rows per thread in a slab
static int64_t slabs_of(int64_t rows, int64_t groups, int cw) {
  if (rows <= 0 || groups <= 0) return 1;
  const int64_t tiles = (groups + cw - 1) / cw, nrl = kColThreads / cw;
  int64_t want = 1024 / tiles;
  const int64_t most = rows / (nrl * 16);
  if (want > most) want = most;
  if (want > 256) want = 256;
  if (want < 1) want = 1;
  const int64_t R = (rows + want - 1) / want;
  return (rows + R - 1) / R;
}

static int vec_of(const void* x, int64_t cols, int64_t ld, int elem) {
  return (cols % 4 == 0 && ld % 4 == 0 && ((uintptr_t)x % (4 * elem)) == 0) ? 4 : 1;
}

template <typename T>
static int launch_colsum(const T* x, int64_t rows, int64_t cols, int64_t ld, int64_t R, int cw, int vec, float* out,
                         hipStream_t st) {
  const int64_t groups = (cols + vec - 1) / vec;
  const int64_t slabs = rows > 0 ? (rows + R - 1) / R : 1;   // no rows: one slab that writes zeros
  const dim3 grid((unsigned)((groups + cw - 1) / cw), (unsigned)slabs);
  if (vec == 4)
    hipLaunchKernelGGL((k_colsum<T, 4>), grid, dim3(kColThreads), 0, st, x, rows, cols, ld, R, cw, out);
  else
    hipLaunchKernelGGL((k_colsum<T, 1>), grid, dim3(kColThreads), 0, st, x, rows, cols, ld, R, cw, out);
  return check_launch("asrn_column_sums");
}

}  // namespace asrn

using namespace asrn;

extern "C" int64_t asrn_column_sums_workspace(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return -1;
  const int64_t groups = (cols + 3) / 4;          // the slab count never grows with a narrower vector
  const int64_t g1 = cols;
  const int64_t s4 = slabs_of(rows, groups, col_lanes(groups, kColThreads));
  const int64_t s1 = slabs_of(rows, g1, col_lanes(g1, kColThreads));
  const int64_t s = s4 > s1 ? s4 : s1;
  if (s <= 1) return 0;
  return (s * cols * 4 + 255) / 256 * 256;
}

extern "C" int asrn_column_sums(const void* x, int32_t bf16, int64_t rows, int64_t cols, int64_t ld, float* out,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(rows >= 0 && cols >= 0 && ld >= cols && ld >= 1, "asrn_column_sums: bad sizes rows=%lld cols=%lld "
               "ld=%lld", (long long)rows, (long long)cols, (long long)ld);
  ASRN_REQUIRE(rows * ld < (int64_t(1) << 40) && cols < (int64_t(1) << 31),
               "asrn_column_sums: matrix too large (rows*ld=%lld)", (long long)(rows * ld));
  if (cols == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  const int elem = bf16 ? 2 : 4;
  const int vec = vec_of(x, cols, ld, elem);
  const int64_t groups = (cols + vec - 1) / vec;
  if (rows == 0)   // one slab of no rows: every column gets 0 (a kernel, not a memset: callers may capture this)
    return bf16 ? launch_colsum((const uint16_t*)x, 0, cols, ld, 1, col_lanes(groups, kColThreads), vec, out, st)
                : launch_colsum((const float*)x, 0, cols, ld, 1, col_lanes(groups, kColThreads), vec, out, st);
  const int cw = col_lanes(groups, kColThreads);
  const int64_t s = slabs_of(rows, groups, cw);
  const int64_t R = (rows + s - 1) / s;
  if (s == 1) {
    return bf16 ? launch_colsum((const uint16_t*)x, rows, cols, ld, R, cw, vec, out, st)
                : launch_colsum((const float*)x, rows, cols, ld, R, cw, vec, out, st);
  }
  const int64_t need = (s * cols * 4 + 255) / 256 * 256;
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= need && ((uintptr_t)workspace % 16) == 0,
               "asrn_column_sums: needs a 16-byte aligned workspace of %lld bytes (got %lld)", (long long)need,
               (long long)workspace_bytes);
  float* part = (float*)workspace;
  const int rc = bf16 ? launch_colsum((const uint16_t*)x, rows, cols, ld, R, cw, vec, part, st)
                      : launch_colsum((const float*)x, rows, cols, ld, R, cw, vec, part, st);
  if (rc) return rc;
  // the slab sums: one slab, more row lanes (at most 16 columns groups per workgroup)
  const int vec2 = cols % 4 == 0 ? 4 : 1;
  const int64_t groups2 = (cols + vec2 - 1) / vec2;
  return launch_colsum((const float*)part, s, cols, cols, s, col_lanes(groups2, 16), vec2, out, st);
}
