// Bitonic sort of one tile per workgroup, for the row sorts (bucket ids, n-gram keys).
//
// A tile of n elements (a power of two, 4 <= n <= 4096) is held 4 per thread, element e = 4 tid + r, by n / 4
// threads. Each (k, j) stage of the network compares e with e ^ j: distances 1 and 2 stay inside a thread's
// registers, 4 .. 128 are a lane exchange inside the wavefront (threads tid ^ j / 4), and only 256 and up go through
// LDS with a barrier (10 of the 78 stages at n = 4096). Elements are unique under the ordering used here (the keys
// carry their position), so the sort is stable by construction.
#pragma once
#include "common.h"

namespace asrn {

// (bucket id << 32 | position): one 64-bit compare
struct SortU64 {
  uint64_t k;
  __device__ __forceinline__ bool lt(const SortU64& o) const { return k < o.k; }
  __device__ __forceinline__ SortU64 xor_lane(int m) const {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)k, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(k >> 32), m, 64);
    return SortU64{((uint64_t)hi << 32) | lo};
  }
};

// (64-bit key code, 32-bit position)
struct SortKI {
  uint64_t k;
  uint32_t i;
  __device__ __forceinline__ bool lt(const SortKI& o) const { return k < o.k || (k == o.k && i < o.i); }
  __device__ __forceinline__ SortKI xor_lane(int m) const {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)k, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(k >> 32), m, 64);
    const uint32_t ii = (uint32_t)__shfl_xor((int)i, m, 64);
    return SortKI{((uint64_t)hi << 32) | lo, ii};
  }
};

template <class E>
__device__ __forceinline__ void cmp_swap(E& a, E& b, bool ascending) {
  const bool swap = ascending ? b.lt(a) : a.lt(b);
  if (swap) {
    const E t = a;
    a = b;
    b = t;
  }
}

// x: this thread's 4 elements (in tile order on entry, sorted ascending across the tile on exit); lds: n elements.
// Every thread of the block calls it (n = 4 * blockDim.x).
template <class E>
__device__ void block_bitonic_sort(E (&x)[4], E* lds, int n) {
  const int tid = threadIdx.x;
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 256) {
#pragma unroll
        for (int r = 0; r < 4; ++r) lds[4 * tid + r] = x[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int e = 4 * tid + r;
          const E p = lds[e ^ j];
          const bool asc = (e & k) == 0, lower = (e & j) == 0;
          const bool take = lower == asc ? p.lt(x[r]) : x[r].lt(p);     // keep the min or the max of the pair
          if (take) x[r] = p;
        }
        __syncthreads();
      } else if (j >= 4) {
        const int m = j >> 2;
        const bool asc = ((tid << 2) & k) == 0, lower = (tid & m) == 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const E p = x[r].xor_lane(m);
          const bool take = lower == asc ? p.lt(x[r]) : x[r].lt(p);
          if (take) x[r] = p;
        }
      } else if (j == 2) {
        const bool asc = ((tid << 2) & k) == 0;
        cmp_swap(x[0], x[2], asc);
        cmp_swap(x[1], x[3], asc);
      } else {
        // k == 2 alternates direction per pair of elements; k >= 4 is uniform across the thread's four
        cmp_swap(x[0], x[1], ((4 * tid) & k) == 0);
        cmp_swap(x[2], x[3], ((4 * tid + 2) & k) == 0);
      }
    }
  }
}

}  // namespace asrn
