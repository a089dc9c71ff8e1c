// A local block's generation step whose last kernel was left to the next kernel that reads its output (the block step
// asrn_block_step_ex with finish = 0): its output is h1 + (the sum of its second feed-forward product's depth splits +
// b2), and its LayerNorm1 row z enters its ring at slot pos mod (k - 1) (the block step's k_finish_res, reference
// nucleo:969-1014 through 1811-1814). The next block's first row kernel or the generation step's producer of an ASRN
// layer finishes it; both form each output value with the expression k_finish_res uses, so the bits are the same.
// Also the block step's workspace layout, which says where those partials are.
#pragma once

#include "common.h"

namespace asrn {

constexpr int kMaxSplits = 16;               // depth splits of a block step's products, at most

// depth splits of a product with depth K: each wavefront's share at most 64 columns (one round of loads)
inline int splits_for(int K) {
  const int s = (K + 4 * 64 - 1) / (4 * 64);
  return s < 1 ? 1 : (s > kMaxSplits ? kMaxSplits : s);
}

// The block step's workspace, in floats: the conv product's partials (kMaxSplits, B, d), the hidden layer (B, ff), the
// second feed-forward product's partials (splits_for(ff), B, d)
inline int64_t block_workspace_floats(int64_t B, int d, int ff) {
  return B * ((int64_t)kMaxSplits * d + (int64_t)ff + (int64_t)splits_for(ff) * d);
}
inline float* block_hidden(void* ws, int64_t B, int d) { return (float*)ws + (int64_t)kMaxSplits * B * d; }
inline float* block_second_parts(void* ws, int64_t B, int d, int ff) { return block_hidden(ws, B, d) + B * ff; }

struct Pending {
  const float* part;  // (splits, B, d), null: no pending block
  int splits;
  const float* bias; const float* h1; const float* z;
  float* ring;        // its ring (B, d, km1) takes z at slot pos mod km1
  int km1;
  float* out;         // its output, written here
};

// The row kernels issue every load before its first use as unconditional loads: columns past d read column d - 1, and
// splits past `splits` re-read the last one, real addresses whose values are not used (a guarded load becomes a branch
// the compiler does not schedule across, and each such load then waits on its own).

// the S (>= splits) partial values of one column, split stride `stride`
template <int S>
__device__ __forceinline__ void split_loads(const float* p, int splits, int64_t stride, float (&v)[S]) {
#pragma unroll
  for (int s = 0; s < S; ++s) v[s] = p[(int64_t)(s < splits ? s : splits - 1) * stride];
}
// their sum in split order (the splits past `splits` add nothing)
template <int S>
__device__ __forceinline__ float split_total(const float (&v)[S], int splits) {
  float y = 0.f;
#pragma unroll
  for (int s = 0; s < S; ++s) y += s < splits ? v[s] : 0.f;
  return y;
}

// the load-count instance for `splits` splits
inline int split_cap(int splits) { return splits <= 4 ? 4 : (splits <= 8 ? 8 : 16); }

}  // namespace asrn
