// a1 + a2: sign hash and stable bucket sort, one workgroup per row r = b*T + tau.
//
// The row's ids are a 14-bit counting sort staged in LDS: a histogram of the 2^nb buckets (LDS integer atomics:
// counts do not depend on order), an exclusive scan, then a stable scatter in text order. Stability inside a wave
// comes from matching the lanes with the same key (nb ballots); across the 16 waves of a tile the waves take their
// bucket offsets one after the other, so ties always land in text order. Matches torch.argsort(stable=True) bit for
// bit (reference asrn/estable.py:283).
#include "common.h"

namespace asrn {

constexpr int kSortThreads = 1024;
constexpr int kMaxBits = 14;

// In-place exclusive scan of n ints in LDS by 1024 threads.
__device__ void block_exclusive_scan(int* data, int n, int* wave_tot) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (n + kSortThreads - 1) / kSortThreads;
  const int lo = min(tid * per, n), hi = min(lo + per, n);
  int s = 0;
  for (int i = lo; i < hi; ++i) s += data[i];
  int v = s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  if (lane == 63) wave_tot[wave] = v;
  __syncthreads();
  if (wave == 0) {
    const int w = lane < 16 ? wave_tot[lane] : 0;
    int x = w;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const int u = __shfl_up(x, off, 64);
      if (lane >= off) x += u;
    }
    if (lane < 16) wave_tot[lane] = x - w;
  }
  __syncthreads();
  int run = wave_tot[wave] + v - s;
  for (int i = lo; i < hi; ++i) {
    const int c = data[i];
    data[i] = run;
    run += c;
  }
  __syncthreads();
}

__global__ __launch_bounds__(kSortThreads) void k_bucket_sort(const float* __restrict__ phi, int64_t L, int T, int nb,
                                                              int64_t stride, int C, int32_t* __restrict__ ids,
                                                              int32_t* __restrict__ order,
                                                              int32_t* __restrict__ ids_sorted,
                                                              int32_t* __restrict__ rank, int32_t* __restrict__ win) {
  __shared__ int cnt[1 << kMaxBits];
  __shared__ int first[(1 << kMaxBits) + 1];     // bucket starts (cnt advances during the scatter)
  __shared__ int wave_tot[16];
  const int r = blockIdx.x;
  const int b = r / T, tau = r % T;
  const int nbins = 1 << nb;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  for (int i = tid; i < nbins; i += kSortThreads) cnt[i] = 0;
  __syncthreads();

  const float* base = phi + (int64_t)b * L * stride + (int64_t)tau * nb;
  int32_t* idr = ids + (int64_t)r * L;
  for (int64_t t = tid; t < L; t += kSortThreads) {
    const float* row = base + t * stride;
    int id = 0;
    for (int j = 0; j < nb; ++j) id |= (row[j] > 0.f ? 1 : 0) << j;   // strict > 0 (nucleo:663)
    idr[t] = id;
    atomicAdd(&cnt[id], 1);
  }
  __syncthreads();
  block_exclusive_scan(cnt, nbins, wave_tot);
  for (int i = tid; i < nbins; i += kSortThreads) first[i] = cnt[i];
  if (tid == 0) first[nbins] = (int)L;
  __syncthreads();

  int32_t* ordr = order + (int64_t)r * L;
  int32_t* idsr = ids_sorted + (int64_t)r * L;
  for (int64_t t0 = 0; t0 < L; t0 += kSortThreads) {
    const int64_t t = t0 + tid;
    const bool valid = t < L;
    const int id = valid ? idr[t] : 0;       // this thread wrote idr[t] above
    const uint64_t peers = match_key(id, nb, valid);
    const int below = __popcll(peers & ((1ull << lane) - 1ull));
    const int together = __popcll(peers);
    const bool last = valid && (peers >> lane) == 1ull;
    int dest = 0;
    for (int w = 0; w < kSortThreads / kWave; ++w) {
      if (wave == w && valid) {
        const int start = cnt[id];
        dest = start + below;
        if (last) cnt[id] = start + together;
      }
      __syncthreads();
    }
    if (valid && dest >= 0 && dest < L) {       // always true for a correct sort; keeps a bug from faulting
      ordr[dest] = (int32_t)t;
      idsr[dest] = id;
      const int64_t o = ((int64_t)b * L + t) * T + tau;
      rank[o] = dest;
      const int before = dest - first[id];               // earlier positions in the bucket
      const int after = first[id + 1] - 1 - dest;          // later positions in the bucket
      win[o] = min(before, C) | (min(after, C) << 8);
    }
  }
}

}  // namespace asrn

extern "C" int asrn_bucket_sort(const float* phi, int64_t B, int64_t L, int32_t T, int32_t nb, int64_t phi_stride,
                                int32_t C, int32_t* ids, int32_t* order, int32_t* ids_sorted, int32_t* rank,
                                int32_t* win, void* stream) {
  ASRN_REQUIRE(nb >= 1 && nb <= asrn::kMaxBits, "asrn_bucket_sort: n_bits must be in [1, %d] (got %d)",
               asrn::kMaxBits, nb);
  ASRN_REQUIRE(B >= 0 && L >= 0 && T >= 1, "asrn_bucket_sort: bad sizes B=%lld L=%lld T=%d", (long long)B,
               (long long)L, T);
  ASRN_REQUIRE(L < (int64_t(1) << 31), "asrn_bucket_sort: L=%lld too long", (long long)L);
  ASRN_REQUIRE(phi_stride >= (int64_t)T * nb, "asrn_bucket_sort: phi row stride %lld < T*nb = %d",
               (long long)phi_stride, T * nb);
  ASRN_REQUIRE(C >= 1 && C <= 255, "asrn_bucket_sort: window C=%d must be in [1, 255]", C);
  if (B == 0 || L == 0) return 0;
  ASRN_REQUIRE(phi && ids && order && ids_sorted && rank && win, "asrn_bucket_sort: null pointer");
  hipLaunchKernelGGL(asrn::k_bucket_sort, dim3((unsigned)(B * T)), dim3(asrn::kSortThreads), 0,
                     (hipStream_t)stream, phi, L, (int)T, (int)nb, phi_stride, (int)C, ids, order, ids_sorted, rank,
                     win);
  return asrn::check_launch("asrn_bucket_sort");
}
