// a1 + a2 + a3: sign hash, stable bucket sort and the recent-mates index, for every row r = b*T + tau.
//
//   k_bucket_rows    one workgroup of 1024 threads per tile of up to 4096 positions of a row: the sign hash of its
//                    positions (their phi columns of table tau, read 4 rows x 16 columns per load instruction and
//                    turned into ids by ballots), then a stable LSD radix sort of the ids in LDS, 7 bits per pass:
//                    each wave owns 256 consecutive positions, ranks equal digits among its lanes by ballots and
//                    across its 4 rounds by a per-wave count in LDS, and one exclusive scan of the (digit, wave)
//                    counts places every group, so ties keep text order and the result equals
//                    torch.argsort(stable=True) bit for bit (reference asrn/estable.py:283). A row that is one tile
//                    also gets its ranks and windows there: the bucket start and end of every sorted index from a
//                    forward max scan and a backward min scan of the run boundaries.
//   k_bucket_merge   rows longer than a tile: merge passes of sorted runs (each element finds its place in the
//                    partner run by a binary search), ping-ponging between the output buffers.
//   k_bucket_finish  (longer rows) per sorted index: the rank of its position and win = min(C, mates before) |
//                    min(C, mates after) << 8, read off the sorted ids within C places on either side.
#include <limits.h>

#include "common.h"

namespace asrn {

constexpr int kMaxBits = 14;
constexpr int kTile = 4096;                        // positions per workgroup
constexpr int kPosBits = 12;                       // a position in the tile
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kSeg = kTile / kWaves;               // 256 consecutive positions per wave, 4 rounds of 64
constexpr int kRadixBits = 7;
constexpr int kBins = 1 << kRadixBits;
static_assert(kBins * kWaves == 2 * kThreads, "two (digit, wave) counts per thread in the scan");

// before / after of sorted index i among n sorted ids: same-bucket neighbours within C places on either side
template <class Ids>
__device__ __forceinline__ int window_of(const Ids& ks, int64_t i, int64_t n, int C) {
  const int id = ks[i];
  int before = C;
  if (i < C || ks[i - C] != id) {                  // the bucket starts after i - C: binary search for it
    int64_t lo = i >= C ? i - C + 1 : 0, hi = i;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (ks[mid] < id) lo = mid + 1; else hi = mid;
    }
    before = (int)(i - lo);
  }
  int after = C;
  if (i + C >= n || ks[i + C] != id) {             // the bucket ends before i + C
    int64_t lo = i, hi = i + C < n ? i + C : n;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (ks[mid] <= id) lo = mid + 1; else hi = mid;
    }
    after = (int)(lo - 1 - i);
  }
  return before | (after << 8);
}

struct GlobalIds {
  const int32_t* p;
  __device__ __forceinline__ int operator[](int64_t i) const { return p[i]; }
};

// the lanes whose 7-bit digit equals this lane's (every lane of the wavefront calls it)
__device__ __forceinline__ uint64_t match7(int d) {
  uint64_t m = __ballot(1);
#pragma unroll
  for (int j = 0; j < kRadixBits; ++j) {
    const bool bit = (d >> j) & 1;
    const uint64_t bj = __ballot(bit);
    m &= bit ? bj : ~bj;
  }
  return m;
}

// LDS reads and writes of one wavefront take effect in program order; the fence keeps the compiler from moving them
__device__ __forceinline__ void wave_lds_order() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// exclusive scans over the workgroup's threads (every thread calls them; wt: kWaves ints of LDS)
__device__ __forceinline__ int block_excl_sum(int a, int* wt) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  int inc = a;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int u = __shfl_up(inc, off, kWave);
    if (lane >= off) inc += u;
  }
  if (lane == kWave - 1) wt[wave] = inc;
  __syncthreads();
  int pre = 0;
  for (int w = 0; w < wave; ++w) pre += wt[w];
  __syncthreads();
  return pre + inc - a;
}
__device__ __forceinline__ int block_excl_max(int a, int* wt) {      // over the threads before this one
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  int inc = a;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int u = __shfl_up(inc, off, kWave);
    if (lane >= off) inc = max(inc, u);
  }
  if (lane == kWave - 1) wt[wave] = inc;
  __syncthreads();
  int pre = INT_MIN;
  for (int w = 0; w < wave; ++w) pre = max(pre, wt[w]);
  int ex = __shfl_up(inc, 1, kWave);
  if (lane == 0) ex = INT_MIN;
  __syncthreads();
  return max(pre, ex);
}
__device__ __forceinline__ int block_excl_min_rev(int a, int* wt) {  // over the threads after this one
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  int inc = a;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int u = __shfl_down(inc, off, kWave);
    if (lane + off < kWave) inc = min(inc, u);
  }
  if (lane == 0) wt[wave] = inc;
  __syncthreads();
  int post = INT_MAX;
  for (int w = wave + 1; w < kWaves; ++w) post = min(post, wt[w]);
  int ex = __shfl_down(inc, 1, kWave);
  if (lane == kWave - 1) ex = INT_MAX;
  __syncthreads();
  return min(post, ex);
}

// Grid (tiles, B * T), kThreads threads. Workgroup y takes table tau = y / B of batch row b = y % B, so with B a
// multiple of 8 every table of one batch row runs on one XCD and its phi rows are read into that XCD's L2 once.
// whole: the tile is the row, so rank and win are written here; otherwise the sorted tile's (id, position) pairs go
// to key_out / pos_out (the merge passes finish them).
__global__ __launch_bounds__(kThreads) void k_bucket_rows(const float* __restrict__ phi, int64_t B, int64_t L, int T,
                                                          int nb, int64_t stride, int C, bool whole,
                                                          int32_t* __restrict__ ids, int32_t* __restrict__ key_out,
                                                          int32_t* __restrict__ pos_out, int32_t* __restrict__ rank,
                                                          int32_t* __restrict__ win) {
  __shared__ uint32_t kb[2][kTile];                // (id << kPosBits | position in the tile)
  __shared__ int hist[kBins * kWaves];             // (digit, wave) counts, digit-major
  __shared__ int wt[kWaves];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int64_t b = blockIdx.y % B, tau = blockIdx.y / B;
  const int64_t r = b * T + tau;
  const int64_t t0 = (int64_t)blockIdx.x * kTile;
  const int n = (int)(L - t0 < kTile ? L - t0 : kTile);
  const int seg = kSeg * wave;                     // element (round q, lane) of this wave: position seg + 64 q + lane

  // sign hash: load u of round q reads position seg + 64 q + 4 u + (lane >> 4), column lane & 15; its ballot holds
  // the ids of 4 positions, one per 16-lane group; lane l keeps load l >> 2's group l & 3
  uint32_t k[4];
  {
    const float* base = phi + (b * L + t0) * stride + tau * nb;
    const int g = lane >> 4, c = lane & 15;
    // 32 loads of the wave in flight at a time: unconditional loads from clamped addresses (a load under a branch is
    // waited for before the branch joins), the out-of-range ones masked afterwards
    const int cc = c < nb ? c : nb - 1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float v[32];
      if (seg + kSeg <= n) {                         // the wave's positions are all in the row
        const float* p0 = base + (int64_t)(seg + 128 * h + g) * stride + cc;
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = p0[(int64_t)(4 * u) * stride];
      } else {
#pragma unroll
        for (int u = 0; u < 32; ++u) {
          const int e = seg + 128 * h + 4 * u + g;
          v[u] = base[(int64_t)(e < n ? e : n - 1) * stride + cc];
        }
      }
#pragma unroll
      for (int u = 0; u < 32; ++u)
        if (!(c < nb && seg + 128 * h + 4 * u + g < n)) v[u] = 0.f;
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
        const int q = 2 * h + qq;
        uint32_t id = 0;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const uint64_t m = __ballot(v[16 * qq + u] > 0.f);       // strict > 0 (nucleo:663)
          if ((lane >> 2) == u) id = (uint32_t)(m >> (16 * (lane & 3))) & 0xFFFFu;
        }
        const int e = seg + 64 * q + lane;
        if (e < n) ids[r * L + t0 + e] = (int32_t)id;
        // padding takes the largest id and sorts after every real position, in order
        k[q] = ((e < n ? id : (1u << nb) - 1u) << kPosBits) | (uint32_t)e;
      }
    }
  }

  // radix passes over the ids, least significant digit first
  int cur = 0;
  const int passes = (nb + kRadixBits - 1) / kRadixBits;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = kPosBits + pass * kRadixBits;
    const int bits = nb - pass * kRadixBits < kRadixBits ? nb - pass * kRadixBits : kRadixBits;
    hist[lane * kWaves + wave] = 0;
    hist[(lane + kWave) * kWaves + wave] = 0;
    wave_lds_order();
    int rk[4], dg[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int d = (int)((k[q] >> shift) & ((1u << bits) - 1u));
      const uint64_t peers = match7(d);
      const int base = hist[d * kWaves + wave];                    // this digit in the wave's earlier rounds
      rk[q] = base + __popcll(peers & ((1ull << lane) - 1ull));
      dg[q] = d;
      wave_lds_order();
      if (lane == __ffsll((unsigned long long)peers) - 1) hist[d * kWaves + wave] = base + __popcll(peers);
      wave_lds_order();
    }
    __syncthreads();
    const int h0 = hist[2 * tid], h1 = hist[2 * tid + 1];
    const int ex = block_excl_sum(h0 + h1, wt);
    hist[2 * tid] = ex;
    hist[2 * tid + 1] = ex + h0;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) kb[cur][hist[dg[q] * kWaves + wave] + rk[q]] = k[q];
    __syncthreads();
    if (pass + 1 < passes) {
#pragma unroll
      for (int q = 0; q < 4; ++q) k[q] = kb[cur][seg + 64 * q + lane];
      cur ^= 1;
    }
  }
  const uint32_t* srt = kb[cur];                   // the sorted tile; real positions first

  // outputs per sorted index i = 4 tid + q
  const int i0 = 4 * tid;
  uint32_t s4[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) s4[q] = srt[i0 + q];
  if (!whole) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (i0 + q < n) {
        key_out[r * L + t0 + i0 + q] = (int32_t)(s4[q] >> kPosBits);
        pos_out[r * L + t0 + i0 + q] = (int32_t)(t0 + (s4[q] & ((1u << kPosBits) - 1u)));
      }
    }
    return;
  }
  // bucket runs: start(i) = the last run start at or before i, end(i) = one past the last index of i's run
  const uint32_t prev = i0 > 0 ? srt[i0 - 1] >> kPosBits : 0u;
  const uint32_t next = i0 + 4 < kTile ? srt[i0 + 4] >> kPosBits : 0u;
  int ls[4], le[4];
  int run = INT_MIN;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = i0 + q;
    const uint32_t id = s4[q] >> kPosBits, pid = q ? s4[q - 1] >> kPosBits : prev;
    if (i == 0 || id != pid) run = i;
    ls[q] = run;
  }
  const int pre = block_excl_max(run, wt);
  int runb = INT_MAX;
#pragma unroll
  for (int q = 3; q >= 0; --q) {
    const int i = i0 + q;
    const uint32_t id = s4[q] >> kPosBits, nid = q < 3 ? s4[q + 1] >> kPosBits : next;
    if (i == n - 1 || (i < n - 1 && id != nid)) runb = i + 1;
    le[q] = runb;
  }
  const int post = block_excl_min_rev(runb, wt);
  uint32_t* by_pos = kb[cur ^ 1];                  // free: rank | win << kPosBits per position in the tile
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = i0 + q;
    if (i >= n) continue;
    const int start = max(pre, ls[q]), end = min(post, le[q]);
    const int before = min(C, i - start), after = min(C, end - 1 - i);
    key_out[r * L + i] = (int32_t)(s4[q] >> kPosBits);
    pos_out[r * L + i] = (int32_t)(s4[q] & ((1u << kPosBits) - 1u));
    by_pos[s4[q] & ((1u << kPosBits) - 1u)] = (uint32_t)i | ((uint32_t)(before | (after << 8)) << kPosBits);
  }
  __syncthreads();
  // consecutive lanes take consecutive positions: T-strided, not scattered, writes
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int t = q * kThreads + tid;
    if (t >= n) continue;
    const uint32_t x = by_pos[t];
    const int64_t o = (b * L + t) * T + tau;
    rank[o] = (int32_t)(x & ((1u << kPosBits) - 1u));
    win[o] = (int32_t)(x >> kPosBits);
  }
}

// merge sorted runs of w into runs of 2w; (key, position) pairs are unique
__global__ void k_bucket_merge(const int32_t* __restrict__ kin, const int32_t* __restrict__ pin,
                               int32_t* __restrict__ kout, int32_t* __restrict__ pout, int64_t rows, int64_t L,
                               int64_t w) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * L) return;
  const int64_t row = e / L, p = e % L;
  const int64_t run = p / w;
  const int64_t start = (run & ~(int64_t)1) * w;                      // first element of the merged pair
  const bool left = (run & 1) == 0;
  const int64_t ob = left ? start + w : start;                        // the partner run [ob, oe)
  const int64_t oe = left ? (start + 2 * w < L ? start + 2 * w : L) : start + w;
  const int64_t rb = row * L;
  const uint64_t me = ((uint64_t)(uint32_t)kin[e] << 32) | (uint32_t)pin[e];
  int64_t lo = ob, hi = oe > ob ? oe : ob;
  while (lo < hi) {                                                   // partner elements below mine
    const int64_t mid = (lo + hi) >> 1;
    const uint64_t km = ((uint64_t)(uint32_t)kin[rb + mid] << 32) | (uint32_t)pin[rb + mid];
    if (km < me) lo = mid + 1; else hi = mid;
  }
  const int64_t own = left ? p - start : p - (start + w);
  const int64_t out = rb + start + own + (lo - ob);
  kout[out] = kin[e];
  pout[out] = pin[e];
}

__global__ void k_bucket_finish(const int32_t* __restrict__ ids_sorted, const int32_t* __restrict__ order,
                                int64_t rows, int64_t L, int T, int C, int32_t* __restrict__ rank,
                                int32_t* __restrict__ win) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * L) return;
  const int64_t r = e / L, i = e % L;
  const int64_t t = order[e];
  if (t >= 0 && t < L) {                           // always true for a correct sort; keeps a bug from faulting
    const int64_t b = r / T, tau = r % T;
    const int64_t o = (b * L + t) * T + tau;
    rank[o] = (int32_t)i;
    win[o] = window_of(GlobalIds{ids_sorted + r * L}, i, L, C);
  }
}

}  // namespace asrn

extern "C" int asrn_bucket_sort(const float* phi, int64_t B, int64_t L, int32_t T, int32_t nb, int64_t phi_stride,
                                int32_t C, int32_t* ids, int32_t* order, int32_t* ids_sorted, int32_t* rank,
                                int32_t* win, void* stream) {
  using namespace asrn;
  ASRN_REQUIRE(nb >= 1 && nb <= kMaxBits, "asrn_bucket_sort: n_bits must be in [1, %d] (got %d)", kMaxBits, nb);
  ASRN_REQUIRE(B >= 0 && L >= 0 && T >= 1 && T <= 32, "asrn_bucket_sort: bad sizes B=%lld L=%lld T=%d (T <= 32)",
               (long long)B, (long long)L, T);
  ASRN_REQUIRE(L < (int64_t(1) << 31), "asrn_bucket_sort: L=%lld too long", (long long)L);
  ASRN_REQUIRE(phi_stride >= (int64_t)T * nb, "asrn_bucket_sort: phi row stride %lld < T*nb = %d",
               (long long)phi_stride, T * nb);
  ASRN_REQUIRE(C >= 1 && C <= 255, "asrn_bucket_sort: window C=%d must be in [1, 255]", C);
  if (B == 0 || L == 0) return 0;
  ASRN_REQUIRE(phi && ids && order && ids_sorted && rank && win, "asrn_bucket_sort: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const int64_t rows = B * T;
  const int64_t tiles = (L + kTile - 1) / kTile;
  int passes = 0;
  for (int64_t w = kTile; w < L; w <<= 1) ++passes;
  // the merge passes ping-pong between (ids_sorted, order) and (rank, win), which the finish overwrites last: start
  // in the buffer that makes the final pass land in (ids_sorted, order)
  int32_t* bufk[2] = {ids_sorted, rank};
  int32_t* bufp[2] = {order, win};
  int cur = passes % 2;
  hipLaunchKernelGGL(k_bucket_rows, dim3((unsigned)tiles, (unsigned)rows), dim3(kThreads), 0, st, phi, B, L, (int)T,
                     (int)nb, phi_stride, (int)C, tiles == 1, ids, bufk[cur], bufp[cur], rank, win);
  if (check_launch("asrn_bucket_sort/rows")) return 1;
  const int threads = 256;
  const unsigned blocks = (unsigned)((rows * L + threads - 1) / threads);
  for (int64_t w = kTile; w < L; w <<= 1) {
    hipLaunchKernelGGL(k_bucket_merge, dim3(blocks), dim3(threads), 0, st, bufk[cur], bufp[cur], bufk[cur ^ 1],
                       bufp[cur ^ 1], rows, L, w);
    if (check_launch("asrn_bucket_sort/merge")) return 1;
    cur ^= 1;
  }
  if (tiles == 1) return 0;                        // the row kernel wrote rank and win
  hipLaunchKernelGGL(k_bucket_finish, dim3(blocks), dim3(threads), 0, st, ids_sorted, order, rows, L, (int)T, (int)C,
                     rank, win);
  return check_launch("asrn_bucket_sort/finish");
}
