// a1 + a2 + a3: sign hash, stable bucket sort and the recent-mates index, for every row r = b*T + tau.
//
//   k_bucket_ids     the sign hash: one thread per position computes every table's id from its phi row.
//   k_bucket_tile    one workgroup per tile of up to 4096 positions of a row: a stable LSD radix sort of the ids in
//                    LDS (7 bits per pass, ranks by wave ballots), so ties keep text order and the result equals
//                    torch.argsort(stable=True) bit for bit (reference asrn/estable.py:283); a row that is one tile
//                    also gets its ranks and windows there, from the sorted ids in LDS.
//   k_bucket_merge   rows longer than a tile: merge passes of sorted runs (each element finds its place in the
//                    partner run by a binary search), ping-ponging between the output buffers.
//   k_bucket_finish  (longer rows) per sorted index: the rank of its position and win = min(C, mates before) |
//                    min(C, mates after) << 8, read off the sorted ids within C places on either side.
#include "common.h"

namespace asrn {

constexpr int kMaxBits = 14;
constexpr int kTileMax = 4096;

// Tile length for rows of L: a power of two, at most kTileMax, at least 4. Shorter tiles mean more workgroups and
// more merge passes.
static int bucket_tile(int64_t L) {
  int tile = 4;
  while (tile < L && tile < kTileMax) tile <<= 1;
  return tile;
}

// The sign hash for kIdTokens positions per workgroup: their phi rows (T*nb floats each) are read with consecutive
// threads on consecutive floats and kept as sign bytes in LDS; then one thread per (table, position) assembles the
// id, positions fastest, so the ids rows are written contiguously.
constexpr int kIdTokens = 16;
constexpr int kIdThreads = 256;

__global__ __launch_bounds__(kIdThreads) void k_bucket_ids(const float* __restrict__ phi, int64_t B, int64_t L, int T,
                                                           int nb, int64_t stride, int32_t* __restrict__ ids) {
  __shared__ uint8_t sgn[kIdTokens * 32 * kMaxBits];
  const int tnb = T * nb;
  const int64_t e0 = (int64_t)blockIdx.x * kIdTokens, n = B * L;
  constexpr int U = 8;                             // loads in flight per thread
  for (int k0 = 0; k0 < kIdTokens * tnb; k0 += kIdThreads * U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + u * kIdThreads + threadIdx.x;
      const int row = k / tnb, col = k - row * tnb;
      const int64_t e = e0 + row;
      v[u] = (k < kIdTokens * tnb && e < n) ? phi[e * stride + col] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + u * kIdThreads + threadIdx.x;
      if (k < kIdTokens * tnb) sgn[k] = v[u] > 0.f ? 1 : 0;        // strict > 0 (nucleo:663)
    }
  }
  __syncthreads();
  for (int p = threadIdx.x; p < kIdTokens * T; p += kIdThreads) {
    const int tau = p / kIdTokens, row = p - tau * kIdTokens;
    const int64_t e = e0 + row;
    if (e < n) {
      uint32_t id = 0;
      for (int j = 0; j < nb; ++j) id |= (uint32_t)sgn[row * tnb + tau * nb + j] << j;
      const int64_t b = e / L, t = e % L;
      ids[(b * T + tau) * L + t] = (int32_t)id;
    }
  }
}

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

// One tile of a row (up to 4096 positions, 1024 threads): a stable LSD radix sort of the ids in LDS, 7 bits per pass.
// A pass visits the tile in 4 rounds of 1024 consecutive positions; inside a round each wave ranks its lanes with
// equal digits by ballots (match_key), and an exclusive scan of the (digit, round, wave) group sizes gives every group
// its output start, so equal digits keep their order and the result equals torch.argsort(stable=True). When the tile
// is the whole row (`whole`), also the rank and window of every position, from the sorted ids in LDS.
constexpr int kRadixBits = 7;
constexpr int kRadixBins = 1 << kRadixBits;
constexpr int kTileThreads = 1024;
constexpr int kRounds = kTileMax / kTileThreads;
constexpr int kTileWaves = kTileThreads / kWave;
constexpr int kGroups = kRadixBins * kRounds * kTileWaves;   // 8192 (digit, round, wave) groups
constexpr int kPerThread = kGroups / kTileThreads;

struct LdsPacked {                                 // (id << 16 | position in the tile) -> id
  const uint32_t* p;
  __device__ __forceinline__ int operator[](int64_t i) const { return (int)(p[i] >> 16); }
};

__global__ __launch_bounds__(kTileThreads) void k_bucket_tile(const int32_t* __restrict__ ids, int64_t L, int T,
                                                              int nb, int tile, int C, bool whole,
                                                              int32_t* __restrict__ key_out,
                                                              int32_t* __restrict__ pos_out,
                                                              int32_t* __restrict__ rank, int32_t* __restrict__ win) {
  __shared__ uint32_t kbuf[2][kTileMax];
  __shared__ int cnt[kGroups];
  __shared__ int wave_tot[kTileWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t r = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * tile;
  const int n = (int)(L - t0 < tile ? L - t0 : tile);
  for (int e = tid; e < kTileMax; e += kTileThreads)   // padding takes the largest id and sorts last, in order
    kbuf[0][e] = e < n ? ((uint32_t)ids[r * L + t0 + e] << 16) | (uint32_t)e : (0xFFFFu << 16) | (uint32_t)e;
  int cur = 0;
  const int passes = (nb + kRadixBits - 1) / kRadixBits;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = 16 + pass * kRadixBits;
    const int bits = nb - pass * kRadixBits < kRadixBits ? nb - pass * kRadixBits : kRadixBits;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) cnt[tid * kPerThread + i] = 0;
    __syncthreads();                               // kbuf[cur] written, counts cleared
    uint32_t v[kRounds];
    int dig[kRounds], below[kRounds];
#pragma unroll
    for (int q = 0; q < kRounds; ++q) {
      v[q] = kbuf[cur][q * kTileThreads + tid];
      dig[q] = (int)((v[q] >> shift) & ((1u << bits) - 1u));
      const uint64_t peers = match_key(dig[q], bits, true);
      below[q] = __popcll(peers & ((1ull << lane) - 1ull));
      if ((peers >> lane) == 1ull) cnt[(dig[q] * kRounds + q) * kTileWaves + wave] = __popcll(peers);
    }
    __syncthreads();
    // exclusive scan of the 8192 group sizes: kPerThread consecutive per thread, then across threads
    int local[kPerThread];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      local[i] = cnt[tid * kPerThread + i];
      sum += local[i];
    }
    int incl = sum;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int u = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += u;
    }
    if (lane == kWave - 1) wave_tot[wave] = incl;
    __syncthreads();
    int wave_base = 0;
    for (int w = 0; w < wave; ++w) wave_base += wave_tot[w];
    int run = wave_base + incl - sum;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      cnt[tid * kPerThread + i] = run;
      run += local[i];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kRounds; ++q)
      kbuf[cur ^ 1][cnt[(dig[q] * kRounds + q) * kTileWaves + wave] + below[q]] = v[q];
    cur ^= 1;
    __syncthreads();                               // before the next pass clears the counts
  }
  for (int i = tid; i < n; i += kTileThreads) {    // the sorted tile has its real elements first
    const uint32_t x = kbuf[cur][i];
    key_out[r * L + t0 + i] = (int32_t)(x >> 16);
    pos_out[r * L + t0 + i] = (int32_t)(t0 + (x & 0xFFFFu));
  }
  if (!whole) return;
  const int64_t b = r / T, tau = r % T;
  for (int i = tid; i < n; i += kTileThreads) {
    const int64_t t = (int64_t)(kbuf[cur][i] & 0xFFFFu);
    const int64_t o = (b * L + t) * T + tau;
    rank[o] = i;
    win[o] = window_of(LdsPacked{kbuf[cur]}, i, n, C);
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
  const int tile = bucket_tile(L);
  const int64_t tiles = (L + tile - 1) / tile;
  int passes = 0;
  for (int64_t w = tile; w < L; w <<= 1) ++passes;
  // the merge passes ping-pong between (ids_sorted, order) and (rank, win), which the finish overwrites last: start
  // in the buffer that makes the final pass land in (ids_sorted, order)
  int32_t* bufk[2] = {ids_sorted, rank};
  int32_t* bufp[2] = {order, win};
  int cur = passes % 2;
  const int threads = 256;
  const unsigned blocks = (unsigned)((rows * L + threads - 1) / threads);
  hipLaunchKernelGGL(k_bucket_ids, dim3((unsigned)((B * L + kIdTokens - 1) / kIdTokens)), dim3(kIdThreads), 0, st, phi,
                     B, L, (int)T, (int)nb, phi_stride, ids);
  hipLaunchKernelGGL(k_bucket_tile, dim3((unsigned)tiles, (unsigned)rows), dim3(kTileThreads), 0, st, ids, L, (int)T,
                     (int)nb, tile, (int)C, tiles == 1, bufk[cur], bufp[cur], rank, win);
  if (check_launch("asrn_bucket_sort/tile")) return 1;
  for (int64_t w = tile; w < L; w <<= 1) {
    hipLaunchKernelGGL(k_bucket_merge, dim3(blocks), dim3(threads), 0, st, bufk[cur], bufp[cur], bufk[cur ^ 1],
                       bufp[cur ^ 1], rows, L, w);
    if (check_launch("asrn_bucket_sort/merge")) return 1;
    cur ^= 1;
  }
  if (tiles == 1) return 0;                        // the tile kernel wrote rank and win
  hipLaunchKernelGGL(k_bucket_finish, dim3(blocks), dim3(threads), 0, st, ids_sorted, order, rows, L, (int)T, (int)C,
                     rank, win);
  return check_launch("asrn_bucket_sort/finish");
}
