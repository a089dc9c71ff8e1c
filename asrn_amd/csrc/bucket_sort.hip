// a1 + a2 + a3: sign hash, stable bucket sort and the recent-mates index, for every row r = b*T + tau.
//
//   k_bucket_rows<R>  one workgroup of 1024 threads per tile of up to 1024 R positions of a row: the sign hash of its
//                     positions (their phi columns of table tau, read 4 rows x 16 columns per load instruction and
//                     turned into ids by ballots; with no phi, the ids the fused hash producer already wrote), then a
//                     stable LSD radix sort of the ids in LDS, 7 bits per pass:
//                     each wave owns 64 R consecutive positions, ranks equal digits among its lanes by ballots and
//                     across its R rounds by a per-wave count in LDS, and one exclusive scan of the (digit, wave)
//                     counts places every group, so ties keep text order and the result equals
//                     torch.argsort(stable=True) bit for bit (reference asrn/estable.py:283). A row that is one tile
//                     also gets its ranks and windows there: the bucket start and end of every sorted index from a
//                     forward max scan and a backward min scan of the run boundaries.
//   k_bucket_place    rows of 1025 to 4096 positions: the row's chunks of 1024 are sorted by k_bucket_rows<1> (a
//                     workgroup each, so a row spreads over up to 4 CUs), and then every sorted element finds its
//                     place in the row: with the row's sorted chunks in LDS, binary searches give, in each chunk,
//                     the count of ids below its own and up to its own; earlier chunks' equal ids go first (they hold
//                     earlier positions), so its sorted index is its index in its chunk plus those counts, and the
//                     sums over all chunks are its bucket's start and end, which give the window.
//   k_bucket_merge    rows longer than 4096: merge passes of sorted tiles of 4096 (each element finds its place in
//                     the partner run by a binary search), ping-ponging between the output buffers.
//   k_bucket_finish   (those rows) per sorted index: the rank of its position and win = min(C, mates before) |
//                     min(C, mates after) << 8, read off the sorted ids within C places on either side.
#include <limits.h>

#include "common.h"

namespace asrn {

constexpr int kMaxBits = 14;
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kChunk = kThreads;                   // R = 1: a round of 64 positions per wave
constexpr int kTile = 4 * kThreads;                // R = 4: the tiles of rows longer than kTile
constexpr int kPlaceChunks = kTile / kChunk;       // rows of up to this many chunks take the place kernel
constexpr int kPosBits = 12;                       // a position in a tile
constexpr int kRadixBits = 7;
constexpr int kBins = 1 << kRadixBits;
static_assert(kBins * kWaves == 2 * kThreads, "two (digit, wave) counts per thread in the scan");
static_assert(kTile <= (1 << kPosBits), "tile positions fit the key's position bits");

// what k_bucket_rows writes: the whole row's outputs (the tile is the row); the sorted tile's (id, position) pairs
// for the merge passes; or the sorted tile's packed keys (id << kPosBits | position in the tile) for k_bucket_place
enum BucketOut { kOutWhole = 0, kOutPairs = 1, kOutPacked = 2 };

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

// Grid of tiles x rows workgroups, kThreads threads, tiles of 1024 R positions; row y takes table tau = y / B of batch
// row b = y % B. by_row (the chunks for k_bucket_place): the grid is xcd_grid(B * T, tiles) and every tile of row y
// runs on XCD y % 8, so with B a multiple of 8 a batch row's tables and tiles share one XCD, which reads its phi rows
// into its L2 once and where k_bucket_place, on the same map, finds the sorted tiles. Otherwise workgroup i takes tile
// i % tiles of row i / tiles, so the tables of one stretch of positions share an XCD.
// out: BucketOut (kOutPacked writes the tile's kTileR keys, padding included, at packed + r * ldp + the tile's start).
template <int R>
__global__ __launch_bounds__(kThreads) void k_bucket_rows(const float* __restrict__ phi, int64_t B, int64_t L, int T,
                                                          int nb, int64_t stride, int C, int out,
                                                          int32_t* __restrict__ ids, int32_t* __restrict__ key_out,
                                                          int32_t* __restrict__ pos_out, int32_t* __restrict__ rank,
                                                          int32_t* __restrict__ win, uint32_t* __restrict__ packed,
                                                          int64_t ldp, int tiles, bool by_row) {
  constexpr int kTileR = kChunk * R;
  constexpr int kSeg = 64 * R;                     // consecutive positions per wave, R rounds of 64
  constexpr int RB = R >= 2 ? 2 : 1;               // rounds per batch of hash loads (16 loads a round)
  __shared__ uint32_t kb[2][kTileR];               // (id << kPosBits | position in the tile)
  __shared__ int hist[kBins * kWaves];             // (digit, wave) counts, digit-major
  __shared__ int wt[kWaves];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  int tile;
  int64_t y;
  if (by_row) {
    xcd_chunk_row(tiles, &tile, &y);
    if (y >= B * T) return;
  } else {
    tile = (int)(blockIdx.x % tiles);
    y = blockIdx.x / tiles;
  }
  const int64_t b = y % B, tau = y / B;
  const int64_t r = b * T + tau;
  const int64_t t0 = (int64_t)tile * kTileR;
  const int n = (int)(L - t0 < kTileR ? L - t0 : kTileR);
  const int seg = kSeg * wave;                     // element (round q, lane) of this wave: position seg + 64 q + lane

  // sign hash: load u of a batch starting at e0 reads position e0 + 4 u + (lane >> 4), column lane & 15; its ballot
  // holds the ids of 4 positions, one per 16-lane group; lane l keeps load l >> 2's group l & 3
  uint32_t k[R];
  if (!phi) {                                      // the hash producer wrote the ids: read them
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const int e = seg + 64 * q + lane;
      const uint32_t id = e < n ? (uint32_t)ids[r * L + t0 + e] : 0u;
      k[q] = ((e < n ? id : (1u << nb) - 1u) << kPosBits) | (uint32_t)e;
    }
  } else {
    const float* base = phi + (b * L + t0) * stride + tau * nb;
    const int g = lane >> 4, c = lane & 15;
    // every load of a batch in flight at once: unconditional loads from clamped addresses (a load under a branch is
    // waited for before the branch joins), the out-of-range ones masked afterwards
    const int cc = c < nb ? c : nb - 1;
#pragma unroll
    for (int h = 0; h < R / RB; ++h) {
      const int e0 = seg + 64 * RB * h;
      float v[16 * RB];
      if (seg + kSeg <= n) {                         // the wave's positions are all in the row
        const float* p0 = base + (int64_t)(e0 + g) * stride + cc;
#pragma unroll
        for (int u = 0; u < 16 * RB; ++u) v[u] = p0[(int64_t)(4 * u) * stride];
      } else {
#pragma unroll
        for (int u = 0; u < 16 * RB; ++u) {
          const int e = e0 + 4 * u + g;
          v[u] = base[(int64_t)(e < n ? e : n - 1) * stride + cc];
        }
      }
#pragma unroll
      for (int u = 0; u < 16 * RB; ++u)
        if (!(c < nb && e0 + 4 * u + g < n)) v[u] = 0.f;
#pragma unroll
      for (int qq = 0; qq < RB; ++qq) {
        const int q = RB * h + qq;
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
    int rk[R], dg[R];
#pragma unroll
    for (int q = 0; q < R; ++q) {
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
    for (int q = 0; q < R; ++q) kb[cur][hist[dg[q] * kWaves + wave] + rk[q]] = k[q];
    __syncthreads();
    if (pass + 1 < passes) {
#pragma unroll
      for (int q = 0; q < R; ++q) k[q] = kb[cur][seg + 64 * q + lane];
      cur ^= 1;
    }
  }
  const uint32_t* srt = kb[cur];                   // the sorted tile; real positions first

  // outputs per sorted index i = R tid + q
  const int i0 = R * tid;
  uint32_t s4[R];
#pragma unroll
  for (int q = 0; q < R; ++q) s4[q] = srt[i0 + q];
  if (out == kOutPacked) {
#pragma unroll
    for (int q = 0; q < R; ++q) packed[r * ldp + t0 + i0 + q] = s4[q];
    return;
  }
  if (out == kOutPairs) {
#pragma unroll
    for (int q = 0; q < R; ++q) {
      if (i0 + q < n) {
        key_out[r * L + t0 + i0 + q] = (int32_t)(s4[q] >> kPosBits);
        pos_out[r * L + t0 + i0 + q] = (int32_t)(t0 + (s4[q] & ((1u << kPosBits) - 1u)));
      }
    }
    return;
  }
  // bucket runs: start(i) = the last run start at or before i, end(i) = one past the last index of i's run
  const uint32_t prev = i0 > 0 ? srt[i0 - 1] >> kPosBits : 0u;
  const uint32_t next = i0 + R < kTileR ? srt[i0 + R] >> kPosBits : 0u;
  int ls[R], le[R];
  int run = INT_MIN;
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int i = i0 + q;
    const uint32_t id = s4[q] >> kPosBits, pid = q ? s4[q - 1] >> kPosBits : prev;
    if (i == 0 || id != pid) run = i;
    ls[q] = run;
  }
  const int pre = block_excl_max(run, wt);
  int runb = INT_MAX;
#pragma unroll
  for (int q = R - 1; q >= 0; --q) {
    const int i = i0 + q;
    const uint32_t id = s4[q] >> kPosBits, nid = q < R - 1 ? s4[q + 1] >> kPosBits : next;
    if (i == n - 1 || (i < n - 1 && id != nid)) runb = i + 1;
    le[q] = runb;
  }
  const int post = block_excl_min_rev(runb, wt);
  uint32_t* by_pos = kb[cur ^ 1];                  // free: rank | win << kPosBits per position in the tile
#pragma unroll
  for (int q = 0; q < R; ++q) {
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
  for (int q = 0; q < R; ++q) {
    const int t = q * kThreads + tid;
    if (t >= n) continue;
    const uint32_t x = by_pos[t];
    const int64_t o = (b * L + t) * T + tau;
    rank[o] = (int32_t)(x & ((1u << kPosBits) - 1u));
    win[o] = (int32_t)(x >> kPosBits);
  }
}

// For each of the kPlaceChunks sorted runs of kChunk keys at s + q kChunk: lb[q] = its keys below lo, ub[q] = below
// hi. Branch-free lower bounds with a fixed trip count (the interval halves whatever the data): the lanes never
// diverge and every step's 2 kPlaceChunks LDS reads are in flight together.
__device__ __forceinline__ void count_below_all(const uint32_t* s, uint32_t lo, uint32_t hi, int (&lb)[kPlaceChunks],
                                                int (&ub)[kPlaceChunks]) {
#pragma unroll
  for (int q = 0; q < kPlaceChunks; ++q) lb[q] = ub[q] = q * kChunk;
#pragma unroll
  for (int len = kChunk; len > 1; len -= len >> 1) {
    const int h = len >> 1;
    uint32_t vl[kPlaceChunks], vu[kPlaceChunks];
#pragma unroll
    for (int q = 0; q < kPlaceChunks; ++q) {
      vl[q] = s[lb[q] + h];
      vu[q] = s[ub[q] + h];
    }
#pragma unroll
    for (int q = 0; q < kPlaceChunks; ++q) {
      lb[q] += vl[q] < lo ? h : 0;
      ub[q] += vu[q] < hi ? h : 0;
    }
  }
#pragma unroll
  for (int q = 0; q < kPlaceChunks; ++q) {
    lb[q] += (s[lb[q]] < lo ? 1 : 0) - q * kChunk;
    ub[q] += (s[ub[q]] < hi ? 1 : 0) - q * kChunk;
  }
}

// Grid xcd_grid(B * T, chunks), kThreads threads; rows of kChunk < L <= kTile positions whose chunks k_bucket_rows<1>
// sorted into packed (row r at packed + r * chunks * kChunk). Thread j takes sorted element j of chunk c.
__global__ __launch_bounds__(kThreads) void k_bucket_place(const uint32_t* __restrict__ packed, int64_t B, int64_t L,
                                                           int T, int C, int chunks,
                                                           int32_t* __restrict__ ids_sorted,
                                                           int32_t* __restrict__ order, int32_t* __restrict__ rank,
                                                           int32_t* __restrict__ win) {
  __shared__ uint32_t ks[kPlaceChunks * kChunk];   // the row's sorted chunks; ~0 past its real keys
  __shared__ uint32_t by_pos[kChunk];              // rank | win << kPosBits per position of the chunk
  const int tid = threadIdx.x;
  int c;
  int64_t y;
  xcd_chunk_row(chunks, &c, &y);
  if (y >= B * T) return;
  const int64_t b = y % B, tau = y / B;
  const int64_t r = b * T + tau;
  const uint32_t* row = packed + r * (int64_t)chunks * kChunk;
#pragma unroll
  for (int q = 0; q < kPlaceChunks; ++q) {
    const int64_t left = L - (int64_t)q * kChunk;                     // <= 0 past the row's chunks
    ks[q * kChunk + tid] = tid < left ? row[q * kChunk + tid] : ~0u;   // ~0 sorts after every bound
  }
  __syncthreads();
  const int nc = (int)(L - (int64_t)c * kChunk < kChunk ? L - (int64_t)c * kChunk : kChunk);
  const bool real = tid < nc;                      // not padding (sorted after the chunk's real positions)
  const uint32_t key = ks[c * kChunk + tid];
  const uint32_t lo_key = key & ~((1u << kPosBits) - 1u);             // (id, position 0)
  const uint32_t hi_key = lo_key + (1u << kPosBits);                  // (id + 1, position 0)
  // per chunk q: lb = its real keys with a smaller id, ub = with an id up to this one (0 past the row's chunks).
  // Unconditional, so that the 2 kPlaceChunks searches share one unrolled loop and their LDS reads overlap.
  int lb[kPlaceChunks], ub[kPlaceChunks];
  count_below_all(ks, lo_key, hi_key, lb, ub);
  int i = tid, start = 0, end = 0;
#pragma unroll
  for (int q = 0; q < kPlaceChunks; ++q) {
    start += lb[q];
    end += ub[q];
    i += q < c ? ub[q] : (q > c ? lb[q] : 0);
  }
  const int p = (int)(key & ((1u << kPosBits) - 1u));
  if (real) {
    ids_sorted[r * L + i] = (int32_t)(key >> kPosBits);
    order[r * L + i] = c * kChunk + p;
    const int before = min(C, i - start), after = min(C, end - 1 - i);
    if (p < nc) by_pos[p] = (uint32_t)i | ((uint32_t)(before | (after << 8)) << kPosBits);   // p < nc: a correct sort
  }
  __syncthreads();
  // consecutive lanes take consecutive positions: T-strided, not scattered, writes
  if (real) {
    const uint32_t x = by_pos[tid];
    const int64_t o = (b * L + (int64_t)c * kChunk + tid) * T + tau;
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

extern "C" int64_t asrn_bucket_sort_workspace(int64_t B, int64_t L, int32_t T) {
  using namespace asrn;
  if (L <= kChunk || L > kTile) return 0;
  return B * T * ((L + kChunk - 1) / kChunk) * kChunk * (int64_t)sizeof(uint32_t);
}

extern "C" int asrn_bucket_sort(const float* phi, int64_t B, int64_t L, int32_t T, int32_t nb, int64_t phi_stride,
                                int32_t C, int32_t* ids, int32_t* order, int32_t* ids_sorted, int32_t* rank,
                                int32_t* win, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace asrn;
  ASRN_REQUIRE(nb >= 1 && nb <= kMaxBits, "asrn_bucket_sort: n_bits must be in [1, %d] (got %d)", kMaxBits, nb);
  ASRN_REQUIRE(B >= 0 && L >= 0 && T >= 1 && T <= 32, "asrn_bucket_sort: bad sizes B=%lld L=%lld T=%d (T <= 32)",
               (long long)B, (long long)L, T);
  ASRN_REQUIRE(L < (int64_t(1) << 31), "asrn_bucket_sort: L=%lld too long", (long long)L);
  ASRN_REQUIRE(phi_stride >= (int64_t)T * nb, "asrn_bucket_sort: phi row stride %lld < T*nb = %d",
               (long long)phi_stride, T * nb);
  ASRN_REQUIRE(C >= 1 && C <= 255, "asrn_bucket_sort: window C=%d must be in [1, 255]", C);
  if (B == 0 || L == 0) return 0;
  ASRN_REQUIRE(ids && order && ids_sorted && rank && win, "asrn_bucket_sort: null pointer");
  const int64_t need = asrn_bucket_sort_workspace(B, L, T);
  ASRN_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
               "asrn_bucket_sort: workspace %lld bytes < %lld needed", (long long)workspace_bytes, (long long)need);
  hipStream_t st = (hipStream_t)stream;
  const int64_t rows = B * T;
  if (L <= kChunk) {                               // one tile per row: everything in one launch
    hipLaunchKernelGGL(k_bucket_rows<1>, dim3(xcd_grid(rows, 1)), dim3(kThreads), 0, st, phi, B, L, (int)T, (int)nb,
                       phi_stride, (int)C, (int)kOutWhole, ids, ids_sorted, order, rank, win, nullptr, (int64_t)0, 1,
                       true);
    return check_launch("asrn_bucket_sort/rows");
  }
  if (L <= kTile) {                                // chunks of 1024 on their own workgroups, then every element placed
    const int chunks = (int)((L + kChunk - 1) / kChunk);
    uint32_t* packed = (uint32_t*)workspace;
    hipLaunchKernelGGL(k_bucket_rows<1>, dim3(xcd_grid(rows, chunks)), dim3(kThreads), 0, st, phi, B, L, (int)T,
                       (int)nb, phi_stride, (int)C, (int)kOutPacked, ids, nullptr, nullptr, nullptr, nullptr, packed,
                       (int64_t)chunks * kChunk, chunks, true);
    if (check_launch("asrn_bucket_sort/chunks")) return 1;
    hipLaunchKernelGGL(k_bucket_place, dim3(xcd_grid(rows, chunks)), dim3(kThreads), 0, st, packed, B, L,
                       (int)T, (int)C, chunks, ids_sorted, order, rank, win);
    return check_launch("asrn_bucket_sort/place");
  }
  const int64_t tiles = (L + kTile - 1) / kTile;
  int passes = 0;
  for (int64_t w = kTile; w < L; w <<= 1) ++passes;
  // the merge passes ping-pong between (ids_sorted, order) and (rank, win), which the finish overwrites last: start
  // in the buffer that makes the final pass land in (ids_sorted, order)
  int32_t* bufk[2] = {ids_sorted, rank};
  int32_t* bufp[2] = {order, win};
  int cur = passes % 2;
  hipLaunchKernelGGL(k_bucket_rows<4>, dim3((unsigned)(tiles * rows)), dim3(kThreads), 0, st, phi, B, L, (int)T,
                     (int)nb, phi_stride, (int)C, (int)kOutPairs, ids, bufk[cur], bufp[cur], rank, win, nullptr,
                     (int64_t)0, (int)tiles, false);
  if (check_launch("asrn_bucket_sort/rows")) return 1;
  const int threads = 256;
  const unsigned blocks = (unsigned)((rows * L + threads - 1) / threads);
  for (int64_t w = kTile; w < L; w <<= 1) {
    hipLaunchKernelGGL(k_bucket_merge, dim3(blocks), dim3(threads), 0, st, bufk[cur], bufp[cur], bufk[cur ^ 1],
                       bufp[cur ^ 1], rows, L, w);
    if (check_launch("asrn_bucket_sort/merge")) return 1;
    cur ^= 1;
  }
  hipLaunchKernelGGL(k_bucket_finish, dim3(blocks), dim3(threads), 0, st, ids_sorted, order, rows, L, (int)T, (int)C,
                     rank, win);
  return check_launch("asrn_bucket_sort/finish");
}
