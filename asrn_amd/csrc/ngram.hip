// a10: n-gram keys, their stable sort per (b, j) row, the repeated flags and the seen flags.
//
// Keys are fp64 and must round exactly as the reference's separate multiply and add (asrn/nucleo.py:182-184): the
// kernels use __dmul_rn / __dadd_rn and this file builds with -ffp-contract=off. The sort orders (key, position)
// pairs, with the key mapped to an order-preserving uint64 (-0 -> +0, every NaN -> the largest code so NaN sorts
// last and stays in text order, as torch.argsort(stable=True) does). The pairs are unique, so any correct sort of
// them is the stable sort.
//
//   k_ngram_rows   one workgroup per tile of a (b, j) row (a row of up to 1024 positions, or a tile of 4096 of a
//                  longer row): the keys of its positions, a sort of the tile in LDS (4 pairs per thread sorted in
//                  registers, then merge levels of doubling runs in which every thread finds its 4 output slots'
//                  split point by a merge-path search and merges them), and, when the tile is the whole row, the
//                  outputs (order, repeated, rank, seen) from the sorted pairs in LDS: one launch.
//   k_ngram_chunk  rows of 1025 to 4096 positions: a workgroup of 1024 threads per chunk of 1024 (so a row spreads
//                  over up to 4 CUs) computes the chunk's keys and sorts its pairs in LDS, one pair per thread: at
//                  each of the 10 merge levels a pair's new index is its index in its run plus the count of the
//                  partner run's codes below its own (the right run's pairs count the left run's codes up to their
//                  own, so ties keep text order), a fixed-length search in LDS.
//   k_ngram_place  then every sorted pair finds its place in the row: with the row's sorted chunk codes in LDS,
//                  searches count, in each chunk, the codes below its own and up to its own; earlier chunks' equal
//                  codes go first (they hold earlier positions), so its sorted index is its index in its chunk plus
//                  those counts, and it repeats its predecessor exactly when codes equal to its own precede it.
//   k_merge_pass   rows longer than 4096: merge passes over the sorted tiles (every element finds its output slot by
//                  a binary search in the partner run), ping-ponging in the workspace.
//   k_ngram_finish those rows: the outputs from the merged pairs.
#include "common.h"

namespace asrn {

constexpr int kRowTile = 4096;                   // pairs sorted per workgroup
constexpr int kRowThreads = kRowTile / 4;
constexpr int kChunk = 1024;                     // the chunks of rows of kChunk < L <= kRowTile (k_ngram_place)
constexpr int kPlaceChunks = kRowTile / kChunk;
constexpr int kPlaceThreads = kChunk;
constexpr uint64_t kNanCode = ~0ull;

__device__ __forceinline__ uint64_t key_code(double x) {
  if (x != x) return kNanCode;
  if (x == 0.0) x = 0.0;
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

__device__ __forceinline__ bool pair_less(uint64_t ka, uint32_t ia, uint64_t kb, uint32_t ib) {
  return ka < kb || (ka == kb && ia < ib);
}

struct NgramDims {
  int64_t B, L, Lp;
  int n, tile;
  bool place;                                    // chunks of kChunk placed by k_ngram_place
};

// the n-gram key of length j + 1 ending at t: sum over i <= j of sig[t - i] * coef[i], each product and sum rounded
// separately, in the reference's order (NaN before the text's start)
__device__ __forceinline__ double ngram_key(const float* __restrict__ sigb, const double* __restrict__ coef,
                                            int64_t t, int j) {
  double key = 0.0;
  for (int i = 0; i <= j; ++i) {
    const float x = sigb[t - i >= 0 ? t - i : 0];              // unconditional load, masked after
    const double s = (t - i >= 0) ? (double)x : __longlong_as_double(0x7ff8000000000000ll);
    key = __dadd_rn(key, __dmul_rn(s, coef[i]));
  }
  return key;
}

template <class T>
__device__ __forceinline__ void swap_if(bool c, T& a, T& b) {
  const T x = c ? b : a, y = c ? a : b;
  a = x;
  b = y;
}

__device__ __forceinline__ void sort_pair(uint64_t (&k)[4], uint32_t (&p)[4], int a, int b) {
  const bool c = pair_less(k[b], p[b], k[a], p[a]);
  swap_if(c, k[a], k[b]);
  swap_if(c, p[a], p[b]);
}

// Grid (Lp / tile, B * n), tile / 4 threads. whole: the tile is the row (Lp == tile), so the outputs are written
// here; otherwise the sorted (code, position) pairs of the tile go to code_out / idx_out at row * Lp + tile start.
__global__ __launch_bounds__(kRowThreads) void k_ngram_rows(const float* __restrict__ sig,
                                                            const double* __restrict__ coef, NgramDims g, bool whole,
                                                            double* __restrict__ keys, int32_t* __restrict__ order,
                                                            uint8_t* __restrict__ repeated,
                                                            int32_t* __restrict__ rank_k, float* __restrict__ vistos,
                                                            uint64_t* __restrict__ code_out,
                                                            uint32_t* __restrict__ idx_out) {
  __shared__ uint64_t ck[2][kRowTile];
  __shared__ uint16_t cp[2][kRowTile];             // position within the tile
  const int tid = threadIdx.x, tile = g.tile;
  const int64_t row = blockIdx.y, b = row / g.n;
  const int j = (int)(row % g.n);
  const int64_t t0 = (int64_t)blockIdx.x * tile;
  const float* sigb = sig + b * g.L;

  uint64_t k[4];
  uint32_t p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int e = 4 * tid + r;
    const int64_t t = t0 + e;
    p[r] = (uint32_t)e;
    k[r] = kNanCode;                                // padding past the row: after every real pair
    if (t < g.L) {
      const double key = ngram_key(sigb, coef, t, j);
      keys[(b * g.L + t) * g.n + j] = key;
      k[r] = key_code(key);
    }
  }
  sort_pair(k, p, 0, 1);
  sort_pair(k, p, 2, 3);
  sort_pair(k, p, 0, 2);
  sort_pair(k, p, 1, 3);
  sort_pair(k, p, 1, 2);

  // merge levels: runs of w sorted pairs become runs of 2w. Run [s, s + w) holds exactly the tile positions
  // [s, s + w), so a merge that takes A's pair on equal codes keeps text order: the search and the merge compare
  // codes only. Thread tid owns output slots 4 tid .. 4 tid + 3 of its pair of runs A = [s, s + w), B = [s + w,
  // s + 2w); the split (i, d - i) of diagonal d = 4 tid - s is the number of A's pairs among the first d of the merge.
  int cur = 0;
  for (int w = 4; w < tile; w <<= 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ck[cur][4 * tid + r] = k[r];
      cp[cur][4 * tid + r] = (uint16_t)p[r];
    }
    __syncthreads();
    const int s = (4 * tid) & ~(2 * w - 1), d = 4 * tid - s;
    const uint64_t* ak = ck[cur] + s;
    const uint16_t* ap = cp[cur] + s;
    const uint64_t* bk = ak + w;
    const uint16_t* bp = ap + w;
    int lo = d > w ? d - w : 0, hi = d < w ? d : w;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (ak[mid] <= bk[d - 1 - mid]) lo = mid + 1; else hi = mid;
    }
    int ia = lo, ib = d - lo;
    uint64_t ka = ia < w ? ak[ia] : 0, kb = ib < w ? bk[ib] : 0;
    uint32_t pa = ia < w ? ap[ia] : 0, pb = ib < w ? bp[ib] : 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool take_a = ia < w && (ib >= w || ka <= kb);
      k[r] = take_a ? ka : kb;
      p[r] = take_a ? pa : pb;
      if (take_a) {
        ++ia;
        ka = ia < w ? ak[ia] : 0;
        pa = ia < w ? ap[ia] : 0;
      } else {
        ++ib;
        kb = ib < w ? bk[ib] : 0;
        pb = ib < w ? bp[ib] : 0;
      }
    }
    cur ^= 1;
  }

  if (!whole) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t o = row * g.Lp + t0 + 4 * tid + r;
      code_out[o] = k[r];
      idx_out[o] = (uint32_t)(t0 + p[r]);
    }
    return;
  }
  // outputs: order and repeated per sorted slot here; rank and seen per position through LDS (sorted slot | repeated
  // << 15 by position), so that both are written in position order
#pragma unroll
  for (int r = 0; r < 4; ++r) ck[cur][4 * tid + r] = k[r];
  __syncthreads();
  uint16_t* by_pos = cp[cur];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * tid + r;
    if (i >= g.L) continue;                         // padding sorts last
    const bool rep = i > 0 && k[r] != kNanCode && ck[cur][i - 1] == k[r];
    order[row * g.L + i] = (int32_t)p[r];
    repeated[row * g.L + i] = rep ? 1 : 0;
    by_pos[p[r]] = (uint16_t)(i | (rep ? 0x8000 : 0));
  }
  __syncthreads();
  for (int t = tid; t < g.L; t += blockDim.x) {
    const uint32_t x = by_pos[t];
    rank_k[row * g.L + t] = (int32_t)(x & 0x7FFFu);
    vistos[(b * g.L + t) * g.n + j] = (x & 0x8000u) ? 1.f : 0.f;
  }
}

// merge runs of width w into runs of 2w: stable (left run first on ties)
__global__ void k_merge_pass(const uint64_t* __restrict__ kin, const uint32_t* __restrict__ iin,
                             uint64_t* __restrict__ kout, uint32_t* __restrict__ iout, int64_t rows, int64_t Lp,
                             int64_t w) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * Lp) return;
  const int64_t row = e / Lp, p = e % Lp;
  const int64_t run = p / w, pos = p % w;
  const bool left = (run & 1) == 0;
  const int64_t other = (left ? run + 1 : run - 1) * w;
  const int64_t rb = row * Lp;
  const uint64_t k = kin[e];
  const uint32_t x = iin[e];
  // left: count of right-run elements strictly below; right: count of left-run elements below or equal
  int64_t lo = 0, hi = w;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    const uint64_t km = kin[rb + other + mid];
    const uint32_t xm = iin[rb + other + mid];
    const bool go_right = left ? pair_less(km, xm, k, x) : !pair_less(k, x, km, xm);
    if (go_right) lo = mid + 1; else hi = mid;
  }
  const int64_t out = rb + (run >> 1) * 2 * w + pos + lo;
  kout[out] = k;
  iout[out] = x;
}

__global__ void k_ngram_finish(const uint64_t* __restrict__ code, const uint32_t* __restrict__ idx, NgramDims g,
                               int32_t* __restrict__ order, uint8_t* __restrict__ repeated,
                               int32_t* __restrict__ rank_k, float* __restrict__ vistos) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows = g.B * g.n;
  if (e >= rows * g.L) return;
  const int64_t row = e / g.L, i = e % g.L;
  const int64_t b = row / g.n;
  const int j = (int)(row % g.n);
  const uint64_t k = code[row * g.Lp + i];
  const uint32_t t = idx[row * g.Lp + i];
  const bool rep = i > 0 && k != kNanCode && code[row * g.Lp + i - 1] == k;
  const bool ok = t < (uint64_t)g.L;             // always true for a correct sort; keeps a bug from faulting
  order[row * g.L + i] = ok ? (int32_t)t : 0;
  repeated[row * g.L + i] = rep ? 1 : 0;
  if (ok) {
    rank_k[row * g.L + t] = (int32_t)i;
    vistos[(b * g.L + t) * g.n + j] = rep ? 1.f : 0.f;
  }
}

// For each of the kPlaceChunks sorted runs of kChunk codes at s + q kChunk: lb[q] = its codes below x, ub[q] = up to
// x. Branch-free lower bounds with a fixed trip count (the interval halves whatever the data): the lanes never
// diverge and every step's 2 kPlaceChunks LDS reads are in flight together.
__device__ __forceinline__ void count_below_all(const uint64_t* s, uint64_t x, int (&lb)[kPlaceChunks],
                                                int (&ub)[kPlaceChunks]) {
#pragma unroll
  for (int q = 0; q < kPlaceChunks; ++q) lb[q] = ub[q] = q * kChunk;
#pragma unroll
  for (int len = kChunk; len > 1; len -= len >> 1) {
    const int h = len >> 1;
    uint64_t vl[kPlaceChunks], vu[kPlaceChunks];
#pragma unroll
    for (int q = 0; q < kPlaceChunks; ++q) {
      vl[q] = s[lb[q] + h];
      vu[q] = s[ub[q] + h];
    }
#pragma unroll
    for (int q = 0; q < kPlaceChunks; ++q) {
      lb[q] += vl[q] < x ? h : 0;
      ub[q] += vu[q] <= x ? h : 0;
    }
  }
#pragma unroll
  for (int q = 0; q < kPlaceChunks; ++q) {
    lb[q] += (s[lb[q]] < x ? 1 : 0) - q * kChunk;
    ub[q] += (s[ub[q]] <= x ? 1 : 0) - q * kChunk;
  }
}

// Grid xcd_grid(B * n, chunks), kPlaceThreads threads: thread e starts with position t0 + e of the chunk and follows
// that pair through the merge levels; the sorted chunk goes to code_out / idx_out at row * Lp + t0. (k_ngram_place,
// on the same map, finds a row's sorted chunks in its XCD's L2.)
__global__ __launch_bounds__(kPlaceThreads) void k_ngram_chunk(const float* __restrict__ sig,
                                                               const double* __restrict__ coef, NgramDims g,
                                                               double* __restrict__ keys,
                                                               uint64_t* __restrict__ code_out,
                                                               uint32_t* __restrict__ idx_out, int chunks) {
  __shared__ uint64_t ck[2][kChunk];
  const int e0 = threadIdx.x;
  int c;
  int64_t row;
  xcd_chunk_row(chunks, &c, &row);
  if (row >= g.B * g.n) return;
  const int64_t b = row / g.n;
  const int j = (int)(row % g.n);
  const int64_t t0 = (int64_t)c * kChunk, t = t0 + e0;
  uint64_t k = kNanCode;                           // padding past the row: after every real pair, in order
  if (t < g.L) {
    const double key = ngram_key(sig + b * g.L, coef, t, j);
    keys[(b * g.L + t) * g.n + j] = key;
    k = key_code(key);
  }
  int e = e0;                                      // the pair's index in the chunk: sorted runs of w after level w
  int cur = 0;
  ck[0][e] = k;
  __syncthreads();
  for (int w = 1; w < kChunk; w <<= 1) {
    const bool left = (e & w) == 0;                // run A (earlier positions) or B of the pair of runs
    const uint64_t* part = ck[cur] + ((e ^ w) & ~(w - 1));   // the partner run
    // count of the partner's codes below k (A) or up to k (B): branch-free lower bound, log2 w + 1 reads
    int base = 0;
    for (int len = w; len > 1; len -= len >> 1) {
      const uint64_t v = part[base + (len >> 1)];
      base += (left ? v < k : v <= k) ? (len >> 1) : 0;
    }
    const uint64_t v = part[base];
    base += (left ? v < k : v <= k) ? 1 : 0;
    e = (e & ~(2 * w - 1)) + (e & (w - 1)) + base;
    ck[cur ^ 1][e] = k;
    __syncthreads();
    cur ^= 1;
  }
  // thread e0's pair ends at sorted index e; the pairs are unique, so the chunk's sorted codes and positions are
  // written from their owners (positions) and from LDS (codes, coalesced)
  code_out[row * g.Lp + t0 + e0] = ck[cur][e0];
  idx_out[row * g.Lp + t0 + e] = (uint32_t)t;
}

// Grid xcd_grid(B * n, chunks), kPlaceThreads threads; the row's chunks sorted by k_ngram_chunk into code / idx (row
// at row * Lp). Thread e takes sorted pair e of chunk c.
__global__ __launch_bounds__(kPlaceThreads) void k_ngram_place(const uint64_t* __restrict__ code,
                                                               const uint32_t* __restrict__ idx, NgramDims g,
                                                               int chunks, int32_t* __restrict__ order,
                                                               uint8_t* __restrict__ repeated,
                                                               int32_t* __restrict__ rank_k,
                                                               float* __restrict__ vistos) {
  __shared__ uint64_t ks[kPlaceChunks * kChunk];  // the row's sorted chunk codes
  __shared__ uint16_t by_pos[kChunk];             // sorted index | repeated << 15 per position of the chunk
  const int tid = threadIdx.x;
  int c;
  int64_t row;
  xcd_chunk_row(chunks, &c, &row);
  if (row >= g.B * g.n) return;
  const int64_t b = row / g.n;
  const int j = (int)(row % g.n);
  const uint64_t* rc = code + row * g.Lp;
#pragma unroll
  for (int q = 0; q < kPlaceChunks; ++q) ks[q * kChunk + tid] = q < chunks ? rc[q * kChunk + tid] : kNanCode;
  const uint32_t t = idx[row * g.Lp + (int64_t)c * kChunk + tid];
  __syncthreads();
  const int nc = (int)(g.L - (int64_t)c * kChunk < kChunk ? g.L - (int64_t)c * kChunk : kChunk);
  const bool real = tid < nc;                     // not padding (sorted after the chunk's real pairs)
  const uint64_t x = ks[c * kChunk + tid];
  // per chunk q: lb = its codes below x, ub = up to x. Padding and the slots past the row's chunks hold the NaN
  // code, which is never below x; ub is used only of the full chunks before this one. Unconditional, so that the
  // 2 kPlaceChunks searches share one unrolled loop and their LDS reads overlap.
  int lb[kPlaceChunks], ub[kPlaceChunks];
  count_below_all(ks, x, lb, ub);
  int i = tid, start = 0;
#pragma unroll
  for (int q = 0; q < kPlaceChunks; ++q) {
    start += lb[q];
    i += q < c ? ub[q] : (q > c ? lb[q] : 0);
  }
  const bool rep = x != kNanCode && i > start;
  const int64_t p = (int64_t)t - (int64_t)c * kChunk;   // in [0, nc) for a correct sort
  if (real) {
    order[row * g.L + i] = (int32_t)t;
    repeated[row * g.L + i] = rep ? 1 : 0;
    if (p >= 0 && p < nc) by_pos[p] = (uint16_t)(i | (rep ? 0x8000 : 0));
  }
  __syncthreads();
  // rank and seen in position order
  if (real) {
    const uint32_t y = by_pos[tid];
    const int64_t tt = (int64_t)c * kChunk + tid;
    rank_k[row * g.L + tt] = (int32_t)(y & 0x7FFFu);
    vistos[(b * g.L + tt) * g.n + j] = (y & 0x8000u) ? 1.f : 0.f;
  }
}

// Rows of up to kChunk: one tile, a power of two >= L (at least 4). Rows of kChunk < L <= kRowTile: tiles of kChunk,
// Lp = the chunks' span (place). Longer rows: tiles of kRowTile, Lp = the row padded to a power-of-two number of
// tiles (merge passes).
static void ngram_dims(int64_t B, int64_t L, int n, NgramDims* g) {
  int tile = 4;
  while (tile < L && tile < kRowTile) tile <<= 1;
  int64_t tiles = 1;
  while (tiles * tile < L) tiles <<= 1;
  g->B = B;
  g->L = L;
  g->n = n;
  g->tile = tile;
  g->Lp = tiles * tile;
  g->place = L > kChunk && L <= kRowTile;
  if (g->place) {
    g->tile = kChunk;
    g->Lp = (L + kChunk - 1) / kChunk * kChunk;
  }
}

}  // namespace asrn

extern "C" int64_t asrn_ngram_sort_workspace(int64_t B, int64_t L, int32_t n) {
  asrn::NgramDims g;
  asrn::ngram_dims(B, L, n, &g);
  const int64_t elems = B * n * g.Lp;
  return 2 * elems * (int64_t)(sizeof(uint64_t) + sizeof(uint32_t)) + 256;
}

extern "C" int asrn_ngram_sort(const float* sig, const double* coef, int64_t B, int64_t L, int32_t n, double* keys,
                               int32_t* order, uint8_t* repeated, int32_t* rank_k, float* vistos, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  using namespace asrn;
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1 && n <= 64, "asrn_ngram_sort: bad sizes B=%lld L=%lld n=%d",
               (long long)B, (long long)L, n);
  ASRN_REQUIRE(L < (int64_t(1) << 31), "asrn_ngram_sort: L=%lld too long", (long long)L);
  if (B == 0 || L == 0) return 0;
  ASRN_REQUIRE(workspace_bytes >= asrn_ngram_sort_workspace(B, L, n),
               "asrn_ngram_sort: workspace %lld bytes < %lld needed", (long long)workspace_bytes,
               (long long)asrn_ngram_sort_workspace(B, L, n));
  NgramDims g;
  ngram_dims(B, L, n, &g);
  const int64_t rows = B * n, elems = rows * g.Lp;
  uint64_t* code0 = (uint64_t*)workspace;
  uint64_t* code1 = code0 + elems;
  uint32_t* idx0 = (uint32_t*)(code1 + elems);
  uint32_t* idx1 = idx0 + elems;
  hipStream_t st = (hipStream_t)stream;
  if (g.place) {
    const int chunks = (int)(g.Lp / kChunk);
    hipLaunchKernelGGL(k_ngram_chunk, dim3(xcd_grid(rows, chunks)), dim3(kPlaceThreads), 0, st, sig, coef, g, keys,
                       code0, idx0, chunks);
    if (check_launch("asrn_ngram_sort/chunks")) return 1;
    hipLaunchKernelGGL(k_ngram_place, dim3(xcd_grid(rows, chunks)), dim3(kPlaceThreads), 0, st, code0,
                       idx0, g, chunks, order, repeated, rank_k, vistos);
    return check_launch("asrn_ngram_sort/place");
  }
  const bool whole = g.Lp == g.tile;
  hipLaunchKernelGGL(k_ngram_rows, dim3((unsigned)(g.Lp / g.tile), (unsigned)rows), dim3(g.tile / 4), 0, st, sig,
                     coef, g, whole, keys, order, repeated, rank_k, vistos, code0, idx0);
  if (check_launch("asrn_ngram_sort/rows")) return 1;
  if (whole) return 0;
  const int threads = 256;
  uint64_t* kc = code0;
  uint32_t* ic = idx0;
  uint64_t* ko = code1;
  uint32_t* io = idx1;
  for (int64_t w = g.tile; w < g.Lp; w <<= 1) {
    hipLaunchKernelGGL(k_merge_pass, dim3((unsigned)((elems + threads - 1) / threads)), dim3(threads), 0, st, kc, ic,
                       ko, io, rows, g.Lp, w);
    if (check_launch("asrn_ngram_sort/merge")) return 1;
    uint64_t* tk = kc; kc = ko; ko = tk;
    uint32_t* ti = ic; ic = io; io = ti;
  }
  hipLaunchKernelGGL(k_ngram_finish, dim3((unsigned)((rows * L + threads - 1) / threads)), dim3(threads), 0, st, kc,
                     ic, g, order, repeated, rank_k, vistos);
  return check_launch("asrn_ngram_sort/finish");
}
