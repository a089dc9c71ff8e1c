// a10: n-gram keys, their stable sort per (b, j) row, the repeated flags and the seen flags.
//
// Keys are fp64 and must round exactly as the reference's separate multiply and add (asrn/nucleo.py:182-184): the
// kernel uses __dmul_rn / __dadd_rn and this file builds with -ffp-contract=off. The sort orders (key, position)
// pairs, with the key mapped to an order-preserving uint64 (-0 -> +0, every NaN -> the largest code so NaN sorts
// last and stays in text order, as torch.argsort(stable=True) does). Tiles of up to 1024 pairs are bitonic-sorted
// in registers, lane exchanges and LDS (block_sort.h); longer rows are finished by merge passes in which every
// element finds its output slot by a binary search in the other run.
#include "block_sort.h"

namespace asrn {

constexpr int kTile = 1024;          // pairs per sorted tile (more workgroups; merges finish longer rows)
constexpr uint64_t kNanCode = ~0ull;
constexpr uint32_t kPadIdx = 0xFFFFFFFFu;

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
};

// keys (B, L, n) and the (code, position) pairs of every (b, j) row, padded to Lp with sentinels
__global__ void k_ngram_keys(const float* __restrict__ sig, const double* __restrict__ coef, NgramDims g,
                             double* __restrict__ keys, uint64_t* __restrict__ code, uint32_t* __restrict__ idx) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = g.B * g.Lp;
  if (e >= total) return;
  const int64_t b = e / g.Lp, t = e % g.Lp;
  if (t >= g.L) {
    for (int j = 0; j < g.n; ++j) {
      code[(b * g.n + j) * g.Lp + t] = kNanCode;
      idx[(b * g.n + j) * g.Lp + t] = kPadIdx;
    }
    return;
  }
  double key = 0.0;
  for (int j = 0; j < g.n; ++j) {
    const double s = (t - j >= 0) ? (double)sig[b * g.L + t - j] : __longlong_as_double(0x7ff8000000000000ll);
    key = __dadd_rn(key, __dmul_rn(s, coef[j]));
    keys[(b * g.L + t) * g.n + j] = key;
    code[(b * g.n + j) * g.Lp + t] = key_code(key);
    idx[(b * g.n + j) * g.Lp + t] = (uint32_t)t;
  }
}

// each tile of `tile` (code, position) pairs sorted by one workgroup of tile / 4 threads (block_sort.h)
__global__ __launch_bounds__(kTile / 4) void k_tile_sort(uint64_t* __restrict__ code, uint32_t* __restrict__ idx,
                                                         int64_t Lp, int tile) {
  __shared__ SortKI lds[kTile];
  const int64_t base = (int64_t)blockIdx.y * Lp + (int64_t)blockIdx.x * tile;
  SortKI x[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t e = base + 4 * threadIdx.x + q;
    x[q] = SortKI{code[e], idx[e]};
  }
  block_bitonic_sort(x, lds, tile);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t e = base + 4 * threadIdx.x + q;
    code[e] = x[q].k;
    idx[e] = x[q].i;
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

static void ngram_dims(int64_t B, int64_t L, int n, NgramDims* g) {
  int tile = 2;
  while (tile < L && tile < kTile) tile <<= 1;
  if (tile < 4) tile = 4;
  int64_t tiles = 1;
  while (tiles * tile < L) tiles <<= 1;
  g->B = B;
  g->L = L;
  g->n = n;
  g->tile = tile;
  g->Lp = tiles * tile;
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

  const int threads = 256;
  hipLaunchKernelGGL(k_ngram_keys, dim3((unsigned)((B * g.Lp + threads - 1) / threads)), dim3(threads), 0, st, sig,
                     coef, g, keys, code0, idx0);
  if (check_launch("asrn_ngram_sort/keys")) return 1;
  hipLaunchKernelGGL(k_tile_sort, dim3((unsigned)(g.Lp / g.tile), (unsigned)rows), dim3(g.tile / 4), 0, st, code0,
                     idx0, g.Lp, g.tile);
  if (check_launch("asrn_ngram_sort/tile")) return 1;
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
