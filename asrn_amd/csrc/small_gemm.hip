// Products of small fp32 matrices (the layer's weight products, a few hundred rows and columns each), where a library
// GEMM picks a single-workgroup tile: here every 16 x 16 tile of C is its own workgroup, the K axis staged through
// LDS 256 at a time (one round of loads for K <= 256). C = op(A) op(B), op = identity or transpose; each C element
// sums over k in increasing order, so the result is deterministic.
#include "common.h"

namespace asrn {

constexpr int kTile = 16;
constexpr int kKc = 256;                        // K staged per round: every load of a round is in flight at once
constexpr int kGemmThreads = kTile * kTile;

struct SmallGemm {
  const float* A; int64_t lda; int ta;
  const float* B; int64_t ldb; int tb;
  float* C; int64_t ldc;
  int M, N, K;
};

// Element e of a round's staging of op(A) (16 rows of the tile, kKc columns of K) and of op(B) (kKc rows of K, 16
// columns of the tile). Consecutive e are consecutive addresses of the stored matrix: along K for a row-major op(A),
// along the tile's rows when A is stored transposed; likewise for B. Out-of-range elements read 0.
template <bool TA>
__device__ __forceinline__ float stage_a(const SmallGemm& g, int i0, int k0, int e, int& r, int& c) {
  r = TA ? e % kTile : e / kKc;               // row of the tile
  c = TA ? e / kTile : e % kKc;               // column within the round's K
  const int i = i0 + r, k = k0 + c;
  const bool ok = i < g.M && k < g.K;
  const int64_t at = TA ? (int64_t)k * g.lda + i : (int64_t)i * g.lda + k;
  const float v = g.A[ok ? at : 0];
  return ok ? v : 0.f;
}
template <bool TB>
__device__ __forceinline__ float stage_b(const SmallGemm& g, int k0, int j0, int e, int& r, int& c) {
  r = TB ? e % kKc : e / kTile;               // row within the round's K
  c = TB ? e / kKc : e % kTile;               // column of the tile
  const int k = k0 + r, j = j0 + c;
  const bool ok = k < g.K && j < g.N;
  const int64_t at = TB ? (int64_t)j * g.ldb + k : (int64_t)k * g.ldb + j;
  const float v = g.B[ok ? at : 0];
  return ok ? v : 0.f;
}

template <bool TA, bool TB>
__global__ __launch_bounds__(kGemmThreads) void k_small_gemm(SmallGemm g) {
  constexpr int kPer = kTile * kKc / kGemmThreads;   // elements of each operand a thread stages per round
  __shared__ float As[kTile][kKc + 1];
  __shared__ float Bs[kKc][kTile + 1];
  const int t = threadIdx.x, tx = t % kTile, ty = t / kTile;
  const int i0 = blockIdx.y * kTile, j0 = blockIdx.x * kTile;
  float acc = 0.f;
  for (int k0 = 0; k0 < g.K; k0 += kKc) {
    float va[kPer], vb[kPer];
    int ra[kPer], ca[kPer], rb[kPer], cb[kPer];
#pragma unroll
    for (int x = 0; x < kPer; ++x) {            // every load of the round issued before any is used
      va[x] = stage_a<TA>(g, i0, k0, t + x * kGemmThreads, ra[x], ca[x]);
      vb[x] = stage_b<TB>(g, k0, j0, t + x * kGemmThreads, rb[x], cb[x]);
    }
#pragma unroll
    for (int x = 0; x < kPer; ++x) {
      As[ra[x]][ca[x]] = va[x];
      Bs[rb[x]][cb[x]] = vb[x];
    }
    __syncthreads();
#pragma unroll 16
    for (int kk = 0; kk < kKc; ++kk) acc += As[ty][kk] * Bs[kk][tx];
    __syncthreads();
  }
  if (i0 + ty < g.M && j0 + tx < g.N) g.C[(int64_t)(i0 + ty) * g.ldc + j0 + tx] = acc;
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_small_gemm(const float* A, int64_t lda, int32_t trans_a, const float* B, int64_t ldb,
                               int32_t trans_b, float* C, int64_t ldc, int32_t M, int32_t N, int32_t K,
                               void* stream) {
  ASRN_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M <= 8192 && N <= 8192 && K <= 8192,
               "asrn_small_gemm: M=%d N=%d K=%d must be in [0, 8192]", M, N, K);
  ASRN_REQUIRE(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N) && ldc >= N && lda >= 1 && ldb >= 1 && ldc >= 1,
               "asrn_small_gemm: leading dimensions too small (lda=%lld ldb=%lld ldc=%lld)", (long long)lda,
               (long long)ldb, (long long)ldc);
  if (M == 0 || N == 0) return 0;
  SmallGemm g = {A, lda, trans_a ? 1 : 0, B, ldb, trans_b ? 1 : 0, C, ldc, M, N, K};
  const dim3 grid((unsigned)((N + kTile - 1) / kTile), (unsigned)((M + kTile - 1) / kTile));
  hipStream_t st = (hipStream_t)stream;
  if (g.ta && g.tb) hipLaunchKernelGGL((k_small_gemm<true, true>), grid, dim3(kGemmThreads), 0, st, g);
  else if (g.ta) hipLaunchKernelGGL((k_small_gemm<true, false>), grid, dim3(kGemmThreads), 0, st, g);
  else if (g.tb) hipLaunchKernelGGL((k_small_gemm<false, true>), grid, dim3(kGemmThreads), 0, st, g);
  else hipLaunchKernelGGL((k_small_gemm<false, false>), grid, dim3(kGemmThreads), 0, st, g);
  return check_launch("asrn_small_gemm");
}
