// The local block's generation step (asrn/nucleo.py:1811-1814; the model's BloqueLocal, nucleo:969-1014, mezcla
// 'conv') for the few rows of a decode batch, in six launches:
//   k_prep_mix    per row: z = LayerNorm1(h) and X1 = [the ring's k - 1 taps; z] in nn.Conv1d's column order
//                 (column c*k + j: channel c, tap j)
//   k_part        P1 = X1 conv_w^T, in depth splits
//   k_finish_mix  per row: h1 = h + GELU(sum of P1 + conv_b); X2 = LayerNorm2(h1)
//   k_part        P2 = X2 w1^T, in depth splits
//   k_part        P3 = GELU(sum of P2 + b1) w2^T (the GELU applied as its operand is loaded), in depth splits
//   k_finish_res  per row: out = h1 + sum of P3 + b2; z enters the ring at slot pos mod (k - 1)
// The ring holds row t (t = position) at slot t mod (k - 1), so tap j of position pos (j = 0 oldest, k - 2 newest) is
// at slot (pos + j) mod (k - 1) and nothing shifts. The position is read on the device (a captured step advances it).
//
// The products (16 rows at most per tile) run on the matrix cores in fp32 (v_mfma_f32_16x16x4f32): a workgroup owns a
// 16 x 16 output tile over one split of the depth, its four wavefronts a quarter each, every lane loading a float4 of
// the weight row and of the operand row per 16 columns of depth (the weights stream once, coalesced). The splits are
// sized so that a wavefront's share is one round of loads issued ahead of its products (at most 64 columns). The wavefronts' tiles are summed in LDS; the splits are summed by the next
// kernel, in split order: deterministic, and no workgroup waits for another (across the chip's eight L2 caches a
// device-wide fence costs more than these products).
#include "common.h"

namespace asrn {
namespace {

constexpr int kTile = 16;
constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kPrepThreads = 1024;
constexpr int kPrepWaves = kPrepThreads / kWave;
constexpr int kMaxSplits = 16;

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }

__device__ __forceinline__ float block_total(float v, float* red) {
  v = wave_sum_u(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kPrepWaves; ++i) t += red[i];
  return t;
}

// mean and 1/sqrt(var + eps) of one row of width d, by a workgroup of kPrepThreads (results in every thread)
__device__ void row_stats(const float* row, int d, float eps, float* red, float* mean, float* rstd) {
  float s = 0.f;
  for (int c = threadIdx.x; c < d; c += kPrepThreads) s += row[c];
  const float m = block_total(s, red) / (float)d;
  float q = 0.f;
  for (int c = threadIdx.x; c < d; c += kPrepThreads) {
    const float t = row[c] - m;
    q += t * t;
  }
  *mean = m;
  *rstd = rsqrtf(block_total(q, red) / (float)d + eps);
}

// the sum over `splits` partial rows (split stride `stride`) at one column, all loads in flight together
__device__ __forceinline__ float split_sum(const float* p, int splits, int64_t stride) {
  float v[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) v[s] = s < splits ? p[s * stride] : 0.f;
  float y = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) y += v[s];
  return y;
}

__global__ __launch_bounds__(kPrepThreads) void k_prep_mix(const float* h, int64_t ldh, const float* ring,
                                                           const int64_t* pos_p, const float* w, const float* bia,
                                                           float eps, int d, int k, float* z, float* x1) {
  __shared__ float red[kPrepWaves];
  const int64_t b = blockIdx.x;
  const float* row = h + b * ldh;
  float m, r;
  row_stats(row, d, eps, red, &m, &r);
  const int km1 = k - 1;
  const int64_t pos = *pos_p;
  for (int c = threadIdx.x; c < d; c += kPrepThreads) {
    const float zc = (row[c] - m) * r * w[c] + bia[c];
    z[b * d + c] = zc;
    float* xr = x1 + (b * d + c) * k;
    for (int j = 0; j < km1; ++j) xr[j] = ring[(b * d + c) * km1 + (pos + j) % km1];
    xr[km1] = zc;
  }
}

// h1 = h + GELU(sum of the splits + bias), then X2 = LayerNorm2(h1), one row per workgroup
__global__ __launch_bounds__(kPrepThreads) void k_finish_mix(const float* part, int splits, int64_t B,
                                                             const float* bias, const float* h, int64_t ldh,
                                                             const float* w2, const float* b2, float eps, int d,
                                                             float* h1, float* x2) {
  __shared__ float red[kPrepWaves];
  const int64_t b = blockIdx.x;
  for (int c = threadIdx.x; c < d; c += kPrepThreads)
    h1[b * d + c] = h[b * ldh + c] + gelu_erf(split_sum(part + b * d + c, splits, B * d) + bias[c]);
  __syncthreads();
  float m, r;
  row_stats(h1 + b * d, d, eps, red, &m, &r);
  for (int c = threadIdx.x; c < d; c += kPrepThreads) x2[b * d + c] = (h1[b * d + c] - m) * r * w2[c] + b2[c];
}

// out = h1 + sum of the splits + bias; z enters the ring, one row per workgroup
__global__ __launch_bounds__(kPrepThreads) void k_finish_res(const float* part, int splits, int64_t B,
                                                             const float* bias, const float* h1, const float* z,
                                                             const int64_t* pos_p, int d, int km1, float* ring,
                                                             float* out) {
  const int64_t b = blockIdx.x;
  const int slot = km1 > 0 ? (int)(*pos_p % km1) : 0;
  for (int c = threadIdx.x; c < d; c += kPrepThreads) {
    out[b * d + c] = h1[b * d + c] + (split_sum(part + b * d + c, splits, B * d) + bias[c]);
    if (km1 > 0) ring[(b * d + c) * km1 + slot] = z[b * d + c];
  }
}

struct Part {
  const float* x;          // (B, K) operand rows, or (splits_x, B, K) partials when x_splits > 0
  int x_splits;            // > 0: the operand is GELU(sum of x's splits + x_bias)
  const float* x_bias;
  const float* w;          // (N, K)
  float* part;             // (splits, B, N) out
  int B, K, N, splits;
};

// 4 values of row `row` of a (nrows, ld) matrix, columns [k, k + 4) clipped to [.., kend); zero outside
__device__ __forceinline__ f4 load4(const float* m, int64_t row, int64_t nrows, int64_t ld, int k, int kend) {
  f4 v = {0.f, 0.f, 0.f, 0.f};
  if (row >= nrows) return v;
  const float* p = m + row * ld + k;
  if (k + 4 <= kend && (((uintptr_t)p) & 15) == 0) return *(const f4*)p;
  if (k + 0 < kend) v.x = p[0];
  if (k + 1 < kend) v.y = p[1];
  if (k + 2 < kend) v.z = p[2];
  if (k + 3 < kend) v.w = p[3];
  return v;
}

__device__ __forceinline__ f4 operand(const Part& g, int64_t row, int k, int kend) {
  if (g.x_splits == 0) return load4(g.x, row, g.B, g.K, k, kend);
  f4 y = {0.f, 0.f, 0.f, 0.f};
  if (row >= g.B) return y;
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s)
    if (s < g.x_splits) y += load4(g.x + (int64_t)s * g.B * g.K, row, g.B, g.K, k, kend);
  f4 bb = load4(g.x_bias, 0, 1, g.K, k, kend);
  f4 o;
  o.x = k + 0 < kend ? gelu_erf(y.x + bb.x) : 0.f;
  o.y = k + 1 < kend ? gelu_erf(y.y + bb.y) : 0.f;
  o.z = k + 2 < kend ? gelu_erf(y.z + bb.z) : 0.f;
  o.w = k + 3 < kend ? gelu_erf(y.w + bb.w) : 0.f;
  return o;
}

__global__ __launch_bounds__(kGemvThreads) void k_part(Part g) {
  __shared__ float tile[kGemvWaves][kTile * kTile];
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int nt = blockIdx.x, s = blockIdx.y, rt = blockIdx.z;
  const int n0 = nt * kTile, r0 = rt * kTile;
  // this workgroup's depth range, then this wave's quarter of it, in steps of 16
  const int per_split = ((g.K + g.splits - 1) / g.splits + 15) & ~15;
  const int kb = s * per_split, ke = kb + per_split < g.K ? kb + per_split : g.K;
  const int per_wave = ((ke - kb + kGemvWaves - 1) / kGemvWaves + 15) & ~15;
  const int wb = kb + wave * per_wave, we = wb + per_wave < ke ? wb + per_wave : ke;
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  const int i16 = lane & 15, q4 = lane >> 4;
  for (int k = wb; k < we; k += 64) {
    f4 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {                     // four steps of loads in flight before their products
      const int kk = k + 16 * u + 4 * q4;
      a[u] = operand(g, r0 + i16, kk, we);
      b[u] = load4(g.w, n0 + i16, g.N, g.K, kk, we);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].x, b[u].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].y, b[u].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].z, b[u].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].w, b[u].w, acc, 0, 0, 0);
    }
  }
  // lane l holds output rows 4 (l / 16) + q, column l % 16
#pragma unroll
  for (int q = 0; q < 4; ++q) tile[wave][(4 * q4 + q) * kTile + i16] = acc[q];
  __syncthreads();
  const int e = threadIdx.x;                          // 256 threads: one output element each
  const int b = r0 + e / kTile, n = n0 + e % kTile;
  if (b < g.B && n < g.N)
    g.part[((int64_t)s * g.B + b) * g.N + n] = ((tile[0][e] + tile[1][e]) + tile[2][e]) + tile[3][e];
}

// depth splits: each wavefront's share at most 64 columns (one round of loads), at most kMaxSplits
int splits_for(int N, int K) {
  (void)N;
  int s = (K + 4 * 64 - 1) / (4 * 64);
  return s < 1 ? 1 : (s > kMaxSplits ? kMaxSplits : s);
}

int launch_part(Part g, hipStream_t st, const char* what) {
  const dim3 grid((unsigned)((g.N + kTile - 1) / kTile), (unsigned)g.splits, (unsigned)((g.B + kTile - 1) / kTile));
  hipLaunchKernelGGL(k_part, grid, dim3(kGemvThreads), 0, st, g);
  return check_launch(what);
}

}  // namespace
}  // namespace asrn

using namespace asrn;

extern "C" int64_t asrn_block_step_workspace(int64_t B, int32_t d, int32_t ff) {
  // the three products' partials, (splits, B, N) floats each (the first sized for the most splits)
  return 4 * B * ((int64_t)kMaxSplits * d + (int64_t)splits_for(ff, d) * ff + (int64_t)splits_for(d, ff) * d);
}

extern "C" int asrn_block_step(const float* h, int64_t ldh, float* ring, const int64_t* pos, int64_t B, int32_t d,
                               int32_t k, int32_t ff, const float* ln1_w, const float* ln1_b, const float* conv_w,
                               const float* conv_b, const float* ln2_w, const float* ln2_b, const float* w1,
                               const float* b1, const float* w2, const float* b2, float eps, float* z, float* x1,
                               float* h1, float* x2, float* out, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  ASRN_REQUIRE(B >= 1 && B <= (int64_t(1) << 20) && d >= 1 && k >= 1 && ff >= 1 && ldh >= d,
               "asrn_block_step: bad sizes B=%lld d=%d k=%d ff=%d", (long long)B, d, k, ff);
  ASRN_REQUIRE((int64_t)d * k <= (int64_t(1) << 30) && ff <= (1 << 30), "asrn_block_step: sizes too large");
  ASRN_REQUIRE(h && pos && ln1_w && ln1_b && conv_w && conv_b && ln2_w && ln2_b && w1 && b1 && w2 && b2 && z && x1 &&
               h1 && x2 && out && (k == 1 || ring), "asrn_block_step: null pointer");
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= asrn_block_step_workspace(B, d, ff),
               "asrn_block_step: workspace of %lld bytes needed (asrn_block_step_workspace)",
               (long long)asrn_block_step_workspace(B, d, ff));
  const hipStream_t st = (hipStream_t)stream;
  const int s1 = splits_for(d, d * k), s2 = splits_for(ff, d), s3 = splits_for(d, ff);
  float* p1 = (float*)workspace;
  float* p2 = p1 + (int64_t)kMaxSplits * B * d;
  float* p3 = p2 + (int64_t)s2 * B * ff;
  hipLaunchKernelGGL(k_prep_mix, dim3((unsigned)B), dim3(kPrepThreads), 0, st, h, ldh, ring, pos, ln1_w, ln1_b, eps, d,
                     k, z, x1);
  if (int rc = check_launch("asrn_block_step (prep)")) return rc;
  if (int rc = launch_part(Part{x1, 0, nullptr, conv_w, p1, (int)B, d * k, d, s1}, st, "asrn_block_step (conv)"))
    return rc;
  hipLaunchKernelGGL(k_finish_mix, dim3((unsigned)B), dim3(kPrepThreads), 0, st, p1, s1, B, conv_b, h, ldh, ln2_w,
                     ln2_b, eps, d, h1, x2);
  if (int rc = check_launch("asrn_block_step (mix)")) return rc;
  if (int rc = launch_part(Part{x2, 0, nullptr, w1, p2, (int)B, d, ff, s2}, st, "asrn_block_step (ff1)")) return rc;
  if (int rc = launch_part(Part{p2, s2, b1, w2, p3, (int)B, ff, d, s3}, st, "asrn_block_step (ff2)")) return rc;
  hipLaunchKernelGGL(k_finish_res, dim3((unsigned)B), dim3(kPrepThreads), 0, st, p3, s3, B, b2, h1, z, pos, d, k - 1,
                     ring, out);
  return check_launch("asrn_block_step (residual)");
}
