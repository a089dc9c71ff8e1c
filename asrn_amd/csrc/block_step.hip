// The local block's generation step (asrn/nucleo.py:1811-1814; the model's BloqueLocal, nucleo:969-1014, mezcla
// 'conv') for the few rows of a decode batch, in six launches:
//   k_prep_mix    per row: z = LayerNorm1(h) and X1 = [the ring's k - 1 taps; z] in nn.Conv1d's column order
//                 (column c*k + j: channel c, tap j)
//   k_part        P1 = X1 conv_w^T, in depth splits
//   k_finish_mix  per row: h1 = h + GELU(sum of P1 + conv_b); X2 = LayerNorm2(h1)
//   k_part        H = GELU(X2 w1^T + b1) over the whole depth (no splits), the bias and GELU in its epilogue
//   k_part        P3 = H w2^T, in depth splits
//   k_finish_res  per row: out = h1 + sum of P3 + b2; z enters the ring at slot pos mod (k - 1)
// The ring holds row t (t = position) at slot t mod (k - 1), so tap j of position pos (j = 0 oldest, k - 2 newest) is
// at slot (pos + j) mod (k - 1) and nothing shifts. The position is read on the device (a captured step advances it).
//
// The products (16 rows at most per tile) run on the matrix cores in fp32 (v_mfma_f32_16x16x4f32): a workgroup owns a
// 16 x 16 output tile over one split of the depth, its four wavefronts a quarter each, every lane loading a float4 of
// the weight row and of the operand row per 16 columns of depth (the weights stream once, coalesced). The splits are
// sized so that a wavefront's share is one round of loads issued ahead of its products (at most 64 columns); the
// first feed-forward product takes its whole depth in one workgroup instead (a wavefront's quarter, up to 256 columns,
// in one round of loads), so that its epilogue can add the bias and apply the GELU once per element and the second
// product reads a plain operand. The wavefronts' tiles are summed in LDS; the splits are summed by the next kernel, in
// split order: deterministic, and no workgroup waits for another (across the chip's eight L2 caches a device-wide
// fence costs more than these products).
//
// The row kernels hold their row in registers (up to kRowVals values a thread), so that the LayerNorm statistics and
// the outputs need no second read of what they loaded or wrote.
#include "block_pending.h"

namespace asrn {
namespace {

constexpr int kTile = 16;
constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kPrepThreads = 1024;
constexpr int kPrepWaves = kPrepThreads / kWave;

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

constexpr int kRowVals = 4;                 // row values a thread holds: rows up to 4,096 columns

// mean and 1/sqrt(var + eps) of a row of width d whose column tid + j * kPrepThreads is v[j] in thread tid (two-pass
// variance; every thread gets the results)
template <int R>
__device__ void row_stats(const float (&v)[R], int d, float eps, float* red, float* mean, float* rstd) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j)
    if ((int)threadIdx.x + j * kPrepThreads < d) s += v[j];
  const float m = block_total(s, red) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j)
    if ((int)threadIdx.x + j * kPrepThreads < d) {
      const float t = v[j] - m;
      q += t * t;
    }
  *mean = m;
  *rstd = rsqrtf(block_total(q, red) / (float)d + eps);
}

// The row kernels below hold R columns a thread (column tid + j kPrepThreads, R = ceil(d / kPrepThreads)) and issue
// every load before its first use as unconditional loads (split_loads).

constexpr int kMaxTaps = 8;                  // ring taps a thread loads ahead of the statistics (k - 1 <= 8)

// With PEND: the row is the pending block's output h1 + (sum of the splits + bias), formed as k_finish_res forms it,
// written to pv.out, and the pending block's z enters its ring (k_finish_res's work, one row per workgroup).
// pos_next (with the count `done`, 0 between launches): the position advanced to *pos_p + 1 once every workgroup has
// used it: each workgroup, past a barrier after its last use, adds 1 to the count, and the one that reads gridDim.x
// - 1 stores the new position and sets the count back to 0 (nothing waits on the count).
template <int R, int S, bool PEND>
__global__ __launch_bounds__(kPrepThreads) void k_prep_mix(const float* h, int64_t ldh, Pending pv, const float* ring,
                                                           const int64_t* pos_p, const float* w, const float* bia,
                                                           float eps, int d, int k, float* z, float* x1,
                                                           int64_t* pos_next, int32_t* done) {
  __shared__ float red[kPrepWaves];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int km1 = k - 1;
  const int64_t pos = *pos_p;
  const int first = km1 > 0 ? (int)(pos % km1) : 0;        // the slot of tap 0; tap i is at (first + i) mod (k - 1)
  auto slot = [&](int i) { return first + i < km1 ? first + i : first + i - km1; };
  // the row (or the pending block's parts), the LayerNorm's weights and, for k <= 9, the ring taps
  float x[R], lw[R], lb[R], tap[R][kMaxTaps], sp[R][S], pb[R], zp[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int c = tid + j * kPrepThreads, cc = c < d ? c : d - 1;
    lw[j] = w[cc];
    lb[j] = bia[cc];
    if constexpr (PEND) {
      x[j] = pv.h1[b * d + cc];
      split_loads<S>(pv.part + b * d + cc, pv.splits, gridDim.x * (int64_t)d, sp[j]);
      pb[j] = pv.bias[cc];
      zp[j] = pv.km1 > 0 ? pv.z[b * d + cc] : 0.f;
    } else {
      x[j] = h[b * ldh + cc];
    }
    if (km1 > 0) {
#pragma unroll
      for (int i = 0; i < kMaxTaps; ++i) tap[j][i] = ring[(b * d + cc) * km1 + slot(i < km1 ? i : km1 - 1)];
    }
  }
  float v[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if constexpr (PEND)
      v[j] = x[j] + (split_total<S>(sp[j], pv.splits) + pb[j]);
    else
      v[j] = x[j];
  }
  if constexpr (PEND) {
    const int ps = pv.km1 > 0 ? (int)(pos % pv.km1) : 0;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int c = tid + j * kPrepThreads;
      if (c >= d) continue;
      pv.out[b * d + c] = v[j];
      if (pv.km1 > 0) pv.ring[(b * d + c) * pv.km1 + ps] = zp[j];
    }
  }
  float m, r;
  row_stats<R>(v, d, eps, red, &m, &r);
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int c = tid + j * kPrepThreads;
    if (c >= d) continue;
    const float zc = (v[j] - m) * r * lw[j] + lb[j];
    z[b * d + c] = zc;
    float* xr = x1 + (b * d + c) * k;
#pragma unroll
    for (int i = 0; i < kMaxTaps; ++i)
      if (i < km1) xr[i] = tap[j][i];
    for (int i = kMaxTaps; i < km1; ++i) xr[i] = ring[(b * d + c) * km1 + slot(i)];
    xr[km1] = zc;
  }
  if (pos_next) {
    __syncthreads();
    if (tid == 0 && atomicAdd(done, 1) == (int)gridDim.x - 1) {
      *pos_next = pos + 1;
      atomicExch(done, 0);
    }
  }
}

// h1 = h + GELU(sum of the splits + bias), then X2 = LayerNorm2(h1), one row per workgroup
template <int R, int S>
__global__ __launch_bounds__(kPrepThreads) void k_finish_mix(const float* part, int splits, int64_t B,
                                                             const float* bias, const float* h, int64_t ldh,
                                                             const float* w2, const float* b2, float eps, int d,
                                                             float* h1, float* x2) {
  __shared__ float red[kPrepWaves];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  float x[R], lw[R], lb[R], bs[R], sp[R][S];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int c = tid + j * kPrepThreads, cc = c < d ? c : d - 1;
    lw[j] = w2[cc];
    lb[j] = b2[cc];
    x[j] = h[b * ldh + cc];
    bs[j] = bias[cc];
    split_loads<S>(part + b * d + cc, splits, B * d, sp[j]);
  }
  float v[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int c = tid + j * kPrepThreads;
    v[j] = x[j] + gelu_erf(split_total<S>(sp[j], splits) + bs[j]);
    if (c < d) h1[b * d + c] = v[j];
  }
  float m, r;
  row_stats<R>(v, d, eps, red, &m, &r);
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int c = tid + j * kPrepThreads;
    if (c < d) x2[b * d + c] = (v[j] - m) * r * lw[j] + lb[j];
  }
}

// out = h1 + sum of the splits + bias; z enters the ring, one row per workgroup
template <int R, int S>
__global__ __launch_bounds__(kPrepThreads) void k_finish_res(const float* part, int splits, int64_t B,
                                                             const float* bias, const float* h1, const float* z,
                                                             const int64_t* pos_p, int d, int km1, float* ring,
                                                             float* out) {
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int slot = km1 > 0 ? (int)(*pos_p % km1) : 0;
  float x[R], bs[R], zv[R], sp[R][S];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int c = tid + j * kPrepThreads, cc = c < d ? c : d - 1;
    x[j] = h1[b * d + cc];
    bs[j] = bias[cc];
    zv[j] = km1 > 0 ? z[b * d + cc] : 0.f;
    split_loads<S>(part + b * d + cc, splits, B * d, sp[j]);
  }
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int c = tid + j * kPrepThreads;
    if (c >= d) continue;
    out[b * d + c] = x[j] + (split_total<S>(sp[j], splits) + bs[j]);
    if (km1 > 0) ring[(b * d + c) * km1 + slot] = zv[j];
  }
}

struct Part {
  const float* x;          // (B, K) operand rows
  const float* w;          // (N, K)
  float* part;             // (splits, B, N) out; with an epilogue (B, N) = GELU(sum + bias)
  const float* bias;       // the epilogue's bias (N), or null: no epilogue
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

// One 16 x 16 output tile over one depth split; each of the NW wavefronts an NW-th of the split, U steps of 16 columns
// of loads issued ahead of their products. With g.bias the workgroup owns the whole depth (splits == 1) and writes
// GELU(sum + bias); it then runs eight wavefronts, so that twice the loads are in flight on its CU.
template <int U, int NW>
__global__ __launch_bounds__(NW * kWave) void k_part(Part g) {
  __shared__ float tile[NW][kTile * kTile];
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int nt = blockIdx.x, s = blockIdx.y, rt = blockIdx.z;
  const int n0 = nt * kTile, r0 = rt * kTile;
  // this workgroup's depth range, then this wave's quarter of it, in steps of 16
  const int per_split = ((g.K + g.splits - 1) / g.splits + 15) & ~15;
  const int kb = s * per_split, ke = kb + per_split < g.K ? kb + per_split : g.K;
  const int per_wave = ((ke - kb + NW - 1) / NW + 15) & ~15;
  const int wb = kb + wave * per_wave, we = wb + per_wave < ke ? wb + per_wave : ke;
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  const int i16 = lane & 15, q4 = lane >> 4;
  for (int k = wb; k < we; k += 16 * U) {
    f4 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {                     // U steps of loads in flight before their products
      const int kk = k + 16 * u + 4 * q4;
      a[u] = load4(g.x, r0 + i16, g.B, g.K, kk, we);
      b[u] = load4(g.w, n0 + i16, g.N, g.K, kk, we);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
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
  const int e = threadIdx.x;                          // the first 256 threads: one output element each
  if (e >= kTile * kTile) return;
  const int b = r0 + e / kTile, n = n0 + e % kTile;
  if (b < g.B && n < g.N) {
    float y = tile[0][e];
#pragma unroll
    for (int w = 1; w < NW; ++w) y += tile[w][e];
    if (g.bias)
      g.part[(int64_t)b * g.N + n] = gelu_erf(y + g.bias[n]);
    else
      g.part[((int64_t)s * g.B + b) * g.N + n] = y;
  }
}

// the row kernels' instances: R columns a thread (ceil(d / kPrepThreads)) and S loads for at most S splits
using PrepFn = void (*)(const float*, int64_t, Pending, const float*, const int64_t*, const float*, const float*, float,
                        int, int, float*, float*, int64_t*, int32_t*);
using MixFn = void (*)(const float*, int, int64_t, const float*, const float*, int64_t, const float*, const float*,
                       float, int, float*, float*);
using ResFn = void (*)(const float*, int, int64_t, const float*, const float*, const float*, const int64_t*, int, int,
                       float*, float*);

template <int R>
PrepFn prep_fn_r(bool pend, int S) {
  if (!pend) return k_prep_mix<R, 4, false>;
  return S == 4 ? k_prep_mix<R, 4, true> : (S == 8 ? k_prep_mix<R, 8, true> : k_prep_mix<R, 16, true>);
}
PrepFn prep_fn(int R, bool pend, int splits) {
  const int S = split_cap(splits);
  return R == 1 ? prep_fn_r<1>(pend, S) : (R == 2 ? prep_fn_r<2>(pend, S) : (R == 3 ? prep_fn_r<3>(pend, S)
                                                                              : prep_fn_r<4>(pend, S)));
}
template <int R>
MixFn mix_fn_r(int S) {
  return S == 4 ? k_finish_mix<R, 4> : (S == 8 ? k_finish_mix<R, 8> : k_finish_mix<R, 16>);
}
MixFn mix_fn(int R, int splits) {
  const int S = split_cap(splits);
  return R == 1 ? mix_fn_r<1>(S) : (R == 2 ? mix_fn_r<2>(S) : (R == 3 ? mix_fn_r<3>(S) : mix_fn_r<4>(S)));
}
template <int R>
ResFn res_fn_r(int S) {
  return S == 4 ? k_finish_res<R, 4> : (S == 8 ? k_finish_res<R, 8> : k_finish_res<R, 16>);
}
ResFn res_fn(int R, int splits) {
  const int S = split_cap(splits);
  return R == 1 ? res_fn_r<1>(S) : (R == 2 ? res_fn_r<2>(S) : (R == 3 ? res_fn_r<3>(S) : res_fn_r<4>(S)));
}

int launch_part(Part g, hipStream_t st, const char* what) {
  const dim3 grid((unsigned)((g.N + kTile - 1) / kTile), (unsigned)g.splits, (unsigned)((g.B + kTile - 1) / kTile));
  if (g.bias) {
    // the whole depth in one workgroup of 8 wavefronts: a wavefront's eighth in rounds of up to 12 steps of 16
    const int per_wave = ((g.K + 8 - 1) / 8 + 15) & ~15;
    if (per_wave <= 16 * 4)
      hipLaunchKernelGGL((k_part<4, 8>), grid, dim3(8 * kWave), 0, st, g);
    else if (per_wave <= 16 * 8)
      hipLaunchKernelGGL((k_part<8, 8>), grid, dim3(8 * kWave), 0, st, g);
    else
      hipLaunchKernelGGL((k_part<12, 8>), grid, dim3(8 * kWave), 0, st, g);
  } else {
    hipLaunchKernelGGL((k_part<4, kGemvWaves>), grid, dim3(kGemvThreads), 0, st, g);
  }
  return check_launch(what);
}

}  // namespace
}  // namespace asrn

using namespace asrn;

extern "C" int64_t asrn_block_step_workspace(int64_t B, int32_t d, int32_t ff) {
  // the conv and second feed-forward products' partials, (splits, B, N) floats each (the first sized for the most
  // splits), and the hidden layer (B, ff)
  return 4 * block_workspace_floats(B, d, ff);
}

namespace asrn {
namespace {

int block_step(const float* h, int64_t ldh, const float* prev_h1, const float* prev_b2, const float* prev_z,
               float* prev_ring, int32_t prev_k, int32_t prev_ff, float* prev_out, float* ring, const int64_t* pos,
               int64_t B, int32_t d, int32_t k, int32_t ff, const float* ln1_w, const float* ln1_b,
               const float* conv_w, const float* conv_b, const float* ln2_w, const float* ln2_b, const float* w1,
               const float* b1, const float* w2, const float* b2, float eps, float* z, float* x1, float* h1, float* x2,
               float* out, int32_t finish, void* workspace, int64_t workspace_bytes, hipStream_t st,
               const char* what) {
  ASRN_REQUIRE(B >= 1 && B <= (int64_t(1) << 20) && d >= 1 && k >= 1 && ff >= 1 && (prev_h1 || ldh >= d),
               "%s: bad sizes B=%lld d=%d k=%d ff=%d", what, (long long)B, d, k, ff);
  ASRN_REQUIRE((int64_t)d * k <= (int64_t(1) << 30) && ff <= (1 << 30), "%s: sizes too large", what);
  ASRN_REQUIRE(d <= kRowVals * kPrepThreads, "%s: d=%d above %d", what, d, kRowVals * kPrepThreads);
  ASRN_REQUIRE((h || prev_h1) && pos && ln1_w && ln1_b && conv_w && conv_b && ln2_w && ln2_b && w1 && b1 && w2 &&
               b2 && z && x1 && h1 && x2 && out && (k == 1 || ring), "%s: null pointer", what);
  ASRN_REQUIRE(!prev_h1 || (prev_b2 && prev_z && prev_out && prev_k >= 1 && prev_ff >= 1 && prev_ff <= (1 << 30) &&
                            (prev_k == 1 || prev_ring)),
               "%s: a pending block needs its b2, z, out, k >= 1, ff >= 1 and (k > 1) its ring", what);
  const int64_t need = asrn_block_step_workspace(B, d, prev_h1 && prev_ff > ff ? prev_ff : ff);
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= need,
               "%s: workspace of %lld bytes needed (asrn_block_step_workspace)", what, (long long)need);
  const int s1 = splits_for(d * k), s3 = splits_for(ff);
  float* p1 = (float*)workspace;
  float* hid = block_hidden(workspace, B, d);
  float* p3 = block_second_parts(workspace, B, d, ff);
  Pending pv = {};
  if (prev_h1)   // the pending block's partials, where its call (same workspace, same B and d) left them
    pv = Pending{block_second_parts(workspace, B, d, prev_ff), splits_for(prev_ff), prev_b2, prev_h1, prev_z,
                 prev_ring, prev_k - 1, prev_out};
  const int R = (d + kPrepThreads - 1) / kPrepThreads;
  hipLaunchKernelGGL(prep_fn(R, prev_h1 != nullptr, pv.splits), dim3((unsigned)B), dim3(kPrepThreads), 0, st,
                     prev_h1 ? prev_out : h, prev_h1 ? (int64_t)d : ldh, pv, ring, pos, ln1_w, ln1_b, eps, d, k, z, x1,
                     nullptr, nullptr);
  if (int rc = check_launch(what)) return rc;
  if (int rc = launch_part(Part{x1, conv_w, p1, nullptr, (int)B, d * k, d, s1}, st, what)) return rc;
  // the residual input h: the pending block's output, which k_prep_mix wrote, or h itself
  hipLaunchKernelGGL(mix_fn(R, s1), dim3((unsigned)B), dim3(kPrepThreads), 0, st, p1, s1, B, conv_b,
                     prev_h1 ? prev_out : h, prev_h1 ? (int64_t)d : ldh, ln2_w, ln2_b, eps, d, h1, x2);
  if (int rc = check_launch(what)) return rc;
  if (int rc = launch_part(Part{x2, w1, hid, b1, (int)B, d, ff, 1}, st, what)) return rc;
  if (int rc = launch_part(Part{hid, w2, p3, nullptr, (int)B, ff, d, s3}, st, what)) return rc;
  if (!finish) return 0;                           // k_finish_res's work left to the next block's k_prep_mix
  hipLaunchKernelGGL(res_fn(R, s3), dim3((unsigned)B), dim3(kPrepThreads), 0, st, p3, s3, B, b2, h1, z, pos, d, k - 1,
                     ring, out);
  return check_launch(what);
}

}  // namespace
}  // namespace asrn

extern "C" int asrn_block_step(const float* h, int64_t ldh, float* ring, const int64_t* pos, int64_t B, int32_t d,
                               int32_t k, int32_t ff, const float* ln1_w, const float* ln1_b, const float* conv_w,
                               const float* conv_b, const float* ln2_w, const float* ln2_b, const float* w1,
                               const float* b1, const float* w2, const float* b2, float eps, float* z, float* x1,
                               float* h1, float* x2, float* out, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  ASRN_REQUIRE(h, "asrn_block_step: null pointer");
  return block_step(h, ldh, nullptr, nullptr, nullptr, nullptr, 0, 0, nullptr, ring, pos, B, d, k, ff, ln1_w, ln1_b,
                    conv_w, conv_b, ln2_w, ln2_b, w1, b1, w2, b2, eps, z, x1, h1, x2, out, 1, workspace,
                    workspace_bytes, (hipStream_t)stream, "asrn_block_step");
}

extern "C" int asrn_block_step_ex(const float* h, int64_t ldh, const float* prev_h1, const float* prev_b2,
                                  const float* prev_z, float* prev_ring, int32_t prev_k, int32_t prev_ff,
                                  float* prev_out, float* ring, const int64_t* pos, int64_t B, int32_t d, int32_t k,
                                  int32_t ff, const float* ln1_w, const float* ln1_b, const float* conv_w,
                                  const float* conv_b, const float* ln2_w, const float* ln2_b, const float* w1,
                                  const float* b1, const float* w2, const float* b2, float eps, float* z, float* x1,
                                  float* h1, float* x2, float* out, int32_t finish, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  return block_step(h, ldh, prev_h1, prev_b2, prev_z, prev_ring, prev_k, prev_ff, prev_out, ring, pos, B, d, k, ff,
                    ln1_w, ln1_b, conv_w, conv_b, ln2_w, ln2_b, w1, b1, w2, b2, eps, z, x1, h1, x2, out, finish,
                    workspace, workspace_bytes, (hipStream_t)stream, "asrn_block_step_ex");
}

extern "C" int asrn_block_finish_norm(const float* prev_h1, const float* prev_b2, const float* prev_z,
                                      float* prev_ring, int32_t prev_k, int32_t prev_ff, float* prev_out,
                                      const int64_t* pos, int64_t B, int32_t d, const float* ln_w, const float* ln_b,
                                      float eps, float* y, void* workspace, int64_t workspace_bytes, int64_t* pos_next,
                                      int32_t* done, void* stream) {
  ASRN_REQUIRE(B >= 1 && B <= (int64_t(1) << 20) && d >= 1 && d <= kRowVals * kPrepThreads,
               "asrn_block_finish_norm: bad sizes B=%lld d=%d (d <= %d)", (long long)B, d, kRowVals * kPrepThreads);
  ASRN_REQUIRE(prev_h1 && prev_b2 && prev_z && prev_out && pos && ln_w && ln_b && y && prev_k >= 1 && prev_ff >= 1 &&
                   prev_ff <= (1 << 30) && (prev_k == 1 || prev_ring),
               "asrn_block_finish_norm: a pending block needs its h1, b2, z, out, k >= 1, ff >= 1 and (k > 1) its "
               "ring, and the norm its weights and output (null pointer)");
  const int64_t need = 4 * block_workspace_floats(B, d, prev_ff);
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= need,
               "asrn_block_finish_norm: the pending block's workspace of %lld bytes needed (asrn_block_step_workspace)",
               (long long)need);
  ASRN_REQUIRE(!pos_next || done, "asrn_block_finish_norm: advancing the position needs its count (done)");
  const Pending pv{block_second_parts(workspace, B, d, prev_ff), splits_for(prev_ff), prev_b2, prev_h1, prev_z,
                   prev_ring, prev_k - 1, prev_out};
  // the row kernel of a block that follows a pending one, with one tap (k = 1): its LayerNorm row is the output, and
  // its conv operand [z] the same values at the same addresses
  const int R = (d + kPrepThreads - 1) / kPrepThreads;
  hipLaunchKernelGGL(prep_fn(R, true, pv.splits), dim3((unsigned)B), dim3(kPrepThreads), 0, (hipStream_t)stream,
                     prev_out, (int64_t)d, pv, nullptr, pos, ln_w, ln_b, eps, d, 1, y, y, pos_next, done);
  return check_launch("asrn_block_finish_norm");
}
