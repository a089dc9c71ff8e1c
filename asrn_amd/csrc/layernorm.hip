// The model's LayerNorms (the local blocks' ln1 / ln2 and the final ln_f; reference asrn/nucleo.py:969-1014, 1047-1125),
// as torch.nn.LayerNorm computes them in fp32 (biased variance, rstd = 1 / sqrt(var + eps)), with two things fused:
//   forward   y = (x - mean) rstd gamma + beta written in fp32 or straight in bf16 (rounded to nearest even, as the cast
//             that autocast puts before the next bf16 product rounds), and (mean, rstd) kept per row;
//   backward  from dy (fp32 or bf16): g = dy gamma, dx = rstd (g - mean(g) - xhat mean(g xhat)) [+ dres, the gradient
//             of the same x through the residual path, so that autograd adds nothing], and d gamma = sum dy xhat,
//             d beta = sum dy as per-workgroup partial rows summed in a fixed order by asrn_column_sums.
// Forward: a workgroup takes 8 rows, each wave 2 with both rows (float4 per lane) loaded at once. Backward: a workgroup
// takes 32 rows, each wave 8 of them, 2 rows' loads at a time.
#include "common.h"

namespace asrn {

constexpr int kLnThreads = 256;
constexpr int kLnWaves = kLnThreads / kWave;
constexpr int kLnFwdRows = 8;
constexpr int kLnFwdPerWave = kLnFwdRows / kLnWaves;
constexpr int kLnBwdRows = 32;
constexpr int kLnBwdPerWave = kLnBwdRows / kLnWaves;
constexpr int kLnBatch = 2;
constexpr int kLnMaxD4 = 4;      // d <= 1024

struct LnArgs {
  const float* x; int64_t ldx; const float* gamma; const float* beta;
  int64_t rows; int d; float eps;
  void* y; int64_t ldy; float2* stats;                                   // forward
  const void* dy; int64_t lddy; const float* dres; float* dx; float* partial;   // backward (dx and dres: ldx)
};

__device__ __forceinline__ uint32_t ln_bf16(float v) {
  const uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;        // NaN stays a (quiet) NaN
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float4 ld_row4(const void* p, bool b16, int64_t off4) {
  if (b16) {
    const uint2 u = reinterpret_cast<const uint2*>(p)[off4];
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
  }
  return reinterpret_cast<const float4*>(p)[off4];
}
__device__ __forceinline__ float ln_dot4(float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }

template <int D4, bool OB16>
__global__ __launch_bounds__(kLnThreads) void k_ln_fwd(LnArgs a) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  const float inv_d = 1.f / (float)a.d;
  const int64_t r0 = (int64_t)blockIdx.x * kLnFwdRows + wave * kLnFwdPerWave;
  float4 xv[kLnFwdPerWave][D4];
  float s[kLnFwdPerWave];
#pragma unroll
  for (int u = 0; u < kLnFwdPerWave; ++u) {
    const int64_t r = r0 + u;
    s[u] = 0.f;
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      const int q = lane + kWave * k;
      xv[u][k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (r < a.rows && q < d4) {
        xv[u][k] = reinterpret_cast<const float4*>(a.x + r * a.ldx)[q];
        s[u] += (xv[u][k].x + xv[u][k].y) + (xv[u][k].z + xv[u][k].w);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kLnFwdPerWave; ++u) {
    const int64_t r = r0 + u;
    if (r >= a.rows) break;
    const float mean = wave_sum_u(s[u]) * inv_d;
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      const int q = lane + kWave * k;
      if (q < d4) {
        const float4 c = make_float4(xv[u][k].x - mean, xv[u][k].y - mean, xv[u][k].z - mean, xv[u][k].w - mean);
        v += ln_dot4(c, c);
      }
    }
    const float rstd = rsqrtf(wave_sum_u(v) * inv_d + a.eps);
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      const int q = lane + kWave * k;
      if (q < d4) {
        const float4 w = reinterpret_cast<const float4*>(a.gamma)[q], b = reinterpret_cast<const float4*>(a.beta)[q];
        const float4 y = make_float4((xv[u][k].x - mean) * rstd * w.x + b.x, (xv[u][k].y - mean) * rstd * w.y + b.y,
                                     (xv[u][k].z - mean) * rstd * w.z + b.z, (xv[u][k].w - mean) * rstd * w.w + b.w);
        if constexpr (OB16) {
          reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.y) + r * a.ldy)[q] =
              make_uint2(ln_bf16(y.x) | (ln_bf16(y.y) << 16), ln_bf16(y.z) | (ln_bf16(y.w) << 16));
        } else {
          reinterpret_cast<float4*>(reinterpret_cast<float*>(a.y) + r * a.ldy)[q] = y;
        }
      }
    }
    if (lane == 0) a.stats[r] = make_float2(mean, rstd);
  }
}

template <int D4, bool DB16>
__global__ __launch_bounds__(kLnThreads) void k_ln_bwd(LnArgs a) {
  __shared__ float red[kLnWaves][2 * 4 * D4 * kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  const float inv_d = 1.f / (float)a.d;
  const int64_t r0 = (int64_t)blockIdx.x * kLnBwdRows + wave * kLnBwdPerWave;
  float4 gw[D4], gb[D4];
#pragma unroll
  for (int k = 0; k < D4; ++k) gw[k] = gb[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int b = 0; b < kLnBwdPerWave; b += kLnBatch) {
    float4 xv[kLnBatch][D4], dv[kLnBatch][D4], rv[kLnBatch][D4];
    float2 st[kLnBatch];
#pragma unroll
    for (int u = 0; u < kLnBatch; ++u) {
      const int64_t r = r0 + b + u;
      const bool ok = r < a.rows;
      st[u] = ok ? a.stats[r] : make_float2(0.f, 1.f);
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        xv[u][k] = dv[u][k] = rv[u][k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok && q < d4) {
          xv[u][k] = reinterpret_cast<const float4*>(a.x + r * a.ldx)[q];
          dv[u][k] = DB16 ? ld_row4(reinterpret_cast<const uint16_t*>(a.dy) + r * a.lddy, true, q)
                          : ld_row4(reinterpret_cast<const float*>(a.dy) + r * a.lddy, false, q);
          if (a.dres) rv[u][k] = reinterpret_cast<const float4*>(a.dres + r * a.ldx)[q];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kLnBatch; ++u) {
      const int64_t r = r0 + b + u;
      if (r >= a.rows) break;
      const float mean = st[u].x, rstd = st[u].y;
      float4 xh[D4], g[D4];
      float m1 = 0.f, m2 = 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (q < d4) {
          const float4 w = reinterpret_cast<const float4*>(a.gamma)[q];
          xh[k] = make_float4((xv[u][k].x - mean) * rstd, (xv[u][k].y - mean) * rstd, (xv[u][k].z - mean) * rstd,
                              (xv[u][k].w - mean) * rstd);
          g[k] = make_float4(dv[u][k].x * w.x, dv[u][k].y * w.y, dv[u][k].z * w.z, dv[u][k].w * w.w);
          m1 += (g[k].x + g[k].y) + (g[k].z + g[k].w);
          m2 += ln_dot4(g[k], xh[k]);
          gw[k].x += dv[u][k].x * xh[k].x; gw[k].y += dv[u][k].y * xh[k].y;
          gw[k].z += dv[u][k].z * xh[k].z; gw[k].w += dv[u][k].w * xh[k].w;
          gb[k].x += dv[u][k].x; gb[k].y += dv[u][k].y; gb[k].z += dv[u][k].z; gb[k].w += dv[u][k].w;
        }
      }
      m1 = wave_sum_u(m1) * inv_d;
      m2 = wave_sum_u(m2) * inv_d;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (q < d4)
          reinterpret_cast<float4*>(a.dx + r * a.ldx)[q] =
              make_float4(rstd * (g[k].x - m1 - xh[k].x * m2) + rv[u][k].x, rstd * (g[k].y - m1 - xh[k].y * m2) + rv[u][k].y,
                          rstd * (g[k].z - m1 - xh[k].z * m2) + rv[u][k].z, rstd * (g[k].w - m1 - xh[k].w * m2) + rv[u][k].w);
      }
    }
  }
  // workgroup partial row [d gamma | d beta], the waves in order
  float* mine = red[wave];
#pragma unroll
  for (int k = 0; k < D4; ++k) {
    const int q = lane + kWave * k;
    float* o = mine + 4 * q;
    o[0] = gw[k].x; o[1] = gw[k].y; o[2] = gw[k].z; o[3] = gw[k].w;
    float* ob = mine + 4 * D4 * kWave + 4 * q;
    ob[0] = gb[k].x; ob[1] = gb[k].y; ob[2] = gb[k].z; ob[3] = gb[k].w;
  }
  __syncthreads();
  float* prow = a.partial + (int64_t)blockIdx.x * 2 * a.d;
  for (int c = threadIdx.x; c < 2 * a.d; c += kLnThreads) {
    const int src = c < a.d ? c : 4 * D4 * kWave + (c - a.d);
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kLnWaves; ++w) v += red[w][src];
    prow[c] = v;
  }
}

static int64_t ln_bwd_groups(int64_t rows) { return rows > 0 ? (rows + kLnBwdRows - 1) / kLnBwdRows : 1; }
static int ln_d4(int d) { return (d + 4 * kWave - 1) / (4 * kWave); }

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_layer_norm_fwd(const float* x, int64_t ldx, const float* gamma, const float* beta, int64_t rows,
                                   int32_t d, float eps, int32_t out_bf16, void* y, int64_t ldy, float* stats,
                                   void* stream) {
  ASRN_REQUIRE(rows >= 0 && d > 0 && d % 4 == 0 && d <= 4 * kLnMaxD4 * kWave && ldx >= d && ldx % 4 == 0 &&
                   ldy >= d && ldy % 4 == 0 && eps > 0.f && (out_bf16 == 0 || out_bf16 == 1),
               "asrn_layer_norm_fwd: bad sizes rows=%lld d=%d (a multiple of 4, <= %d) ldx=%lld ldy=%lld",
               (long long)rows, d, 4 * kLnMaxD4 * kWave, (long long)ldx, (long long)ldy);
  if (rows == 0) return 0;
  ASRN_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)y & (out_bf16 ? 7 : 15)) == 0 && ((uintptr_t)gamma & 15) == 0 &&
                   ((uintptr_t)beta & 15) == 0,
               "asrn_layer_norm_fwd: rows and parameters must be 16-byte aligned (8 for bf16 output)");
  LnArgs a{};
  a.x = x; a.ldx = ldx; a.gamma = gamma; a.beta = beta; a.rows = rows; a.d = d; a.eps = eps; a.y = y; a.ldy = ldy;
  a.stats = reinterpret_cast<float2*>(stats);
  const dim3 grid((unsigned)((rows + kLnFwdRows - 1) / kLnFwdRows)), block(kLnThreads);
  hipStream_t st = (hipStream_t)stream;
#define LN_FWD(D4)                                                                                   \
  if (out_bf16) hipLaunchKernelGGL((k_ln_fwd<D4, true>), grid, block, 0, st, a);                    \
  else hipLaunchKernelGGL((k_ln_fwd<D4, false>), grid, block, 0, st, a);
  switch (ln_d4(d)) {
    case 1: LN_FWD(1) break;
    case 2: LN_FWD(2) break;
    case 3: LN_FWD(3) break;
    default: LN_FWD(4) break;
  }
#undef LN_FWD
  return check_launch("asrn_layer_norm_fwd");
}

extern "C" int64_t asrn_layer_norm_bwd_workspace(int64_t rows, int32_t d) {
  if (rows < 0 || d <= 0) return -1;
  const int64_t groups = ln_bwd_groups(rows);
  const int64_t part = (groups * 2 * d * 4 + 255) / 256 * 256;
  const int64_t sums = asrn_column_sums_workspace(groups, 2 * (int64_t)d);
  return sums < 0 ? -1 : part + sums;
}

extern "C" int asrn_layer_norm_bwd(const float* x, int64_t ldx, const float* gamma, const float* stats, int64_t rows,
                                   int32_t d, const void* dy, int32_t dy_bf16, int64_t lddy, const float* dres,
                                   float* dx, float* dparams, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  ASRN_REQUIRE(rows >= 0 && d > 0 && d % 4 == 0 && d <= 4 * kLnMaxD4 * kWave && ldx >= d && ldx % 4 == 0 &&
                   lddy >= d && lddy % 4 == 0 && (dy_bf16 == 0 || dy_bf16 == 1),
               "asrn_layer_norm_bwd: bad sizes rows=%lld d=%d (a multiple of 4, <= %d) ldx=%lld lddy=%lld",
               (long long)rows, d, 4 * kLnMaxD4 * kWave, (long long)ldx, (long long)lddy);
  const int64_t need = asrn_layer_norm_bwd_workspace(rows, d);
  ASRN_REQUIRE(need >= 0 && workspace_bytes >= need && workspace != nullptr && ((uintptr_t)workspace % 256) == 0,
               "asrn_layer_norm_bwd: needs a 256-byte aligned workspace of %lld bytes", (long long)need);
  if (rows == 0) return asrn_column_sums(nullptr, 0, 0, 2 * (int64_t)d, 2 * (int64_t)d, dparams, nullptr, 0, stream);
  ASRN_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)dx & 15) == 0 && ((uintptr_t)dy & (dy_bf16 ? 7 : 15)) == 0 &&
                   ((uintptr_t)dres & 15) == 0 && ((uintptr_t)gamma & 15) == 0,
               "asrn_layer_norm_bwd: rows and parameters must be 16-byte aligned (8 for bf16 dy)");
  LnArgs a{};
  a.x = x; a.ldx = ldx; a.gamma = gamma; a.rows = rows; a.d = d; a.stats = reinterpret_cast<float2*>(const_cast<float*>(stats));
  a.dy = dy; a.lddy = lddy; a.dres = dres; a.dx = dx; a.partial = (float*)workspace;
  const int64_t groups = ln_bwd_groups(rows);
  ASRN_REQUIRE(groups < (int64_t(1) << 31), "asrn_layer_norm_bwd: too many rows");
  const dim3 grid((unsigned)groups), block(kLnThreads);
  hipStream_t st = (hipStream_t)stream;
#define LN_BWD(D4)                                                                                   \
  if (dy_bf16) hipLaunchKernelGGL((k_ln_bwd<D4, true>), grid, block, 0, st, a);                     \
  else hipLaunchKernelGGL((k_ln_bwd<D4, false>), grid, block, 0, st, a);
  switch (ln_d4(d)) {
    case 1: LN_BWD(1) break;
    case 2: LN_BWD(2) break;
    case 3: LN_BWD(3) break;
    default: LN_BWD(4) break;
  }
#undef LN_BWD
  if (check_launch("asrn_layer_norm_bwd")) return 1;
  const int64_t part_bytes = (groups * 2 * d * 4 + 255) / 256 * 256;
  return asrn_column_sums(a.partial, 0, groups, 2 * (int64_t)d, 2 * (int64_t)d, dparams,
                          (char*)workspace + part_bytes, need - part_bytes, stream);
}
