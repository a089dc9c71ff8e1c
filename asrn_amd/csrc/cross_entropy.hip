// The model's loss: cross-entropy of fp32 or bf16 logits (rows x V) against integer targets, computed in fp32 as the
// reference's F.cross_entropy(logits.float(), y, ignore_index) does (asrn/nucleo.py:1108), without the fp32 copy of
// the logits it makes.
//
//   k_ce_fwd  one workgroup per row: the row's max, then the sum of exp(x - max) (the row is read twice; the second
//             read comes from L2), lse = max + log(sum); loss = lse - x[target] (0 for an ignored row, NaN for a
//             target outside [0, V)).
//   k_ce_bwd  one workgroup per row: d logits = (exp(x - lse) - [v == target]) * scale, in the logits' dtype (bf16
//             rounded to nearest even, as the cast back from fp32 rounds); an ignored row's gradient is 0.
// The mean over the rows that are not ignored is left to the caller (a fixed-order sum of the per-row losses).
#include <math.h>

#include "common.h"

namespace asrn {

constexpr int kCeThreads = 1024;
constexpr int kCeWaves = kCeThreads / kWave;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);   // NaN stays a (quiet) NaN
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// every element v of row `row`: f(v, x) for the vectorized body (8 elements per 16-byte load, all of a thread's loads
// for one sweep issued together) and the scalar tail
template <bool B16, class F>
__device__ __forceinline__ void sweep_row(const void* logits, int64_t ld, int64_t row, int64_t V, F f) {
  const int tid = threadIdx.x;
  if constexpr (B16) {
    const uint16_t* r = reinterpret_cast<const uint16_t*>(logits) + row * ld;
    const int64_t nvec = V / 8;
    for (int64_t v0 = tid; v0 < nvec; v0 += 4 * kCeThreads) {
      uint4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + (int64_t)u * kCeThreads;
        q[u] = *reinterpret_cast<const uint4*>(r + 8 * (v < nvec ? v : 0));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + (int64_t)u * kCeThreads;
        if (v >= nvec) continue;
        const uint32_t w[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          f(8 * v + 2 * k, __uint_as_float(w[k] << 16));
          f(8 * v + 2 * k + 1, __uint_as_float(w[k] & 0xffff0000u));
        }
      }
    }
    for (int64_t v = 8 * nvec + tid; v < V; v += kCeThreads) f(v, bf16_to_f32(r[v]));
  } else {
    const float* r = reinterpret_cast<const float*>(logits) + row * ld;
    const int64_t nvec = V / 4;
    for (int64_t v0 = tid; v0 < nvec; v0 += 4 * kCeThreads) {
      float4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + (int64_t)u * kCeThreads;
        q[u] = *reinterpret_cast<const float4*>(r + 4 * (v < nvec ? v : 0));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + (int64_t)u * kCeThreads;
        if (v >= nvec) continue;
        f(4 * v, q[u].x);
        f(4 * v + 1, q[u].y);
        f(4 * v + 2, q[u].z);
        f(4 * v + 3, q[u].w);
      }
    }
    for (int64_t v = 4 * nvec + tid; v < V; v += kCeThreads) f(v, r[v]);
  }
}

// max that keeps a NaN (fmaxf drops it; torch's max propagates it)
__device__ __forceinline__ float nan_max(float a, float b) { return (a != a || b != b) ? NAN : fmaxf(a, b); }

__device__ __forceinline__ float block_reduce(float x, float* red, bool is_max) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float o = __shfl_xor(x, m, kWave);
    x = is_max ? nan_max(x, o) : x + o;
  }
  if (lane == 0) red[wave] = x;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kCeWaves; ++w) r = is_max ? nan_max(r, red[w]) : r + red[w];   // in wave order
  __syncthreads();
  return r;
}

template <bool B16>
__global__ __launch_bounds__(kCeThreads) void k_ce_fwd(const void* logits, int64_t ld, const int64_t* target,
                                                       int64_t V, int64_t ignore, float* lse, float* loss) {
  __shared__ float red[kCeWaves];
  const int64_t row = blockIdx.x;
  float m = -INFINITY;
  sweep_row<B16>(logits, ld, row, V, [&](int64_t, float x) { m = nan_max(m, x); });
  const float mx = block_reduce(m, red, true);
  float s = 0.f;
  sweep_row<B16>(logits, ld, row, V, [&](int64_t, float x) { s += __expf(x - mx); });
  const float tot = block_reduce(s, red, false);
  if (threadIdx.x == 0) {
    const float l = mx + __logf(tot);
    lse[row] = l;
    const int64_t t = target[row];
    float xt = 0.f;
    if (t != ignore && t >= 0 && t < V) {
      xt = B16 ? bf16_to_f32(reinterpret_cast<const uint16_t*>(logits)[row * ld + t])
               : reinterpret_cast<const float*>(logits)[row * ld + t];
    }
    // a target outside [0, V) (PyTorch stops with a device assertion) makes the row's loss NaN
    loss[row] = t == ignore ? 0.f : (t >= 0 && t < V ? l - xt : NAN);
  }
}

// one output element: (exp(x - lse) - [v == t]) * scale, 0 for an ignored row
__device__ __forceinline__ float ce_grad(float x, int64_t v, int64_t t, float l, float sc, bool skip) {
  return skip ? 0.f : (__expf(x - l) - (v == t ? 1.f : 0.f)) * sc;
}

template <bool B16>
__global__ __launch_bounds__(kCeThreads) void k_ce_bwd(const void* logits, int64_t ld, const int64_t* target,
                                                       const float* lse, int64_t V, int64_t ignore,
                                                       const float* scale, void* dlogits, int64_t ldd) {
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t t = target[row];
  const bool skip = t == ignore;
  const float l = lse[row], sc = *scale;
  if constexpr (B16) {                             // 8 elements per 16-byte load and store
    const uint16_t* r = reinterpret_cast<const uint16_t*>(logits) + row * ld;
    uint16_t* o = reinterpret_cast<uint16_t*>(dlogits) + row * ldd;
    const int64_t nvec = V / 8;
    for (int64_t v0 = tid; v0 < nvec; v0 += 4 * kCeThreads) {
      uint4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + (int64_t)u * kCeThreads;
        q[u] = *reinterpret_cast<const uint4*>(r + 8 * (v < nvec ? v : 0));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + (int64_t)u * kCeThreads;
        if (v >= nvec) continue;
        const uint32_t w[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
        uint32_t out[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int64_t e = 8 * v + 2 * k;
          const uint16_t lo = f32_to_bf16(ce_grad(__uint_as_float(w[k] << 16), e, t, l, sc, skip));
          const uint16_t hi = f32_to_bf16(ce_grad(__uint_as_float(w[k] & 0xffff0000u), e + 1, t, l, sc, skip));
          out[k] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *reinterpret_cast<uint4*>(o + 8 * v) = make_uint4(out[0], out[1], out[2], out[3]);
      }
    }
    for (int64_t v = 8 * nvec + tid; v < V; v += kCeThreads)
      o[v] = f32_to_bf16(ce_grad(bf16_to_f32(r[v]), v, t, l, sc, skip));
  } else {                                         // 4 elements per 16-byte load and store
    const float* r = reinterpret_cast<const float*>(logits) + row * ld;
    float* o = reinterpret_cast<float*>(dlogits) + row * ldd;
    const int64_t nvec = V / 4;
    for (int64_t v0 = tid; v0 < nvec; v0 += 4 * kCeThreads) {
      float4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + (int64_t)u * kCeThreads;
        q[u] = *reinterpret_cast<const float4*>(r + 4 * (v < nvec ? v : 0));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + (int64_t)u * kCeThreads;
        if (v >= nvec) continue;
        const int64_t e = 4 * v;
        *reinterpret_cast<float4*>(o + e) =
            make_float4(ce_grad(q[u].x, e, t, l, sc, skip), ce_grad(q[u].y, e + 1, t, l, sc, skip),
                        ce_grad(q[u].z, e + 2, t, l, sc, skip), ce_grad(q[u].w, e + 3, t, l, sc, skip));
      }
    }
    for (int64_t v = 4 * nvec + tid; v < V; v += kCeThreads) o[v] = ce_grad(r[v], v, t, l, sc, skip);
  }
}

static int ce_check(const void* logits, int32_t bf16, int64_t ld, int64_t rows, int64_t V, const char* what) {
  ASRN_REQUIRE(rows >= 0 && V >= 1 && ld >= V && (bf16 == 0 || bf16 == 1) && rows < (int64_t(1) << 31),
               "%s: bad sizes rows=%lld V=%lld ld=%lld", what, (long long)rows, (long long)V, (long long)ld);
  ASRN_REQUIRE(((uintptr_t)logits & 15) == 0 && ld % (bf16 ? 8 : 4) == 0,
               "%s: logits must be 16-byte aligned with a row stride that keeps them so", what);
  return 0;
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_cross_entropy_fwd(const void* logits, int32_t logits_bf16, int64_t ld, const int64_t* target,
                                      int64_t rows, int64_t V, int64_t ignore_index, float* lse, float* loss,
                                      void* stream) {
  if (ce_check(logits, logits_bf16, ld, rows, V, "asrn_cross_entropy_fwd")) return 1;
  if (rows == 0) return 0;
  if (logits_bf16)
    hipLaunchKernelGGL(k_ce_fwd<true>, dim3((unsigned)rows), dim3(kCeThreads), 0, (hipStream_t)stream, logits, ld,
                       target, V, ignore_index, lse, loss);
  else
    hipLaunchKernelGGL(k_ce_fwd<false>, dim3((unsigned)rows), dim3(kCeThreads), 0, (hipStream_t)stream, logits, ld,
                       target, V, ignore_index, lse, loss);
  return check_launch("asrn_cross_entropy_fwd");
}

extern "C" int asrn_cross_entropy_bwd(const void* logits, int32_t logits_bf16, int64_t ld, const int64_t* target,
                                      const float* lse, int64_t rows, int64_t V, int64_t ignore_index,
                                      const float* scale, void* dlogits, int64_t ldd, void* stream) {
  if (ce_check(logits, logits_bf16, ld, rows, V, "asrn_cross_entropy_bwd")) return 1;
  ASRN_REQUIRE(ldd >= V && ldd % (logits_bf16 ? 8 : 4) == 0 && ((uintptr_t)dlogits & 15) == 0,
               "asrn_cross_entropy_bwd: the gradient needs a row stride >= V that keeps 16-byte aligned rows");
  if (rows == 0) return 0;
  if (logits_bf16)
    hipLaunchKernelGGL(k_ce_bwd<true>, dim3((unsigned)rows), dim3(kCeThreads), 0, (hipStream_t)stream, logits, ld,
                       target, lse, V, ignore_index, scale, dlogits, ldd);
  else
    hipLaunchKernelGGL(k_ce_bwd<false>, dim3((unsigned)rows), dim3(kCeThreads), 0, (hipStream_t)stream, logits, ld,
                       target, lse, V, ignore_index, scale, dlogits, ldd);
  return check_launch("asrn_cross_entropy_bwd");
}
