// The local block's causal convolution window (asrn/nucleo.py:969-1014, a 'conv' BloqueLocal): the columns the
// convolution's GEMM multiplies, cols[b, t, c k + j] = z[b, t + j - (k - 1), c] (zero before the row's start), which
// PyTorch builds as pad + unfold + a reshaping copy in fp32 and then casts to the autocast dtype. Here they are
// written once, in the GEMM's dtype (fp32 or bf16, rounded to nearest even as the cast rounds), and the backward
// folds the columns' gradient back, dz[b, s, c] = sum_j dcols[b, s + k - 1 - j, c k + j] (j ascending, in fp32).
//
//   k_window_fwd  one thread per (token, channel): its k taps from k rows of z (coalesced across channels), k
//                 consecutive outputs (one 8- or 16-byte store when k = 4). With k = 4 a thread takes 4 consecutive
//                 tokens of its channel instead: 7 rows of z serve its 16 outputs.
//   k_window_bwd  one thread per (token, channel): k columns' gradients from the k later rows. With k = 4 a thread
//                 takes 4 consecutive tokens of its channel: one 4-column load from each of 7 rows serves all 4.
#include "common.h"

namespace asrn {

constexpr int kWinThreads = 256;

__device__ __forceinline__ uint16_t win_bf16(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);   // NaN stays a (quiet) NaN
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// K > 0: the tap count at compile time (the stores vectorize at K = 4); K = 0: k at run time
template <int K, bool B16>
__global__ __launch_bounds__(kWinThreads) void k_window_fwd(const float* __restrict__ z, int64_t ldz, int64_t BL,
                                                             int64_t L, int d, int kr, void* __restrict__ cols) {
  const int k = K > 0 ? K : kr;
  const int64_t e = (int64_t)blockIdx.x * kWinThreads + threadIdx.x;
  if (e >= BL * d) return;
  const int64_t bt = e / d, t = bt % L;
  const int c = (int)(e - bt * d);
  float v[16];
#pragma unroll
  for (int j = 0; j < (K > 0 ? K : 16); ++j) {
    if (K == 0 && j >= k) break;
    const int64_t s = t + j - (k - 1);
    v[j] = s >= 0 ? z[(bt + j - (k - 1)) * ldz + c] : 0.f;
  }
  const int64_t o = e * k;                        // (bt d + c) k = bt (d k) + c k
  if constexpr (B16) {
    uint16_t* out = reinterpret_cast<uint16_t*>(cols) + o;
    if constexpr (K == 4) {
      *reinterpret_cast<uint2*>(out) = make_uint2((uint32_t)win_bf16(v[0]) | ((uint32_t)win_bf16(v[1]) << 16),
                                                  (uint32_t)win_bf16(v[2]) | ((uint32_t)win_bf16(v[3]) << 16));
    } else {
      for (int j = 0; j < k; ++j) out[j] = win_bf16(v[j]);
    }
  } else {
    float* out = reinterpret_cast<float*>(cols) + o;
    if constexpr (K == 4) {
      *reinterpret_cast<float4*>(out) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      for (int j = 0; j < k; ++j) out[j] = v[j];
    }
  }
}

template <int K, bool B16>
__global__ __launch_bounds__(kWinThreads) void k_window_bwd(const void* __restrict__ dcols, int64_t BL, int64_t L,
                                                             int d, int kr, float* __restrict__ dz, int64_t lddz) {
  const int k = K > 0 ? K : kr;
  const int64_t e = (int64_t)blockIdx.x * kWinThreads + threadIdx.x;
  if (e >= BL * d) return;
  const int64_t bs = e / d, s = bs % L;
  const int c = (int)(e - bs * d);
  const int64_t dk = (int64_t)d * k;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < (K > 0 ? K : 16); ++j) {
    if (K == 0 && j >= k) break;
    const int64_t t = s + (k - 1) - j;            // the window that holds z[s] at tap j
    if (t < L) {
      const int64_t i = (bs + (k - 1) - j) * dk + (int64_t)c * k + j;
      acc += B16 ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(dcols)[i] << 16)
                 : reinterpret_cast<const float*>(dcols)[i];
    }
  }
  dz[bs * lddz + c] = acc;
}

// k = 4, 4 consecutive tokens t0 .. t0 + 3 of one channel a thread (rows of L tokens, L a multiple of 4; thread e:
// channel e % d of token group e / d): z rows t0 - 3 .. t0 + 3, each read once
constexpr int kTokPer = 4;
template <bool B16>
__global__ __launch_bounds__(kWinThreads) void k_window_fwd4(const float* __restrict__ z, int64_t ldz, int64_t BL,
                                                             int64_t L, int d, void* __restrict__ cols) {
  const int64_t e = (int64_t)blockIdx.x * kWinThreads + threadIdx.x;
  if (e >= BL / kTokPer * d) return;
  const int64_t grp = e / d, bt0 = grp * kTokPer, t0 = bt0 % L;
  const int c = (int)(e - grp * d);
  float v[kTokPer + 3];
#pragma unroll
  for (int i = 0; i < kTokPer + 3; ++i) {
    const int64_t s = t0 + i - 3;                  // row position of tap source i
    v[i] = s >= 0 ? z[(bt0 + i - 3) * ldz + c] : 0.f;
  }
#pragma unroll
  for (int u = 0; u < kTokPer; ++u) {
    const int64_t o = ((bt0 + u) * d + c) * 4;     // cols[bt0 + u, c * 4 + j] = v[u + j]
    if constexpr (B16) {
      *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(cols) + o) =
          make_uint2((uint32_t)win_bf16(v[u]) | ((uint32_t)win_bf16(v[u + 1]) << 16),
                     (uint32_t)win_bf16(v[u + 2]) | ((uint32_t)win_bf16(v[u + 3]) << 16));
    } else {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(cols) + o) = make_float4(v[u], v[u + 1], v[u + 2], v[u + 3]);
    }
  }
}

// k = 4, 4 consecutive tokens s0 .. s0 + 3 of one channel a thread: dcols rows s0 .. s0 + 6 (within the row), each
// row's 4 columns of the channel in one load; dz[s0 + u] = sum over j (ascending) of dcols[s0 + u + 3 - j][4 c + j]
template <bool B16>
__global__ __launch_bounds__(kWinThreads) void k_window_bwd4(const void* __restrict__ dcols, int64_t BL, int64_t L,
                                                             int d, float* __restrict__ dz, int64_t lddz) {
  const int64_t e = (int64_t)blockIdx.x * kWinThreads + threadIdx.x;
  if (e >= BL / kTokPer * d) return;
  const int64_t grp = e / d, bs0 = grp * kTokPer, s0 = bs0 % L;
  const int c = (int)(e - grp * d);
  float w[kTokPer + 3][4];
#pragma unroll
  for (int i = 0; i < kTokPer + 3; ++i) {
    const bool in = s0 + i < L;                     // windows past the row's end hold nothing
    const int64_t r = in ? bs0 + i : bs0;
    const int64_t off = (r * d + c) * 4;
    if constexpr (B16) {
      const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(dcols) + off);
      w[i][0] = __uint_as_float(u.x << 16); w[i][1] = __uint_as_float(u.x & 0xffff0000u);
      w[i][2] = __uint_as_float(u.y << 16); w[i][3] = __uint_as_float(u.y & 0xffff0000u);
    } else {
      const float4 f = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(dcols) + off);
      w[i][0] = f.x; w[i][1] = f.y; w[i][2] = f.z; w[i][3] = f.w;
    }
    if (!in) w[i][0] = w[i][1] = w[i][2] = w[i][3] = 0.f;
  }
#pragma unroll
  for (int u = 0; u < kTokPer; ++u) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += w[u + 3 - j][j];
    dz[(bs0 + u) * lddz + c] = acc;
  }
}

template <bool B16>
static void launch_fwd(const float* z, int64_t ldz, int64_t BL, int64_t L, int d, int k, void* cols,
                       hipStream_t st) {
  const dim3 grid((unsigned)((BL * d + kWinThreads - 1) / kWinThreads));
  if (k == 4 && L % kTokPer == 0)
    hipLaunchKernelGGL((k_window_fwd4<B16>), dim3((unsigned)((BL / kTokPer * d + kWinThreads - 1) / kWinThreads)),
                       dim3(kWinThreads), 0, st, z, ldz, BL, L, d, cols);
  else if (k == 4)
    hipLaunchKernelGGL((k_window_fwd<4, B16>), grid, dim3(kWinThreads), 0, st, z, ldz, BL, L, d, k, cols);
  else
    hipLaunchKernelGGL((k_window_fwd<0, B16>), grid, dim3(kWinThreads), 0, st, z, ldz, BL, L, d, k, cols);
}

template <bool B16>
static void launch_bwd(const void* dcols, int64_t BL, int64_t L, int d, int k, float* dz, int64_t lddz,
                       hipStream_t st) {
  const dim3 grid((unsigned)((BL * d + kWinThreads - 1) / kWinThreads));
  if (k == 4 && L % kTokPer == 0)
    hipLaunchKernelGGL((k_window_bwd4<B16>), dim3((unsigned)((BL / kTokPer * d + kWinThreads - 1) / kWinThreads)),
                       dim3(kWinThreads), 0, st, dcols, BL, L, d, dz, lddz);
  else if (k == 4)
    hipLaunchKernelGGL((k_window_bwd<4, B16>), grid, dim3(kWinThreads), 0, st, dcols, BL, L, d, k, dz, lddz);
  else
    hipLaunchKernelGGL((k_window_bwd<0, B16>), grid, dim3(kWinThreads), 0, st, dcols, BL, L, d, k, dz, lddz);
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_conv_window_fwd(const float* z, int64_t ldz, int64_t B, int64_t L, int32_t d, int32_t k,
                                    int32_t cols_bf16, void* cols, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && d >= 1 && ldz >= d && k >= 1 && k <= 16 && (cols_bf16 == 0 || cols_bf16 == 1),
               "asrn_conv_window_fwd: bad sizes B=%lld L=%lld d=%d k=%d", (long long)B, (long long)L, d, k);
  ASRN_REQUIRE(((uintptr_t)cols & 15) == 0, "asrn_conv_window_fwd: cols must be 16-byte aligned");
  if (B == 0 || L == 0) return 0;
  if (cols_bf16) launch_fwd<true>(z, ldz, B * L, L, d, k, cols, (hipStream_t)stream);
  else launch_fwd<false>(z, ldz, B * L, L, d, k, cols, (hipStream_t)stream);
  return check_launch("asrn_conv_window_fwd");
}

extern "C" int asrn_conv_window_bwd(const void* dcols, int32_t cols_bf16, int64_t B, int64_t L, int32_t d, int32_t k,
                                    float* dz, int64_t lddz, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && d >= 1 && lddz >= d && k >= 1 && k <= 16 && (cols_bf16 == 0 || cols_bf16 == 1),
               "asrn_conv_window_bwd: bad sizes B=%lld L=%lld d=%d k=%d", (long long)B, (long long)L, d, k);
  if (B == 0 || L == 0) return 0;
  if (cols_bf16) launch_bwd<true>(dcols, B * L, L, d, k, dz, lddz, (hipStream_t)stream);
  else launch_bwd<false>(dcols, B * L, L, d, k, dz, lddz, (hipStream_t)stream);
  return check_launch("asrn_conv_window_bwd");
}
