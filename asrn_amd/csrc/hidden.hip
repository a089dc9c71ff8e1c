// a0 (part): the hash MLPs' hidden layer, between the layer's two producer GEMMs (asrn/nucleo.py:644-659).
//
// The first GEMM gives, per token t of a batch row, y[t] = [W_p E_t | W_a E_t | W_b E_t | ...] with no bias. The word
// MLP's hidden units are gelu(W_p E_t + b_p); the context MLP's are gelu(W_a E_t + W_b E_{t-1} + b_c), its first layer
// applied to the key [E_t; E_{t-1}] split by linearity (the W_b term is absent at t = 0, where the key's second half
// is the zero pad). Forward: g[t] = [gelu(hp + b_p) | gelu(za + zb_prev + b_c)], one float4 of one token per thread.
// Backward: from dg, the pre-activation gradients go straight into the first GEMM's output gradient dy: the word
// block, the W_a block, and the W_b block one position earlier (dy_zb[t] = d pre[t + 1], 0 at a row's last position),
// each element written by exactly one thread. gelu is the exact erf form of torch.nn.GELU().
#include "common.h"

namespace asrn {

constexpr int kHidThreads = 256;

struct HidArgs {
  const float* y; int64_t ldy;      // (B*L, ldy): hp at columns [0, m), za at [m, m + mc), zb at [m + mc, m + 2 mc)
  const float* bp; const float* bc; // biases of the word (m) and context (mc) first layers
  float* g;                         // (B*L, m + mc)
  const float* dg;                  // (B*L, m + mc)
  float* dy; int64_t ldd;           // (B*L, ldd): columns [0, m + 2 mc) written
  int64_t B, L;
  int m, mc;
};

__device__ __forceinline__ float gelu_f(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }
__device__ __forceinline__ float gelu_grad(float x) {
  return 0.5f * (1.f + erff(x * 0.70710678118654752f)) + x * 0.39894228040143268f * __expf(-0.5f * x * x);
}

// the pre-activations of hidden columns j .. j + 3 of token row `row` (position t in its batch row)
__device__ __forceinline__ float4 pre_act(const HidArgs& a, int64_t row, int64_t t, int j) {
  if (j < a.m) {
    const float4 y = *reinterpret_cast<const float4*>(a.y + row * a.ldy + j);
    const float4 b = *reinterpret_cast<const float4*>(a.bp + j);
    return make_float4(y.x + b.x, y.y + b.y, y.z + b.z, y.w + b.w);
  }
  const int c = j - a.m;
  const float4 za = *reinterpret_cast<const float4*>(a.y + row * a.ldy + a.m + c);
  const float4 b = *reinterpret_cast<const float4*>(a.bc + c);
  float4 r = make_float4(za.x + b.x, za.y + b.y, za.z + b.z, za.w + b.w);
  if (t > 0) {
    const float4 zb = *reinterpret_cast<const float4*>(a.y + (row - 1) * a.ldy + a.m + a.mc + c);
    r.x += zb.x; r.y += zb.y; r.z += zb.z; r.w += zb.w;
  }
  return r;
}

__global__ __launch_bounds__(kHidThreads) void k_hidden_fwd(HidArgs a) {
  const int w4 = (a.m + a.mc) / 4;
  const int64_t i = (int64_t)blockIdx.x * kHidThreads + threadIdx.x;
  if (i >= a.B * a.L * w4) return;
  const int64_t row = i / w4;
  const int j = (int)(i - row * w4) * 4;
  const float4 x = pre_act(a, row, row % a.L, j);
  *reinterpret_cast<float4*>(a.g + row * (a.m + a.mc) + j) = make_float4(gelu_f(x.x), gelu_f(x.y), gelu_f(x.z),
                                                                          gelu_f(x.w));
}

__global__ __launch_bounds__(kHidThreads) void k_hidden_bwd(HidArgs a) {
  const int w4 = (a.m + a.mc) / 4;
  const int64_t i = (int64_t)blockIdx.x * kHidThreads + threadIdx.x;
  if (i >= a.B * a.L * w4) return;
  const int64_t row = i / w4, t = row % a.L;
  const int j = (int)(i - row * w4) * 4;
  const float4 x = pre_act(a, row, t, j);
  const float4 d = *reinterpret_cast<const float4*>(a.dg + row * (a.m + a.mc) + j);
  const float4 dp = make_float4(d.x * gelu_grad(x.x), d.y * gelu_grad(x.y), d.z * gelu_grad(x.z),
                                d.w * gelu_grad(x.w));
  *reinterpret_cast<float4*>(a.dy + row * a.ldd + j) = dp;   // the word block, or the W_a block (columns m + c)
  if (j >= a.m) {
    const int c = j - a.m;
    if (t > 0) *reinterpret_cast<float4*>(a.dy + (row - 1) * a.ldd + a.m + a.mc + c) = dp;
    if (t == a.L - 1)
      *reinterpret_cast<float4*>(a.dy + row * a.ldd + a.m + a.mc + c) = make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

static int check(const HidArgs& a, const char* what) {
  ASRN_REQUIRE(a.B >= 0 && a.L >= 0 && a.m >= 4 && a.mc >= 4 && a.m % 4 == 0 && a.mc % 4 == 0,
               "%s: bad sizes B=%lld L=%lld m=%d mc=%d (m and mc: multiples of 4)", what, (long long)a.B,
               (long long)a.L, a.m, a.mc);
  ASRN_REQUIRE(a.ldy >= a.m + 2 * a.mc && a.ldy % 4 == 0 && ((uintptr_t)a.y & 15) == 0,
               "%s: y needs a row stride >= m + 2 mc, a multiple of 4, and 16-byte aligned rows", what);
  return 0;
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_hidden_fwd(const float* y, int64_t ldy, const float* b_word, const float* b_ctx, int64_t B,
                               int64_t L, int32_t m, int32_t mc, float* g, void* stream) {
  HidArgs a = {};
  a.y = y; a.ldy = ldy; a.bp = b_word; a.bc = b_ctx; a.g = g; a.B = B; a.L = L; a.m = m; a.mc = mc;
  if (check(a, "asrn_hidden_fwd")) return 1;
  ASRN_REQUIRE(((uintptr_t)g & 15) == 0 && ((uintptr_t)b_word & 15) == 0 && ((uintptr_t)b_ctx & 15) == 0,
               "asrn_hidden_fwd: g and the biases must be 16-byte aligned");
  const int64_t n = B * L * ((m + mc) / 4);
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_hidden_fwd, dim3((unsigned)((n + kHidThreads - 1) / kHidThreads)), dim3(kHidThreads), 0,
                     (hipStream_t)stream, a);
  return check_launch("asrn_hidden_fwd");
}

extern "C" int asrn_hidden_bwd(const float* y, int64_t ldy, const float* b_word, const float* b_ctx, int64_t B,
                               int64_t L, int32_t m, int32_t mc, const float* dg, float* dy, int64_t ldd,
                               void* stream) {
  HidArgs a = {};
  a.y = y; a.ldy = ldy; a.bp = b_word; a.bc = b_ctx; a.dg = dg; a.dy = dy; a.ldd = ldd;
  a.B = B; a.L = L; a.m = m; a.mc = mc;
  if (check(a, "asrn_hidden_bwd")) return 1;
  ASRN_REQUIRE(ldd >= m + 2 * mc && ldd % 4 == 0 && ((uintptr_t)dy & 15) == 0 && ((uintptr_t)dg & 15) == 0 &&
                   ((uintptr_t)b_word & 15) == 0 && ((uintptr_t)b_ctx & 15) == 0,
               "asrn_hidden_bwd: dy needs a row stride >= m + 2 mc (a multiple of 4); dy, dg and the biases must be "
               "16-byte aligned");
  const int64_t n = B * L * ((m + mc) / 4);
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_hidden_bwd, dim3((unsigned)((n + kHidThreads - 1) / kHidThreads)), dim3(kHidThreads), 0,
                     (hipStream_t)stream, a);
  return check_launch("asrn_hidden_bwd");
}
