// a13: the gate consumer, fused (reference asrn/estable.py:376-403, asrn/nucleo.py:865-878).
//
// Per token t, with A = W_o salida (the hipBLASLt GEMM, before the division by the table count):
//   r = 1 / max(1, peso_total)
//   sen = [peso_total / T, clip(mejor, +-mejor_max) (0 when no table has a candidate), pico / max(1, peso_total),
//          peso_ctx / Tc]
//   logit = (h . w_g + b_g) + (sen . w_c + b_c) + vistos . w_v + log1p(hawkes) . u_h + f(racha)
//   f(racha): x = min(log1p(racha) / paso, nodes - 1), i = clamp(floor(x), 0, nodes - 2),
//             f = cumsum(d_racha)[i] + (x - i) d_racha[i + 1]
//   h' = h + sigmoid(cap(logit)) r A,        cap(l) = tope tanh(l / tope) when a cap is set
// (W_o (salida r) = r (W_o salida): the division by the table count is folded into the per-token factor.)
//
// One wavefront per token (grid-stride), the d-rows read as float4 per lane: h, A and h' stream through HBM once.
// The backward gives dh, dA, dhawkes, dracha per token and the parameter gradients as per-workgroup partials summed
// in a fixed order by a second launch (deterministic, no atomics).
#include "common.h"

namespace asrn {

constexpr int kGateThreads = 256;
constexpr int kGateWaves = kGateThreads / kWave;
constexpr int kGateMaxBlocks = 512;
constexpr int kGateMaxD4 = 4;    // d <= 1024
constexpr int kGateCols = 64;    // lanes that carry the small parameters' gradients: 6 + 2 n + nodes <= 64

struct GateArgs {
  const float* h; const void* A; int a_bf16;
  const float* sig; const float* vistos; const float* hawkes; const float* racha;
  const float* wg; const float* bg; const float* wc; const float* bc; const float* wv; const float* uh;
  const float* dr;
  int64_t BL; int d; int n; int nodes; int T; int Tc; float paso; float mejor_max; float tope;
  float* logit; float* out;                                        // forward
  const float* dout; float* dh; void* dA; float* dhawkes; float* dracha; float* partial;   // backward
};

__device__ __forceinline__ float4 load_a4(const void* p, int bf16, int64_t q) {
  if (!bf16) return ((const float4*)p)[q];
  const uint2 u = ((const uint2*)p)[q];   // four bf16, element 0 in the low half
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                     __uint_as_float(u.y & 0xffff0000u));
}

// fp32 -> bf16 bits, round to nearest even (NaN stays a quiet NaN)
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ void store_a4(void* p, int bf16, int64_t q, float4 v) {
  if (!bf16) {
    ((float4*)p)[q] = v;
    return;
  }
  ((uint2*)p)[q] = make_uint2(bf16_bits(v.x) | (bf16_bits(v.y) << 16), bf16_bits(v.z) | (bf16_bits(v.w) << 16));
}

// The per-token inputs of the logit other than h, and the streak response's position.
struct Small {
  float r, sen[4], x, frac, sum;   // sum: every logit term but h . w_g + b_g
  int i;
  bool xpass;                      // the clamp of x passes the gradient
};

__device__ __forceinline__ Small small_terms(const GateArgs& a, int64_t t) {
  Small s;
  const float4 g = ((const float4*)a.sig)[t];     // peso_total, mejor, pico, peso_ctx
  const float pt = g.x;
  s.r = 1.f / fmaxf(pt, 1.f);
  float mejor = pt > 0.f ? g.y : 0.f;
  if (a.mejor_max >= 0.f) mejor = fminf(fmaxf(mejor, -a.mejor_max), a.mejor_max);
  s.sen[0] = pt / (float)a.T;
  s.sen[1] = mejor;
  s.sen[2] = g.z / fmaxf(pt, 1.f);
  s.sen[3] = g.w / (float)a.Tc;
  float conf = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) conf += s.sen[k] * a.wc[k];
  conf += a.bc[0];
  float vis = 0.f, haw = 0.f;
  for (int j = 0; j < a.n; ++j) {
    vis += a.vistos[t * a.n + j] * a.wv[j];
    haw += log1pf(a.hawkes[t * a.n + j]) * a.uh[j];
  }
  const float top = (float)(a.nodes - 1);
  const float xr = log1pf(a.racha[t]) / a.paso;
  s.xpass = xr <= top;
  s.x = fminf(xr, top);
  float fi = s.x != s.x ? 0.f : floorf(s.x);
  fi = fminf(fmaxf(fi, 0.f), (float)(a.nodes - 2));
  s.i = (int)fi;
  s.frac = s.x - fi;
  float cum = 0.f;
  for (int k = 0; k <= s.i; ++k) cum += a.dr[k];
  const float resp = cum + s.frac * a.dr[s.i + 1];
  s.sum = conf + vis + haw + resp;
  return s;
}

__device__ __forceinline__ float capped(float l, float tope) { return tope > 0.f ? tope * tanhf(l / tope) : l; }

template <int D4>
__global__ __launch_bounds__(kGateThreads) void k_gate_fwd(GateArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int d4 = a.d >> 2;
  const int64_t stride = (int64_t)gridDim.x * kGateWaves;
  for (int64_t t = (int64_t)blockIdx.x * kGateWaves + (threadIdx.x >> 6); t < a.BL; t += stride) {
    const float4* h4 = (const float4*)(a.h + t * a.d);
    float4 hv[D4], av[D4];
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      const int q = lane + kWave * k;
      if (q < d4) {
        hv[k] = h4[q];
        av[k] = load_a4(a.A, a.a_bf16, t * d4 + q);
        const float4 w = ((const float4*)a.wg)[q];
        dot += hv[k].x * w.x + hv[k].y * w.y + hv[k].z * w.z + hv[k].w * w.w;
      }
    }
    const Small s = small_terms(a, t);
    const float logit = (wave_sum_u(dot) + a.bg[0]) + s.sum;
    if (lane == 0) a.logit[t] = logit;
    const float sr = s.r / (1.f + expf(-capped(logit, a.tope)));
    float4* o4 = (float4*)(a.out + t * a.d);
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      const int q = lane + kWave * k;
      if (q < d4)
        o4[q] = make_float4(hv[k].x + sr * av[k].x, hv[k].y + sr * av[k].y, hv[k].z + sr * av[k].z,
                            hv[k].w + sr * av[k].w);
    }
  }
}

template <int D4>
__global__ __launch_bounds__(kGateThreads) void k_gate_bwd(GateArgs a) {
  __shared__ float red[kGateWaves][4 * D4 * kWave + kGateCols];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  const int n = a.n, base_v = 6, base_u = 6 + n, base_r = 6 + 2 * n;
  const int64_t stride = (int64_t)gridDim.x * kGateWaves;
  float4 gw[D4];
#pragma unroll
  for (int k = 0; k < D4; ++k) gw[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  float gs = 0.f;   // this lane's small parameter (column d + lane)
  for (int64_t t = (int64_t)blockIdx.x * kGateWaves + wave; t < a.BL; t += stride) {
    const float4* g4 = (const float4*)(a.dout + t * a.d);
    const float4* h4 = (const float4*)(a.h + t * a.d);
    float4 gv[D4], hv[D4], av[D4];
    float ga = 0.f;
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      const int q = lane + kWave * k;
      if (q < d4) {
        gv[k] = g4[q];
        hv[k] = h4[q];
        av[k] = load_a4(a.A, a.a_bf16, t * d4 + q);
        ga += gv[k].x * av[k].x + gv[k].y * av[k].y + gv[k].z * av[k].z + gv[k].w * av[k].w;
      }
    }
    const Small s = small_terms(a, t);
    const float l = a.logit[t];
    float dcap = 1.f;
    float lc = l;
    if (a.tope > 0.f) {
      const float th = tanhf(l / a.tope);
      lc = a.tope * th;
      dcap = 1.f - th * th;
    }
    const float sg = 1.f / (1.f + expf(-lc));
    const float dlogit = wave_sum_u(ga) * s.r * (sg * (1.f - sg)) * dcap;
    const float sr = sg * s.r;
    float4* dh4 = (float4*)(a.dh + t * a.d);
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      const int q = lane + kWave * k;
      if (q < d4) {
        const float4 w = ((const float4*)a.wg)[q];
        dh4[q] = make_float4(gv[k].x + dlogit * w.x, gv[k].y + dlogit * w.y, gv[k].z + dlogit * w.z,
                             gv[k].w + dlogit * w.w);
        store_a4(a.dA, a.a_bf16, t * d4 + q, make_float4(gv[k].x * sr, gv[k].y * sr, gv[k].z * sr, gv[k].w * sr));
        gw[k].x += dlogit * hv[k].x;
        gw[k].y += dlogit * hv[k].y;
        gw[k].z += dlogit * hv[k].z;
        gw[k].w += dlogit * hv[k].w;
      }
    }
    // small parameters: one lane each
    float f = 0.f;
    if (lane == 0 || lane == 5) f = 1.f;
    else if (lane <= 4) f = lane == 1 ? s.sen[0] : lane == 2 ? s.sen[1] : lane == 3 ? s.sen[2] : s.sen[3];
    else if (lane < base_u) f = a.vistos[t * n + lane - base_v];
    else if (lane < base_r) f = log1pf(a.hawkes[t * n + lane - base_u]);
    else if (lane < base_r + a.nodes) {
      const int m = lane - base_r;
      f = (m <= s.i ? 1.f : 0.f) + (m == s.i + 1 ? s.frac : 0.f);
    }
    gs += dlogit * f;
    if (lane < n) a.dhawkes[t * n + lane] = dlogit * a.uh[lane] / (1.f + a.hawkes[t * n + lane]);
    if (lane == 0)
      a.dracha[t] = s.xpass ? dlogit * a.dr[s.i + 1] / ((1.f + a.racha[t]) * a.paso) : 0.f;
  }
  // workgroup partial: the waves' sums in wave order
  float* mine = red[wave];
#pragma unroll
  for (int k = 0; k < D4; ++k) {
    const int q = lane + kWave * k;
    mine[4 * q + 0] = gw[k].x;
    mine[4 * q + 1] = gw[k].y;
    mine[4 * q + 2] = gw[k].z;
    mine[4 * q + 3] = gw[k].w;
  }
  mine[4 * D4 * kWave + lane] = gs;
  __syncthreads();
  const int cols = a.d + kGateCols;
  for (int c = threadIdx.x; c < cols; c += kGateThreads) {
    const int src = c < a.d ? c : 4 * D4 * kWave + (c - a.d);
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kGateWaves; ++w) v += red[w][src];
    a.partial[(int64_t)blockIdx.x * cols + c] = v;
  }
}

// dparams[c] = sum over workgroups g of partial[g][c], in workgroup order
__global__ void k_gate_params(const float* __restrict__ partial, int groups, int cols, float* __restrict__ dparams) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  float v = 0.f;
  for (int g = 0; g < groups; ++g) v += partial[(int64_t)g * cols + c];
  dparams[c] = v;
}

static int gate_check(const GateArgs& a, const char* what) {
  ASRN_REQUIRE(a.BL >= 0, "%s: bad sizes", what);
  ASRN_REQUIRE(a.d > 0 && a.d % 4 == 0 && a.d <= 4 * kGateMaxD4 * kWave, "%s: d=%d must be a multiple of 4, <= %d",
               what, a.d, 4 * kGateMaxD4 * kWave);
  ASRN_REQUIRE(a.n >= 1 && a.nodes >= 2 && 6 + 2 * a.n + a.nodes <= kGateCols,
               "%s: n=%d, nodes=%d: need 6 + 2 n + nodes <= %d", what, a.n, a.nodes, kGateCols);
  ASRN_REQUIRE(a.T >= 1 && a.Tc >= 1 && a.paso > 0.f, "%s: T, Tc and the streak step must be positive", what);
  return 0;
}

static int gate_groups(int64_t BL) {
  const int64_t g = (BL + kGateWaves - 1) / kGateWaves;
  return (int)(g < kGateMaxBlocks ? (g > 0 ? g : 1) : kGateMaxBlocks);
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_gate_fwd(const float* h, const void* aporte, int32_t aporte_bf16, const float* signals,
                             const float* vistos, const float* hawkes, const float* racha, const float* w_g,
                             const float* b_g, const float* w_conf, const float* b_conf, const float* w_vistos,
                             const float* u_hawkes, const float* d_racha, int64_t BL, int32_t d, int32_t n,
                             int32_t nodes, int32_t T, int32_t Tc, float racha_paso, float mejor_max, float tope,
                             float* logit, float* out, void* stream) {
  GateArgs a{};
  a.h = h; a.A = aporte; a.a_bf16 = aporte_bf16 != 0; a.sig = signals; a.vistos = vistos; a.hawkes = hawkes;
  a.racha = racha; a.wg = w_g; a.bg = b_g; a.wc = w_conf; a.bc = b_conf; a.wv = w_vistos; a.uh = u_hawkes;
  a.dr = d_racha; a.BL = BL; a.d = d; a.n = n; a.nodes = nodes; a.T = T; a.Tc = Tc; a.paso = racha_paso;
  a.mejor_max = mejor_max; a.tope = tope; a.logit = logit; a.out = out;
  if (gate_check(a, "asrn_gate_fwd")) return 1;
  if (BL == 0) return 0;
  const dim3 grid(gate_groups(BL)), block(kGateThreads);
  hipStream_t st = (hipStream_t)stream;
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {
    case 1: hipLaunchKernelGGL(k_gate_fwd<1>, grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL(k_gate_fwd<2>, grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL(k_gate_fwd<3>, grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL(k_gate_fwd<4>, grid, block, 0, st, a); break;
  }
  return check_launch("asrn_gate_fwd");
}

extern "C" int64_t asrn_gate_bwd_workspace(int64_t BL, int32_t d) {
  return (int64_t)gate_groups(BL) * (d + kGateCols) * (int64_t)sizeof(float);
}

extern "C" int asrn_gate_bwd(const float* h, const void* aporte, int32_t aporte_bf16, const float* signals,
                             const float* vistos, const float* hawkes, const float* racha, const float* w_g,
                             const float* b_g, const float* w_conf, const float* b_conf, const float* w_vistos,
                             const float* u_hawkes, const float* d_racha, int64_t BL, int32_t d, int32_t n,
                             int32_t nodes, int32_t T, int32_t Tc, float racha_paso, float mejor_max, float tope,
                             const float* logit, const float* dout, float* dh, void* daporte, float* dhawkes,
                             float* dracha, float* dparams, void* workspace, int64_t workspace_bytes, void* stream) {
  GateArgs a{};
  a.h = h; a.A = aporte; a.a_bf16 = aporte_bf16 != 0; a.sig = signals; a.vistos = vistos; a.hawkes = hawkes;
  a.racha = racha; a.wg = w_g; a.bg = b_g; a.wc = w_conf; a.bc = b_conf; a.wv = w_vistos; a.uh = u_hawkes;
  a.dr = d_racha; a.BL = BL; a.d = d; a.n = n; a.nodes = nodes; a.T = T; a.Tc = Tc; a.paso = racha_paso;
  a.mejor_max = mejor_max; a.tope = tope; a.logit = (float*)logit; a.dout = dout; a.dh = dh; a.dA = daporte;
  a.dhawkes = dhawkes; a.dracha = dracha; a.partial = (float*)workspace;
  if (gate_check(a, "asrn_gate_bwd")) return 1;
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= asrn_gate_bwd_workspace(BL, d),
               "asrn_gate_bwd: workspace too small");
  const int groups = gate_groups(BL);
  const int cols = d + kGateCols;
  hipStream_t st = (hipStream_t)stream;
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {
    case 1: hipLaunchKernelGGL(k_gate_bwd<1>, dim3(groups), dim3(kGateThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL(k_gate_bwd<2>, dim3(groups), dim3(kGateThreads), 0, st, a); break;
    case 3: hipLaunchKernelGGL(k_gate_bwd<3>, dim3(groups), dim3(kGateThreads), 0, st, a); break;
    default: hipLaunchKernelGGL(k_gate_bwd<4>, dim3(groups), dim3(kGateThreads), 0, st, a); break;
  }
  if (check_launch("asrn_gate_bwd")) return 1;
  hipLaunchKernelGGL(k_gate_params, dim3((cols + 255) / 256), dim3(256), 0, st, (const float*)workspace, groups,
                     cols, dparams);
  return check_launch("asrn_gate_bwd/params");
}
