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
// A workgroup takes 32 tokens: their small inputs (signals, seen flags, Hawkes, streak) are turned into features by one
// thread per token, then each wave runs 8 tokens' d-rows, as float4 per lane, loading 4 tokens' rows at a time so the
// loads overlap: h, A and h' stream through HBM once. In the forward wave w takes tokens w, w + 4, ... of the
// workgroup, so a short input (the generation step's B tokens) still spreads over all four waves.
// The backward gives dh, dA, dhawkes, dracha per token and the parameter gradients as per-workgroup partials summed
// in a fixed order by a second launch (deterministic, no atomics).
#include "common.h"

namespace asrn {

constexpr int kGateThreads = 256;
constexpr int kGateWaves = kGateThreads / kWave;
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

template <bool B16>
__device__ __forceinline__ float4 load_a4t(const void* p, int64_t q) {
  if constexpr (!B16) {
    return ((const float4*)p)[q];
  } else {
    const uint2 u = ((const uint2*)p)[q];   // four bf16, element 0 in the low half
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
  }
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

// The small part of the logit is linear in the packed small parameters P = [b_g | w_conf (4) | b_conf | w_vistos (n)
// | u_hawkes (n) | d_racha (nodes)]: logit = h . w_g + sum_c P_c f_c(t), with the features
//   f = [1 | sen (4) | 1 | vistos (n) | log1p(hawkes) (n) | [m <= i] + (x - i) [m == i + 1] for m < nodes]
// (the streak response cumsum(d_racha)[i] + (x - i) d_racha[i + 1] written per node). Phase 1 of each workgroup
// computes f for its tokens, one thread per token, into LDS; the d-row work then runs a wave per token.
constexpr int kGateTok = 32;             // tokens per workgroup
constexpr int kGateTokPerWave = kGateTok / kGateWaves;
constexpr int kGateBatch = 4;            // tokens whose rows a wave loads together
constexpr int kFeatStride = kGateCols + 1;

struct TokenInfo {
  float r;       // 1 / max(1, peso_total)
  float small;   // sum_c P_c f_c
  float dxdr;    // d x / d racha where the clamp passes, else 0
  int i;         // streak segment
};

__device__ __forceinline__ float small_param(const GateArgs& a, int c) {
  const int n = a.n;
  if (c == 0) return a.bg[0];
  if (c <= 4) return a.wc[c - 1];
  if (c == 5) return a.bc[0];
  if (c < 6 + n) return a.wv[c - 6];
  if (c < 6 + 2 * n) return a.uh[c - 6 - n];
  return a.dr[c - 6 - 2 * n];
}

constexpr int kGateMaxN = (kGateCols - 8) / 2;   // tables, at most (6 + 2 n + nodes <= kGateCols, nodes >= 2)

// phase 1: a token's features into f (LDS row), its info into ti, from its signals g (peso_total, mejor, pico,
// peso_ctx) and streak ra; P the staged small parameters, vis and haw the token's staged rows
__device__ void token_features_of(const GateArgs& a, float4 g, float ra, const float* P, const float* vis,
                                  const float* haw, float* f, TokenInfo* ti) {
  const int n = a.n, S = 6 + 2 * n + a.nodes;
  const float pt = g.x;
  float mejor = pt > 0.f ? g.y : 0.f;
  if (a.mejor_max >= 0.f) mejor = fminf(fmaxf(mejor, -a.mejor_max), a.mejor_max);
  f[0] = 1.f;
  f[1] = pt / (float)a.T;
  f[2] = mejor;
  f[3] = g.z / fmaxf(pt, 1.f);
  f[4] = g.w / (float)a.Tc;
  f[5] = 1.f;
  for (int j = 0; j < n; ++j) {
    f[6 + j] = vis[j];
    f[6 + n + j] = log1pf(haw[j]);
  }
  const float top = (float)(a.nodes - 1);
  const float xr = log1pf(ra) / a.paso;
  const float x = fminf(xr, top);
  float fi = x != x ? 0.f : floorf(x);
  fi = fminf(fmaxf(fi, 0.f), (float)(a.nodes - 2));
  const int i = (int)fi;
  for (int m = 0; m < a.nodes; ++m) f[6 + 2 * n + m] = (m <= i ? 1.f : 0.f) + (m == i + 1 ? x - fi : 0.f);
  float small = 0.f;
  for (int c = 0; c < S; ++c) small += P[c] * f[c];
  ti->r = 1.f / fmaxf(pt, 1.f);
  ti->small = small;
  ti->dxdr = xr <= top ? 1.f / ((1.f + ra) * a.paso) : 0.f;
  ti->i = i;
}

// the same for token t, its signals and streak read here
__device__ void token_features(const GateArgs& a, int64_t t, const float* P, const float* vis, const float* haw,
                               float* f, TokenInfo* ti) {
  token_features_of(a, ((const float4*)a.sig)[t], a.racha[t], P, vis, haw, f, ti);
}

// Phase 1 of the whole-text gate kernels with every load in one round: the small parameters, the workgroup's seen and
// Hawkes rows, and each token's signals and streak (one thread per token), as unconditional loads from clamped
// indices (a guarded load becomes a branch the compiler waits at), then the LDS staging and the features.
__device__ __forceinline__ void gate_prologue(const GateArgs& a, int64_t t0, float* P, float* vis, float* haw,
                                              float (*feat)[kFeatStride], TokenInfo* info) {
  constexpr int kRowLoads = (kGateTok * kGateMaxN + kGateThreads - 1) / kGateThreads;
  const int tid = threadIdx.x;
  const int64_t nt = a.BL - t0 < kGateTok ? a.BL - t0 : kGateTok;
  const int S = 6 + 2 * a.n + a.nodes, nr = (int)nt * a.n;
  const float pv = small_param(a, tid < S ? tid : S - 1);
  float vv[kRowLoads], hw[kRowLoads];
#pragma unroll
  for (int r = 0; r < kRowLoads; ++r) {
    const int i = tid + r * kGateThreads, ic = i < nr ? i : nr - 1;
    vv[r] = a.vistos[t0 * a.n + ic];
    hw[r] = a.hawkes[t0 * a.n + ic];
  }
  const int64_t tt = t0 + (tid < nt ? tid : nt - 1);
  const float4 sg = ((const float4*)a.sig)[tt];
  const float ra = a.racha[tt];
  if (tid < S) P[tid] = pv;
#pragma unroll
  for (int r = 0; r < kRowLoads; ++r) {
    const int i = tid + r * kGateThreads;
    if (i < nr) {
      vis[i] = vv[r];
      haw[i] = hw[r];
    }
  }
  __syncthreads();
  if (tid < nt) token_features_of(a, sg, ra, P, vis + tid * a.n, haw + tid * a.n, feat[tid], &info[tid]);
  __syncthreads();
}

__device__ __forceinline__ float capped(float l, float tope) { return tope > 0.f ? tope * tanhf(l / tope) : l; }

// AB16: A (the W_o product) in bf16. A batch's rows are loaded unconditionally from clamped indices (tokens past BL
// read the last token, columns past d the last column; those values are not used), so each batch is one round.
template <int D4, bool AB16>
__global__ __launch_bounds__(kGateThreads) void k_gate_fwd(GateArgs a) {
  __shared__ float feat[kGateTok][kFeatStride];
  __shared__ TokenInfo info[kGateTok];
  __shared__ float P[kGateCols];
  __shared__ float vh[2][kGateTok * kGateMaxN];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  const int64_t t0 = (int64_t)blockIdx.x * kGateTok;
  gate_prologue(a, t0, P, vh[0], vh[1], feat, info);
  constexpr int kB = D4 == 1 ? kGateBatch : 2;           // a batch's rows are all live at once: fewer past d 256
  float4 w[D4];
#pragma unroll
  for (int k = 0; k < D4; ++k) w[k] = ((const float4*)a.wg)[lane + kWave * k < d4 ? lane + kWave * k : d4 - 1];
  for (int b = 0; b < kGateTokPerWave; b += kB) {
    float4 hv[kB][D4], av[kB][D4];
    float dot[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int64_t t = t0 + wave + kGateWaves * (b + u), tc = t < a.BL ? t : a.BL - 1;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k, qc = q < d4 ? q : d4 - 1;
        hv[u][k] = ((const float4*)(a.h + tc * a.d))[qc];
        av[u][k] = load_a4t<AB16>(a.A, tc * d4 + qc);
      }
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int64_t t = t0 + wave + kGateWaves * (b + u);
      dot[u] = 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k)
        if (t < a.BL && lane + kWave * k < d4)
          dot[u] += hv[u][k].x * w[k].x + hv[u][k].y * w[k].y + hv[u][k].z * w[k].z + hv[u][k].w * w[k].w;
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int tl = wave + kGateWaves * (b + u);
      const int64_t t = t0 + tl;
      if (t >= a.BL) break;
      const float logit = wave_sum_u(dot[u]) + info[tl].small;
      if (lane == 0) a.logit[t] = logit;
      const float sr = info[tl].r / (1.f + expf(-capped(logit, a.tope)));
      float4* o4 = (float4*)(a.out + t * a.d);
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (q < d4)
          o4[q] = make_float4(hv[u][k].x + sr * av[u][k].x, hv[u][k].y + sr * av[u][k].y,
                              hv[u][k].z + sr * av[u][k].z, hv[u][k].w + sr * av[u][k].w);
      }
    }
  }
}

template <int D4, bool AB16>
__global__ __launch_bounds__(kGateThreads) void k_gate_bwd(GateArgs a) {
  __shared__ float feat[kGateTok][kFeatStride];
  __shared__ TokenInfo info[kGateTok];
  __shared__ float dl[kGateTok];
  __shared__ float red[kGateWaves][4 * D4 * kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  const int n = a.n, S = 6 + 2 * n + a.nodes;
  const int64_t t0 = (int64_t)blockIdx.x * kGateTok;
  __shared__ float P[kGateCols];
  __shared__ float vh[2][kGateTok * kGateMaxN];
  if (threadIdx.x < kGateTok) dl[threadIdx.x] = 0.f;         // ordered before its use by the prologue's barriers
  gate_prologue(a, t0, P, vh[0], vh[1], feat, info);
  // a batch's rows are all live at once: 4 tokens a batch at d <= 256, 2 past it (register pressure)
  constexpr int kB = D4 == 1 ? kGateBatch : 2;
  float4 gw[D4], w[D4];
#pragma unroll
  for (int k = 0; k < D4; ++k) {
    gw[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    w[k] = ((const float4*)a.wg)[lane + kWave * k < d4 ? lane + kWave * k : d4 - 1];
  }
  for (int b = 0; b < kGateTokPerWave; b += kB) {
    float4 gv[kB][D4], hv[kB][D4], av[kB][D4];
    float ga[kB], lg[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {                         // the batch's loads, unconditional (clamped indices)
      const int64_t t = t0 + wave * kGateTokPerWave + b + u, tc = t < a.BL ? t : a.BL - 1;
      lg[u] = a.logit[tc];
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k, qc = q < d4 ? q : d4 - 1;
        gv[u][k] = ((const float4*)(a.dout + tc * a.d))[qc];
        hv[u][k] = ((const float4*)(a.h + tc * a.d))[qc];
        av[u][k] = load_a4t<AB16>(a.A, tc * d4 + qc);
      }
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int64_t t = t0 + wave * kGateTokPerWave + b + u;
      ga[u] = 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k)
        if (t < a.BL && lane + kWave * k < d4)
          ga[u] += gv[u][k].x * av[u][k].x + gv[u][k].y * av[u][k].y + gv[u][k].z * av[u][k].z +
                   gv[u][k].w * av[u][k].w;
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int tl = wave * kGateTokPerWave + b + u;
      const int64_t t = t0 + tl;
      if (t >= a.BL) break;
      float dcap = 1.f, lc = lg[u];
      if (a.tope > 0.f) {
        const float th = tanhf(lg[u] / a.tope);
        lc = a.tope * th;
        dcap = 1.f - th * th;
      }
      const float sg = 1.f / (1.f + expf(-lc));
      const float r = info[tl].r;
      const float dlogit = wave_sum_u(ga[u]) * r * (sg * (1.f - sg)) * dcap;
      if (lane == 0) dl[tl] = dlogit;
      const float sr = sg * r;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (q < d4) {
          ((float4*)(a.dh + t * a.d))[q] = make_float4(gv[u][k].x + dlogit * w[k].x, gv[u][k].y + dlogit * w[k].y,
                                                       gv[u][k].z + dlogit * w[k].z, gv[u][k].w + dlogit * w[k].w);
          store_a4(a.dA, a.a_bf16, t * d4 + q,
                   make_float4(gv[u][k].x * sr, gv[u][k].y * sr, gv[u][k].z * sr, gv[u][k].w * sr));
          gw[k].x += dlogit * hv[u][k].x;
          gw[k].y += dlogit * hv[u][k].y;
          gw[k].z += dlogit * hv[u][k].z;
          gw[k].w += dlogit * hv[u][k].w;
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < D4; ++k) {
    const int q = lane + kWave * k;
    red[wave][4 * q + 0] = gw[k].x;
    red[wave][4 * q + 1] = gw[k].y;
    red[wave][4 * q + 2] = gw[k].z;
    red[wave][4 * q + 3] = gw[k].w;
  }
  __syncthreads();
  const int cols = a.d + kGateCols;
  float* prow = a.partial + (int64_t)blockIdx.x * cols;
  for (int c = threadIdx.x; c < a.d; c += kGateThreads) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kGateWaves; ++w) v += red[w][c];
    prow[c] = v;
  }
  const int tid = threadIdx.x;
  if (tid < kGateCols) {                 // the small parameters: tokens in order
    const int64_t left = a.BL - t0;
    const int ntok = left < kGateTok ? (int)left : kGateTok;
    float v = 0.f;
    if (tid < S)
      for (int tl = 0; tl < ntok; ++tl) v += dl[tl] * feat[tl][tid];
    prow[a.d + tid] = v;
  } else if (tid >= 128 && tid < 128 + kGateTok && t0 + (tid - 128) < a.BL) {   // per-token gradients
    const int tl = tid - 128;
    const int64_t t = t0 + tl;
    const float g = dl[tl];
    for (int j = 0; j < n; ++j) a.dhawkes[t * n + j] = g * a.uh[j] / (1.f + a.hawkes[t * n + j]);
    a.dracha[t] = g * a.dr[info[tl].i + 1] * info[tl].dxdr;
  }
}

// The generation step's W_o and gate in one launch (fp32, a few tokens): workgroup (nt, rt) owns output columns
// [16 nt, 16 nt + 16) of tokens [16 rt, 16 rt + 16). It forms the 16 x 16 tile of A = salida W_o^T on the matrix cores
// (v_mfma_f32_16x16x4f32) over the whole depth, each wave a quarter of it with all its loads in one round, and every
// token's logit (h . w_g as the fused gate forms it, and the small part from one thread per token), so that
// h' = h + sigmoid(cap(logit)) r A leaves for the tile's columns: the library GEMM and its A round trip through HBM
// are gone, and 48 workgroups (d = 768) share what was one workgroup's gate.
constexpr int kStepTok = 16;
typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4v ld4_rows(const float* m, int64_t row, int64_t nrows, int64_t ld, int k, int kend) {
  f4v v = {0.f, 0.f, 0.f, 0.f};
  if (row >= nrows) return v;
  const float* p = m + row * ld + k;
  if (k + 4 <= kend) return *(const f4v*)p;
  if (k + 0 < kend) v.x = p[0];
  if (k + 1 < kend) v.y = p[1];
  if (k + 2 < kend) v.z = p[2];
  if (k + 3 < kend) v.w = p[3];
  return v;
}

constexpr int kStepWaves = 8;                // a workgroup's waves, each an eighth of the depth in one round of loads
constexpr int kStepThreads = kStepWaves * kWave;
constexpr int kStepTokPerWave = kStepTok / kStepWaves;   // tokens whose h . w_g a wave forms

template <int D4, int U>
__global__ __launch_bounds__(kStepThreads) void k_gate_step(GateArgs a, const float* __restrict__ salida,
                                                            const float* __restrict__ wo) {
  __shared__ float tile[kStepWaves][kStepTok * kStepTok];
  __shared__ float feat[kStepTok][kFeatStride];
  __shared__ TokenInfo info[kStepTok];
  __shared__ float P[kGateCols];
  __shared__ float vh[2][kStepTok * kGateMaxN];
  __shared__ float hdot[kStepTok];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int d = a.d, d4 = d >> 2;
  const int n0 = blockIdx.x * kStepTok;
  const int64_t t0 = (int64_t)blockIdx.y * kStepTok;
  const int nt = a.BL - t0 < kStepTok ? (int)(a.BL - t0) : kStepTok;
  // Every load first, so that the kernel waits for memory once: the product's operands (wave w: depth [w per,
  // (w + 1) per) in U steps of 16 columns), the h . w_g operands (wave w: tokens w + kStepWaves j), the small
  // parameters, the tokens' seen and Hawkes rows, signals and streaks, and the h values the epilogue adds to.
  const int per = ((d + kStepWaves - 1) / kStepWaves + 15) & ~15;
  const int wb = wave * per, we = wb + per < d ? wb + per : d;
  const int i16 = lane & 15, q4 = lane >> 4;
  f4v x[U], w[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int kk = wb + 16 * u + 4 * q4;
    x[u] = ld4_rows(salida, t0 + i16, a.BL, d, kk, we);
    w[u] = ld4_rows(wo, n0 + i16, d, d, kk, we);
  }
  // (unconditional float4 loads: tokens past nt read token 0 and lanes past d column d - 4, values never used)
  float4 hv[kStepTokPerWave][D4], wg[D4];
#pragma unroll
  for (int k = 0; k < D4; ++k) {
    const int q = lane + kWave * k < d4 ? lane + kWave * k : d4 - 1;
    wg[k] = ((const float4*)a.wg)[q];
#pragma unroll
    for (int j = 0; j < kStepTokPerWave; ++j) {
      const int tl = wave + kStepWaves * j;
      hv[j][k] = ((const float4*)(a.h + (t0 + (tl < nt ? tl : 0)) * d))[q];
    }
  }
  const int S = 6 + 2 * a.n + a.nodes;
  const float pv = tid < S ? small_param(a, tid) : 0.f;
  const bool vin = tid < nt * a.n;                          // nt n <= kStepTok kGateMaxN < kStepThreads
  const float vv = vin ? a.vistos[t0 * a.n + tid] : 0.f, hw = vin ? a.hawkes[t0 * a.n + tid] : 0.f;
  float4 sg = make_float4(0.f, 0.f, 0.f, 0.f);
  float ra = 0.f;
  if (tid < nt) {
    sg = ((const float4*)a.sig)[t0 + tid];
    ra = a.racha[t0 + tid];
  }
  const int tl = tid / kStepTok, c = tid % kStepTok;        // the epilogue's element of the tile
  const int64_t t = t0 + tl;
  const int col = n0 + c;
  const bool mine = tid < kStepTok * kStepTok && tl < nt && col < d;
  const float hx = mine ? a.h[t * d + col] : 0.f;
  // the tile: rows 4 (l / 16) + q, column l % 16 of each wave's partial
  f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].x, w[u].x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].y, w[u].y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].z, w[u].z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].w, w[u].w, acc, 0, 0, 0);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) tile[wave][(4 * q4 + q) * kStepTok + i16] = acc[q];
  // h . w_g per token, as the fused gate forms it (float4 lanes, then the wave sum)
#pragma unroll
  for (int j = 0; j < kStepTokPerWave; ++j) {
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < D4; ++k)
      if (lane + kWave * k < d4)
        dot += hv[j][k].x * wg[k].x + hv[j][k].y * wg[k].y + hv[j][k].z * wg[k].z + hv[j][k].w * wg[k].w;
    dot = wave_sum_u(dot);
    if (lane == 0) hdot[wave + kStepWaves * j] = dot;
  }
  if (tid < S) P[tid] = pv;
  if (vin) {
    vh[0][tid] = vv;
    vh[1][tid] = hw;
  }
  __syncthreads();
  if (tid < nt) token_features_of(a, sg, ra, P, vh[0] + tid * a.n, vh[1] + tid * a.n, feat[tid], &info[tid]);
  __syncthreads();
  if (mine) {
    const int e = tl * kStepTok + c;
    float A = tile[0][e];
#pragma unroll
    for (int i = 1; i < kStepWaves; ++i) A += tile[i][e];
    const float logit = hdot[tl] + info[tl].small;
    if (blockIdx.x == 0 && c == 0) a.logit[t] = logit;
    const float sr = info[tl].r / (1.f + expf(-capped(logit, a.tope)));
    a.out[t * d + col] = hx + sr * A;
  }
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

// one workgroup per kGateTok tokens (the backward writes a row of parameter partials per workgroup)
static int64_t gate_groups(int64_t BL) { return BL > 0 ? (BL + kGateTok - 1) / kGateTok : 1; }

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
  ASRN_REQUIRE(gate_groups(BL) < (int64_t(1) << 31), "asrn_gate_fwd: too many tokens");
  const dim3 grid((unsigned)gate_groups(BL)), block(kGateThreads);
  hipStream_t st = (hipStream_t)stream;
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {
    case 1: hipLaunchKernelGGL((a.a_bf16 ? k_gate_fwd<1, true> : k_gate_fwd<1, false>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((a.a_bf16 ? k_gate_fwd<2, true> : k_gate_fwd<2, false>), grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL((a.a_bf16 ? k_gate_fwd<3, true> : k_gate_fwd<3, false>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((a.a_bf16 ? k_gate_fwd<4, true> : k_gate_fwd<4, false>), grid, block, 0, st, a); break;
  }
  return check_launch("asrn_gate_fwd");
}

extern "C" int asrn_gate_step(const float* h, const float* salida, const float* w_o, const float* signals,
                              const float* vistos, const float* hawkes, const float* racha, const float* w_g,
                              const float* b_g, const float* w_conf, const float* b_conf, const float* w_vistos,
                              const float* u_hawkes, const float* d_racha, int64_t BL, int32_t d, int32_t n,
                              int32_t nodes, int32_t T, int32_t Tc, float racha_paso, float mejor_max, float tope,
                              float* logit, float* out, void* stream) {
  GateArgs a{};
  a.h = h; a.A = nullptr; a.sig = signals; a.vistos = vistos; a.hawkes = hawkes;
  a.racha = racha; a.wg = w_g; a.bg = b_g; a.wc = w_conf; a.bc = b_conf; a.wv = w_vistos; a.uh = u_hawkes;
  a.dr = d_racha; a.BL = BL; a.d = d; a.n = n; a.nodes = nodes; a.T = T; a.Tc = Tc; a.paso = racha_paso;
  a.mejor_max = mejor_max; a.tope = tope; a.logit = logit; a.out = out;
  if (gate_check(a, "asrn_gate_step")) return 1;
  ASRN_REQUIRE(n <= kGateMaxN, "asrn_gate_step: n=%d above %d", n, kGateMaxN);
  ASRN_REQUIRE(BL <= (int64_t(1) << 20), "asrn_gate_step: %lld tokens: the step's few tokens only", (long long)BL);
  for (const void* p : {(const void*)h, (const void*)salida, (const void*)w_o, (const void*)w_g, (const void*)out})
    ASRN_REQUIRE(((uintptr_t)p & 15) == 0, "asrn_gate_step: rows are read as float4: 16-byte alignment");
  if (BL == 0) return 0;
  const dim3 grid((unsigned)((d + kStepTok - 1) / kStepTok), (unsigned)((BL + kStepTok - 1) / kStepTok));
  const dim3 block(kStepThreads);
  hipStream_t st = (hipStream_t)stream;
  const int per = ((d + kStepWaves - 1) / kStepWaves + 15) & ~15;   // a wave's depth
  // the kernels make one pass of U steps: 16 U covers per for every d <= 1024 with the U picked below
  ASRN_REQUIRE(per <= 16 * 8, "asrn_gate_step: d=%d: a wave's depth %d above 128", d, per);
  auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, st, a, salida, w_o); };
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {              // float4 columns a lane holds of h; U steps of 16
    case 1: per <= 16 ? launch(k_gate_step<1, 1>) : (per <= 32 ? launch(k_gate_step<1, 2>) : launch(k_gate_step<1, 4>));
            break;
    case 2: launch(k_gate_step<2, 4>); break;
    case 3: launch(k_gate_step<3, 6>); break;
    default: launch(k_gate_step<4, 8>); break;
  }
  return check_launch("asrn_gate_step");
}

extern "C" int64_t asrn_gate_bwd_workspace(int64_t BL, int32_t d) {
  return gate_groups(BL) * (d + kGateCols) * (int64_t)sizeof(float);
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
  ASRN_REQUIRE(gate_groups(BL) < (int64_t(1) << 31), "asrn_gate_bwd: too many tokens");
  const int groups = (int)gate_groups(BL);
  const int cols = d + kGateCols;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)groups), block(kGateThreads);
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {
    case 1: hipLaunchKernelGGL((a.a_bf16 ? k_gate_bwd<1, true> : k_gate_bwd<1, false>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((a.a_bf16 ? k_gate_bwd<2, true> : k_gate_bwd<2, false>), grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL((a.a_bf16 ? k_gate_bwd<3, true> : k_gate_bwd<3, false>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((a.a_bf16 ? k_gate_bwd<4, true> : k_gate_bwd<4, false>), grid, block, 0, st, a); break;
  }
  if (check_launch("asrn_gate_bwd")) return 1;
  return group_sums((const float*)workspace, groups, cols, dparams, st);
}
