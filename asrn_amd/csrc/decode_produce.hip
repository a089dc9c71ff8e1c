// a14 (part): the generation step's per-token producers, fused (reference asrn/nucleo.py:1797-1826, the producers of
// asrn/nucleo.py:644-659, 683 and asrn/estable.py:153-194 applied to one new token).
//
// For each of the B texts, the new token at position t (e_t its embedding, e_prev the previous one, h_t its layer
// input, its id) gives the rows the step's attention reads, written straight into the caches (B, cap, .):
//   V[t-1]  = W_v e_t                                            (the value of the previous position)
//   phi[t]  = [W2w gelu(W_p e_t + b_p) + b2w | W2c gelu((W_a e_t + b_c) + W_b e_prev) + b2c]
//   Qc[t], Kc[t] = cq hh, ck hh with hh = LayerNorm(h_t) (biased variance, two passes)
//   log_alfa[t] = max(logsigmoid(u_1) + log 2, log_alfa_min), and beta = min(softplus(u_0), beta_max) returned in fp64
//              for the repetition step, u_k = hh . w_reloj[k] + b_reloj[k]
//   sig[t]  = the token id in fp32
// The context MLP's first layer is read in place as its (mc, 2 d) weight: a row's first d columns act on e_t (W_a) and
// its last d on e_prev (W_b).
//
// Two launches. The first splits the weight rows into blocks of 4 (W_v, W_p, W_a, W_b, cq, ck); a workgroup stages
// 4 tokens' input vectors in LDS (e_t, e_prev, or hh with the LayerNorm done there) and each wave dots one row with
// them, so every weight row is read once per 4 tokens. The step is latency-bound, not bandwidth-bound: one row and
// 4 tokens per wave keep each wave's chain of dot products short and spread the launch over the whole chip (d = 768,
// B = 16: about 1080 workgroups; 16 tokens and 16 rows per workgroup took 31 us, this 8). The second takes one token per workgroup: the hidden units,
// both second layers and the clock. Every sum runs in a fixed order. The position is t, or *t_dev (a step replayed
// from a graph); a position outside [1, cap) writes nothing.
#include "block_pending.h"

namespace asrn {

constexpr int kProdThreads = 256;
constexpr int kProdWaves = kProdThreads / kWave;
constexpr int kProdRows = kProdWaves; // weight rows per workgroup of the first launch: one per wave
constexpr int kProdTok = 4;            // tokens per workgroup of the first launch
constexpr int kProdMaxD4 = 4;          // d <= 1024
constexpr int kProdMax = 64;           // hidden units, outputs per hash MLP, and cf, at most

struct ProdArgs {
  const float* e; const float* e_prev; const float* h; const int64_t* pieza; int64_t B; int d;
  const float* wv; const float* ww; const float* wc;        // W_v (d, d), W_p (m, d), the context first layer (mc, 2d)
  const float* bw; const float* bc;                         // first-layer biases (m), (mc)
  const float* w2w; const float* b2w; const float* w2c; const float* b2c;
  const float* lnw; const float* lnb; float eps;
  const float* wr; const float* br; float beta_max; float la_min;
  const float* wq; const float* wk;                         // cq (cf, d), ck (cf, d)
  int m, mc, Pw, Pc, cf;
  float* phi; float* V; float* Qc; float* Kc; float* sig; float* la; int64_t cap; int64_t t; const int64_t* t_dev;
  double* beta; float* y;                                   // beta (B); y (B, m + 2 mc): the first layers' products
};

constexpr int kMaxLayers = 8;          // layers one batched launch takes
struct ProdBatch {                     // every layer's arguments (the same sizes and position in each)
  ProdArgs l[kMaxLayers];
};

__device__ __forceinline__ int64_t prod_pos(const ProdArgs& a) { return a.t_dev ? *a.t_dev : a.t; }

__device__ __forceinline__ float dot4(float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }

// rows of kind k: 0 W_v (on e), 1 W_p (on e), 2 W_a (on e), 3 W_b (on e_prev), 4 cq (on hh), 5 ck (on hh)
__device__ __forceinline__ int kind_rows(const ProdArgs& a, int k) {
  return k == 0 ? a.d : (k == 1 ? a.m : (k <= 3 ? a.mc : a.cf));
}

// LayerNorm of the staged rows x[tok][.] (d4 float4 each) in place: wave w takes tokens w, w + 4, ...; lw and lb the
// lane's columns lane + 64 k of the weights, loaded beforehand
template <int D4>
__device__ __forceinline__ void layer_norm_rows(const ProdArgs& a, float4* xs, int ntok, int d4, const float4 (&lw)[D4],
                                                const float4 (&lb)[D4]) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const float inv_d = 1.f / (float)a.d;
  for (int j = wave; j < ntok; j += kProdWaves) {
    float4* x = xs + j * d4;
    float s = 0.f;
    for (int q = lane; q < d4; q += kWave) s += (x[q].x + x[q].y) + (x[q].z + x[q].w);
    const float mean = wave_sum_u(s) * inv_d;
    float v = 0.f;
    for (int q = lane; q < d4; q += kWave) {
      const float4 c = make_float4(x[q].x - mean, x[q].y - mean, x[q].z - mean, x[q].w - mean);
      v += dot4(c, c);
    }
    const float rstd = rsqrtf(wave_sum_u(v) * inv_d + a.eps);
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      const int q = lane + kWave * k;
      if (q >= d4) continue;
      const float4 w = lw[k], b = lb[k];
      x[q] = make_float4((x[q].x - mean) * rstd * w.x + b.x, (x[q].y - mean) * rstd * w.y + b.y,
                         (x[q].z - mean) * rstd * w.z + b.z, (x[q].w - mean) * rstd * w.w + b.w);
    }
  }
}

// the products of the rows of kinds [k_lo, k_hi) (blockIdx.x: a block of kProdRows rows of one kind; blockIdx.y: a
// group of kProdTok tokens)
template <int D4>
__device__ __forceinline__ void rows_body(const ProdArgs& a, int k_lo, int k_hi, float4* xs) {
  const int64_t t = prod_pos(a);
  if (t < 1 || t >= a.cap) return;                          // the same for the whole grid
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  // which kind and block
  int k = k_lo, blk = blockIdx.x;
  for (; k < k_hi - 1; ++k) {
    const int nb = (kind_rows(a, k) + kProdRows - 1) / kProdRows;
    if (blk < nb) break;
    blk -= nb;
  }
  const int nrows = kind_rows(a, k);
  const int64_t b0 = (int64_t)blockIdx.y * kProdTok;
  const int ntok = a.B - b0 < kProdTok ? (int)(a.B - b0) : kProdTok;
  // wave w dots row w of the block with every token: the row, and for the LayerNorm kinds the LayerNorm's weights,
  // are loaded first (they do not depend on the inputs staged next)
  const int r = blk * kProdRows + wave;
  float4 w[D4], lw[D4], lb[D4];
#pragma unroll
  for (int kk = 0; kk < D4; ++kk) {
    const int q = lane + kWave * kk;
    const bool in = k >= 4 && q < d4;
    lw[kk] = in ? ((const float4*)a.lnw)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    lb[kk] = in ? ((const float4*)a.lnb)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  {
    const float* row = k == 0 ? a.wv + (int64_t)r * a.d
                     : (k == 1 ? a.ww + (int64_t)r * a.d
                     : (k == 2 ? a.wc + (int64_t)r * 2 * a.d
                     : (k == 3 ? a.wc + (int64_t)r * 2 * a.d + a.d
                     : (k == 4 ? a.wq + (int64_t)r * a.d : a.wk + (int64_t)r * a.d))));
#pragma unroll
    for (int kk = 0; kk < D4; ++kk) {
      const int q = lane + kWave * kk;
      w[kk] = r < nrows && q < d4 ? ((const float4*)row)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  // stage the input vectors
  const float* src = k == 3 ? a.e_prev : (k >= 4 ? a.h : a.e);
  for (int i = threadIdx.x; i < ntok * d4; i += kProdThreads) {
    const int j = i / d4, q = i - j * d4;
    xs[j * d4 + q] = ((const float4*)(src + (b0 + j) * a.d))[q];
  }
  __syncthreads();
  if (k >= 4) {
    layer_norm_rows(a, xs, ntok, d4, lw, lb);
    __syncthreads();
  }
  for (int j = 0; j < ntok; ++j) {
    const int64_t b = b0 + j;
    {
      float p = 0.f;
#pragma unroll
      for (int kk = 0; kk < D4; ++kk) {
        const int q = lane + kWave * kk;
        if (q < d4) p += dot4(w[kk], xs[j * d4 + q]);
      }
      const float s = wave_sum_u(p);
      if (lane == 0 && r < nrows) {
        const int n1 = a.m + 2 * a.mc;
        if (k == 0) a.V[(b * a.cap + t - 1) * a.d + r] = s;
        else if (k == 1) a.y[b * n1 + r] = s;
        else if (k == 2) a.y[b * n1 + a.m + r] = s;
        else if (k == 3) a.y[b * n1 + a.m + a.mc + r] = s;
        else if (k == 4) a.Qc[(b * a.cap + t) * a.cf + r] = s;
        else a.Kc[(b * a.cap + t) * a.cf + r] = s;
      }
    }
  }
}

template <int D4>
__global__ __launch_bounds__(kProdThreads) void k_produce_rows(ProdArgs a) {
  __shared__ float4 xs[kProdTok * kProdMaxD4 * kWave];
  rows_body<D4>(a, 0, 6, xs);
}

// every layer's rows that act on e_t and e_prev (kinds 0-3), layer blockIdx.z
template <int D4>
__global__ __launch_bounds__(kProdThreads) void k_produce_rows_e(ProdBatch pb) {
  __shared__ float4 xs[kProdTok * kProdMaxD4 * kWave];
  rows_body<D4>(pb.l[blockIdx.z], 0, 4, xs);
}

__device__ __forceinline__ float gelu_exact(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }
__device__ __forceinline__ float softplus_p(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float logsigmoid_p(float x) { return fminf(x, 0.f) - log1pf(expf(-fabsf(x))); }

// one token per workgroup (row b): with E, the hidden units, both second layers and the token id; with H, the clock
template <bool E, bool H>
__device__ __forceinline__ void token_body(const ProdArgs& a, int64_t b, float* g) {
  const int64_t t = prod_pos(a);
  if (t < 1 || t >= a.cap) return;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  if constexpr (E) {
    const int n1 = a.m + 2 * a.mc;
    const float* yb = a.y + b * n1;
    if (tid < a.m) g[tid] = gelu_exact(yb[tid] + a.bw[tid]);
    else if (tid < a.m + a.mc) {
      const int j = tid - a.m;
      g[tid] = gelu_exact((yb[a.m + j] + a.bc[j]) + yb[a.m + a.mc + j]);
    }
    __syncthreads();
    const int P = a.Pw + a.Pc;
    if (tid < a.Pw) {
      float s = 0.f;
      for (int j = 0; j < a.m; ++j) s += a.w2w[tid * a.m + j] * g[j];
      a.phi[(b * a.cap + t) * P + tid] = s + a.b2w[tid];
    } else if (tid < P) {
      const int o = tid - a.Pw;
      float s = 0.f;
      for (int j = 0; j < a.mc; ++j) s += a.w2c[o * a.mc + j] * g[a.m + j];
      a.phi[(b * a.cap + t) * P + tid] = s + a.b2c[o];
    }
    if (tid == kProdThreads - 1) a.sig[b * a.cap + t] = (float)a.pieza[b];
  }
  if (H && wave == kProdWaves - 1) {                        // the clock: LayerNorm of h_t and its two projections
    const int d4 = a.d >> 2;
    const float inv_d = 1.f / (float)a.d;
    const float4* x = (const float4*)(a.h + b * a.d);
    float s = 0.f;
    for (int q = lane; q < d4; q += kWave) s += (x[q].x + x[q].y) + (x[q].z + x[q].w);
    const float mean = wave_sum_u(s) * inv_d;
    float v = 0.f;
    for (int q = lane; q < d4; q += kWave) {
      const float4 c = make_float4(x[q].x - mean, x[q].y - mean, x[q].z - mean, x[q].w - mean);
      v += dot4(c, c);
    }
    const float rstd = rsqrtf(wave_sum_u(v) * inv_d + a.eps);
    float u0 = 0.f, u1 = 0.f;
    for (int q = lane; q < d4; q += kWave) {
      const float4 w = ((const float4*)a.lnw)[q], bb = ((const float4*)a.lnb)[q];
      const float4 yv = make_float4((x[q].x - mean) * rstd * w.x + bb.x, (x[q].y - mean) * rstd * w.y + bb.y,
                                    (x[q].z - mean) * rstd * w.z + bb.z, (x[q].w - mean) * rstd * w.w + bb.w);
      u0 += dot4(yv, ((const float4*)a.wr)[q]);
      u1 += dot4(yv, ((const float4*)(a.wr + a.d))[q]);
    }
    u0 = wave_sum_u(u0) + a.br[0];
    u1 = wave_sum_u(u1) + a.br[1];
    if (lane == 0) {
      float be = softplus_p(u0);
      if (a.beta_max >= 0.f) be = fminf(be, a.beta_max);
      a.beta[b] = (double)be;
      a.la[b * a.cap + t] = fmaxf(logsigmoid_p(u1) + 0.69314718055994530942f, a.la_min);
    }
  }
}

__global__ __launch_bounds__(kProdThreads) void k_produce_token(ProdArgs a) {
  __shared__ float g[2 * kProdMax];
  token_body<true, true>(a, blockIdx.x, g);
}

// every layer's hidden units, second layers and token id (layer blockIdx.y)
__global__ __launch_bounds__(kProdThreads) void k_produce_token_e(ProdBatch pb) {
  __shared__ float g[2 * kProdMax];
  token_body<true, false>(pb.l[blockIdx.y], blockIdx.x, g);
}

// The rows that act on the layer input h_t, one token per workgroup of kHWaves waves: hh = LayerNorm(h_t), each wave
// forming it for itself; Qc = cq hh and Kc = ck hh, rows r = w, w + (kHWaves - 1), ... of the 2 cf by wave w, kHChunk
// rows in flight; the clock from w_reloj hh + b_reloj by the last wave. The sums are those of the two-kernel producer
// in the same order (layer_norm_rows, the rows' products, the clock), so the outputs are the same bits. Every load of
// the first chunk is issued before the row's statistics.
// PEND: h_t is the output of a local block step left pending (block_pending.h), formed here first: thread c sums
// column c as the block step's k_finish_res does, writes it to pv.out and the block's z into its ring (slot *pend_pos
// mod k - 1), and stages it in LDS for the waves' LayerNorm. Those loads are issued before the weight rows', so the
// sum waits only on them (the load counter counts in order); the block's output is formed whatever the position.
constexpr int kHWaves = 16;
constexpr int kHChunk = 4;

template <int D4, int S, bool PEND>
__global__ __launch_bounds__(kHWaves * kWave) void k_produce_h(ProdArgs a, Pending pv, const int64_t* pend_pos) {
  __shared__ float row_s[PEND ? 4 * kProdMaxD4 * kWave : 1];
  const int64_t t = prod_pos(a);
  const bool live = t >= 1 && t < a.cap;
  if (!PEND && !live) return;
  const int64_t b = blockIdx.x;
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  float pv_x = 0.f, pv_b = 0.f, pv_z = 0.f, pv_p[S];
  const int c = threadIdx.x, cc = c < a.d ? c : a.d - 1;   // d <= 4 kProdMaxD4 kWave = the workgroup's threads
  int slot = 0;
  if constexpr (PEND) {
    slot = pv.km1 > 0 ? (int)(*pend_pos % pv.km1) : 0;
    pv_x = pv.h1[b * a.d + cc];
    split_loads<S>(pv.part + b * a.d + cc, pv.splits, gridDim.x * (int64_t)a.d, pv_p);
    pv_b = pv.bias[cc];
    pv_z = pv.km1 > 0 ? pv.z[b * a.d + cc] : 0.f;
  }
  const float inv_d = 1.f / (float)a.d;
  const bool clk = wave == kHWaves - 1;
  const int nr = 2 * a.cf;
  // rows past 2 cf read row 0 and lanes past d read column d - 4: every load is an unconditional float4 (a guarded
  // one is split by the compiler into four predicated loads), and those values are never used
  auto row_of = [&](int r) {
    r = r < nr ? r : 0;
    return r < a.cf ? a.wq + (int64_t)r * a.d : a.wk + (int64_t)(r - a.cf) * a.d;
  };
  float4 x[D4], lw[D4], lb[D4], w[kHChunk][D4];
#pragma unroll
  for (int k = 0; k < D4; ++k) {
    const int q = lane + kWave * k < d4 ? lane + kWave * k : d4 - 1;
    if constexpr (!PEND) x[k] = ((const float4*)(a.h + b * a.d))[q];
    lw[k] = ((const float4*)a.lnw)[q];
    lb[k] = ((const float4*)a.lnb)[q];
#pragma unroll
    for (int i = 0; i < kHChunk; ++i) {
      const float* row = clk ? a.wr + (int64_t)(i & 1) * a.d : row_of(wave + (kHWaves - 1) * i);
      w[i][k] = ((const float4*)row)[q];
    }
  }
  if constexpr (PEND) {
    const float v = pv_x + (split_total<S>(pv_p, pv.splits) + pv_b);
    if (c < a.d) {
      pv.out[b * a.d + c] = v;
      if (pv.km1 > 0) pv.ring[(b * a.d + c) * pv.km1 + slot] = pv_z;
      row_s[c] = v;
    }
    __syncthreads();
    if (!live) return;
#pragma unroll
    for (int k = 0; k < D4; ++k)
      x[k] = reinterpret_cast<const float4*>(row_s)[lane + kWave * k < d4 ? lane + kWave * k : d4 - 1];
  }
  // hh, as layer_norm_rows forms it
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < D4; ++k)
    if (lane + kWave * k < d4) s += (x[k].x + x[k].y) + (x[k].z + x[k].w);
  const float mean = wave_sum_u(s) * inv_d;
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < D4; ++k) {
    if (lane + kWave * k >= d4) continue;
    const float4 c = make_float4(x[k].x - mean, x[k].y - mean, x[k].z - mean, x[k].w - mean);
    v += dot4(c, c);
  }
  const float rstd = rsqrtf(wave_sum_u(v) * inv_d + a.eps);
  float4 hh[D4];
#pragma unroll
  for (int k = 0; k < D4; ++k)
    hh[k] = make_float4((x[k].x - mean) * rstd * lw[k].x + lb[k].x, (x[k].y - mean) * rstd * lw[k].y + lb[k].y,
                        (x[k].z - mean) * rstd * lw[k].z + lb[k].z, (x[k].w - mean) * rstd * lw[k].w + lb[k].w);
  if (clk) {                                                // the clock
    float u0 = 0.f, u1 = 0.f;
#pragma unroll
    for (int k = 0; k < D4; ++k) {
      if (lane + kWave * k >= d4) continue;
      u0 += dot4(hh[k], w[0][k]);
      u1 += dot4(hh[k], w[1][k]);
    }
    u0 = wave_sum_u(u0) + a.br[0];
    u1 = wave_sum_u(u1) + a.br[1];
    if (lane == 0) {
      float be = softplus_p(u0);
      if (a.beta_max >= 0.f) be = fminf(be, a.beta_max);
      a.beta[b] = (double)be;
      a.la[b * a.cap + t] = fmaxf(logsigmoid_p(u1) + 0.69314718055994530942f, a.la_min);
    }
    return;
  }
  for (int i0 = 0;; i0 += kHChunk) {                        // Qc and Kc, kHChunk rows of this wave at a time
    if (wave + (kHWaves - 1) * i0 >= nr) break;             // wave-uniform
    if (i0 > 0) {
#pragma unroll
      for (int i = 0; i < kHChunk; ++i) {
        const float* row = row_of(wave + (kHWaves - 1) * (i0 + i));
#pragma unroll
        for (int k = 0; k < D4; ++k) w[i][k] = ((const float4*)row)[lane + kWave * k < d4 ? lane + kWave * k : d4 - 1];
      }
    }
#pragma unroll
    for (int i = 0; i < kHChunk; ++i) {
      const int r = wave + (kHWaves - 1) * (i0 + i);
      float p = 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k)
        if (lane + kWave * k < d4) p += dot4(w[i][k], hh[k]);
      const float sr = wave_sum_u(p);
      if (lane == 0 && r < nr) {
        if (r < a.cf) a.Qc[(b * a.cap + t) * a.cf + r] = sr;
        else a.Kc[(b * a.cap + t) * a.cf + r - a.cf] = sr;
      }
    }
  }
}

static int kind_rows_host(int d, int m, int mc, int cf, int k) {
  return k == 0 ? d : (k == 1 ? m : (k <= 3 ? mc : cf));
}

}  // namespace asrn

using namespace asrn;

extern "C" int64_t asrn_decode_produce_workspace(int64_t B, int32_t m, int32_t mc) {
  if (B < 0 || m < 0 || mc < 0) return -1;
  return B * (int64_t)(m + 2 * mc) * (int64_t)sizeof(float);
}

extern "C" int asrn_decode_produce(const float* e, const float* e_prev, const float* h, const int64_t* pieza,
                                   int64_t B, int32_t d, const float* w_v, const float* w_word, const float* w_ctx,
                                   const float* b_word, const float* b_ctx, const float* w2_word,
                                   const float* b2_word, const float* w2_ctx, const float* b2_ctx, int32_t m,
                                   int32_t mc, int32_t p_word, int32_t p_ctx, const float* ln_w, const float* ln_b,
                                   float eps, const float* w_reloj, const float* b_reloj, float beta_max,
                                   float log_alfa_min, const float* w_cq, const float* w_ck, int32_t cf, float* phi,
                                   float* V, float* Qc, float* Kc, float* sig, float* log_alfa, int64_t cap,
                                   int64_t t, const int64_t* t_dev, double* beta, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(B >= 0 && d > 0 && d % 4 == 0 && d <= 4 * kProdMaxD4 * kWave,
               "asrn_decode_produce: d=%d must be a positive multiple of 4, <= %d", d, 4 * kProdMaxD4 * kWave);
  ASRN_REQUIRE(m >= 1 && mc >= 1 && m <= kProdMax && mc <= kProdMax && p_word >= 1 && p_ctx >= 1 &&
                   p_word + p_ctx <= kProdThreads && cf >= 1 && cf <= kProdMax,
               "asrn_decode_produce: m=%d, mc=%d, cf=%d must be in [1, %d], Pw + Pc=%d in [2, %d]", m, mc, cf, kProdMax,
               p_word + p_ctx, kProdThreads);
  ASRN_REQUIRE(eps > 0.f, "asrn_decode_produce: eps must be positive");
  ASRN_REQUIRE(t >= 1 && t < cap, "asrn_decode_produce: position t=%lld outside [1, capacity %lld)", (long long)t,
               (long long)cap);
  const int64_t need = asrn_decode_produce_workspace(B, m, mc);
  ASRN_REQUIRE(workspace != nullptr || need == 0, "asrn_decode_produce: needs a workspace of %lld bytes",
               (long long)need);
  ASRN_REQUIRE(workspace_bytes >= need, "asrn_decode_produce: workspace of %lld bytes, needs %lld",
               (long long)workspace_bytes, (long long)need);
  for (const void* p : {(const void*)e, (const void*)e_prev, (const void*)h, (const void*)w_v, (const void*)w_word,
                        (const void*)w_ctx, (const void*)ln_w, (const void*)ln_b, (const void*)w_reloj,
                        (const void*)w_cq, (const void*)w_ck})
    ASRN_REQUIRE(((uintptr_t)p & 15) == 0, "asrn_decode_produce: the rows are read as float4: 16-byte alignment");
  if (B == 0) return 0;
  ProdArgs a = {e, e_prev, h, pieza, B, d, w_v, w_word, w_ctx, b_word, b_ctx, w2_word, b2_word, w2_ctx, b2_ctx, ln_w,
                ln_b, eps, w_reloj, b_reloj, beta_max, log_alfa_min, w_cq, w_ck, m, mc, p_word, p_ctx, cf, phi, V, Qc,
                Kc, sig, log_alfa, cap, t, t_dev, beta, (float*)workspace};
  int blocks = 0;
  for (int k = 0; k < 6; ++k) blocks += (kind_rows_host(d, m, mc, cf, k) + kProdRows - 1) / kProdRows;
  const dim3 grid((unsigned)blocks, (unsigned)((B + kProdTok - 1) / kProdTok));
  hipStream_t st = (hipStream_t)stream;
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {
    case 1: hipLaunchKernelGGL(k_produce_rows<1>, grid, dim3(kProdThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL(k_produce_rows<2>, grid, dim3(kProdThreads), 0, st, a); break;
    case 3: hipLaunchKernelGGL(k_produce_rows<3>, grid, dim3(kProdThreads), 0, st, a); break;
    default: hipLaunchKernelGGL(k_produce_rows<4>, grid, dim3(kProdThreads), 0, st, a); break;
  }
  if (check_launch("asrn_decode_produce/rows")) return 1;
  hipLaunchKernelGGL(k_produce_token, dim3((unsigned)B), dim3(kProdThreads), 0, st, a);
  return check_launch("asrn_decode_produce/token");
}

extern "C" int64_t asrn_decode_produce_e_workspace(int32_t L, int64_t B, int32_t m, int32_t mc) {
  if (L < 0 || B < 0 || m < 0 || mc < 0) return -1;
  return (int64_t)L * B * (int64_t)(m + 2 * mc) * (int64_t)sizeof(float);
}

extern "C" int asrn_decode_produce_e(int32_t L, const float* e, const float* e_prev, const int64_t* pieza, int64_t B,
                                     int32_t d, const float* const* w_v, const float* const* w_word,
                                     const float* const* w_ctx, const float* const* b_word, const float* const* b_ctx,
                                     const float* const* w2_word, const float* const* b2_word,
                                     const float* const* w2_ctx, const float* const* b2_ctx, int32_t m, int32_t mc,
                                     int32_t p_word, int32_t p_ctx, float* const* phi, float* const* V,
                                     float* const* sig, int64_t cap, int64_t t, const int64_t* t_dev, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(L >= 1 && L <= kMaxLayers, "asrn_decode_produce_e: L=%d layers must be in [1, %d]", L, kMaxLayers);
  ASRN_REQUIRE(B >= 0 && B <= 65535 && d > 0 && d % 4 == 0 && d <= 4 * kProdMaxD4 * kWave,
               "asrn_decode_produce_e: B=%lld, d=%d: d a positive multiple of 4, <= %d", (long long)B, d,
               4 * kProdMaxD4 * kWave);
  ASRN_REQUIRE(m >= 1 && mc >= 1 && m <= kProdMax && mc <= kProdMax && p_word >= 1 && p_ctx >= 1 &&
                   p_word + p_ctx <= kProdThreads,
               "asrn_decode_produce_e: m=%d, mc=%d must be in [1, %d], Pw + Pc=%d in [2, %d]", m, mc, kProdMax,
               p_word + p_ctx, kProdThreads);
  ASRN_REQUIRE(t >= 1 && t < cap, "asrn_decode_produce_e: position t=%lld outside [1, capacity %lld)", (long long)t,
               (long long)cap);
  ASRN_REQUIRE(e && e_prev && pieza && w_v && w_word && w_ctx && b_word && b_ctx && w2_word && b2_word && w2_ctx &&
                   b2_ctx && phi && V && sig,
               "asrn_decode_produce_e: null pointer");
  const int64_t need = asrn_decode_produce_e_workspace(L, B, m, mc);
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "asrn_decode_produce_e: workspace of %lld bytes, "
               "needs %lld", (long long)workspace_bytes, (long long)need);
  ProdBatch pb = {};
  for (int l = 0; l < L; ++l) {
    ASRN_REQUIRE(w_v[l] && w_word[l] && w_ctx[l] && b_word[l] && b_ctx[l] && w2_word[l] && b2_word[l] && w2_ctx[l] &&
                     b2_ctx[l] && phi[l] && V[l] && sig[l],
                 "asrn_decode_produce_e: layer %d: null pointer", l);
    for (const void* p : {(const void*)w_v[l], (const void*)w_word[l], (const void*)w_ctx[l]})
      ASRN_REQUIRE(((uintptr_t)p & 15) == 0, "asrn_decode_produce_e: layer %d: rows are read as float4: 16-byte "
                   "alignment", l);
    ProdArgs& a = pb.l[l];
    a.e = e; a.e_prev = e_prev; a.pieza = pieza; a.B = B; a.d = d;
    a.wv = w_v[l]; a.ww = w_word[l]; a.wc = w_ctx[l]; a.bw = b_word[l]; a.bc = b_ctx[l];
    a.w2w = w2_word[l]; a.b2w = b2_word[l]; a.w2c = w2_ctx[l]; a.b2c = b2_ctx[l];
    a.m = m; a.mc = mc; a.Pw = p_word; a.Pc = p_ctx;
    a.phi = phi[l]; a.V = V[l]; a.sig = sig[l]; a.cap = cap; a.t = t; a.t_dev = t_dev;
    a.y = (float*)workspace + (int64_t)l * B * (m + 2 * mc);
  }
  for (const void* p : {(const void*)e, (const void*)e_prev})
    ASRN_REQUIRE(((uintptr_t)p & 15) == 0, "asrn_decode_produce_e: rows are read as float4: 16-byte alignment");
  if (B == 0) return 0;
  int blocks = 0;
  for (int k = 0; k < 4; ++k) blocks += (kind_rows_host(d, m, mc, 1, k) + kProdRows - 1) / kProdRows;
  const dim3 grid((unsigned)blocks, (unsigned)((B + kProdTok - 1) / kProdTok), (unsigned)L);
  hipStream_t st = (hipStream_t)stream;
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {
    case 1: hipLaunchKernelGGL(k_produce_rows_e<1>, grid, dim3(kProdThreads), 0, st, pb); break;
    case 2: hipLaunchKernelGGL(k_produce_rows_e<2>, grid, dim3(kProdThreads), 0, st, pb); break;
    case 3: hipLaunchKernelGGL(k_produce_rows_e<3>, grid, dim3(kProdThreads), 0, st, pb); break;
    default: hipLaunchKernelGGL(k_produce_rows_e<4>, grid, dim3(kProdThreads), 0, st, pb); break;
  }
  if (check_launch("asrn_decode_produce_e/rows")) return 1;
  hipLaunchKernelGGL(k_produce_token_e, dim3((unsigned)B, (unsigned)L), dim3(kProdThreads), 0, st, pb);
  return check_launch("asrn_decode_produce_e/token");
}

namespace asrn {
namespace {

using ProduceH = void (*)(ProdArgs, Pending, const int64_t*);

template <int D4>
ProduceH produce_h_fn(bool pend, int S) {
  if (!pend) return k_produce_h<D4, 1, false>;
  return S == 4 ? k_produce_h<D4, 4, true> : (S == 8 ? k_produce_h<D4, 8, true> : k_produce_h<D4, 16, true>);
}

int produce_h(const float* h, const float* prev_h1, const float* prev_b2, const float* prev_z, float* prev_ring,
              int32_t prev_k, int32_t prev_ff, float* prev_out, const int64_t* prev_pos, void* workspace,
              int64_t workspace_bytes, int64_t B, int32_t d, const float* ln_w, const float* ln_b, float eps,
              const float* w_reloj, const float* b_reloj, float beta_max, float log_alfa_min, const float* w_cq,
              const float* w_ck, int32_t cf, float* Qc, float* Kc, float* log_alfa, int64_t cap, int64_t t,
              const int64_t* t_dev, double* beta, hipStream_t st, const char* what) {
  ASRN_REQUIRE(B >= 0 && B <= (int64_t(1) << 20) && d > 0 && d % 4 == 0 && d <= 4 * kProdMaxD4 * kWave,
               "%s: d=%d must be a positive multiple of 4, <= %d (B=%lld)", what, d, 4 * kProdMaxD4 * kWave,
               (long long)B);
  ASRN_REQUIRE(cf >= 1 && cf <= kProdMax, "%s: cf=%d must be in [1, %d]", what, cf, kProdMax);
  ASRN_REQUIRE(eps > 0.f, "%s: eps must be positive", what);
  ASRN_REQUIRE(t >= 1 && t < cap, "%s: position t=%lld outside [1, capacity %lld)", what, (long long)t,
               (long long)cap);
  ASRN_REQUIRE((h || prev_h1) && ln_w && ln_b && w_reloj && b_reloj && w_cq && w_ck && Qc && Kc && log_alfa && beta,
               "%s: null pointer", what);
  for (const void* p : {(const void*)(prev_h1 ? prev_out : h), (const void*)ln_w, (const void*)ln_b,
                        (const void*)w_reloj, (const void*)w_cq, (const void*)w_ck})
    ASRN_REQUIRE(((uintptr_t)p & 15) == 0, "%s: the rows are read as float4: 16-byte alignment", what);
  Pending pv = {};
  if (prev_h1) {
    ASRN_REQUIRE(prev_b2 && prev_z && prev_out && prev_pos && prev_k >= 1 && prev_ff >= 1 && prev_ff <= (1 << 30) &&
                     (prev_k == 1 || prev_ring),
                 "%s: a pending block needs its b2, z, out, position, k >= 1, ff >= 1 and (k > 1) its ring", what);
    const int64_t need = 4 * block_workspace_floats(B, d, prev_ff);
    ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= need,
                 "%s: the pending block's workspace of %lld bytes needed (asrn_block_step_workspace)", what,
                 (long long)need);
    // its partials, where its block step call (same workspace, same B and d) left them
    pv = Pending{block_second_parts(workspace, B, d, prev_ff), splits_for(prev_ff), prev_b2, prev_h1, prev_z,
                 prev_ring, prev_k - 1, prev_out};
  }
  if (B == 0) return 0;
  ProdArgs a = {};
  a.h = h; a.B = B; a.d = d; a.lnw = ln_w; a.lnb = ln_b; a.eps = eps; a.wr = w_reloj; a.br = b_reloj;
  a.beta_max = beta_max; a.la_min = log_alfa_min; a.wq = w_cq; a.wk = w_ck; a.cf = cf;
  a.Qc = Qc; a.Kc = Kc; a.la = log_alfa; a.cap = cap; a.t = t; a.t_dev = t_dev; a.beta = beta;
  const bool pend = prev_h1 != nullptr;
  const int S = split_cap(pv.splits);
  ProduceH fn;
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {
    case 1: fn = produce_h_fn<1>(pend, S); break;
    case 2: fn = produce_h_fn<2>(pend, S); break;
    case 3: fn = produce_h_fn<3>(pend, S); break;
    default: fn = produce_h_fn<4>(pend, S); break;
  }
  hipLaunchKernelGGL(fn, dim3((unsigned)B), dim3(kHWaves * kWave), 0, st, a, pv, prev_pos);
  return check_launch(what);
}

}  // namespace
}  // namespace asrn

extern "C" int asrn_decode_produce_h(const float* h, int64_t B, int32_t d, const float* ln_w, const float* ln_b,
                                     float eps, const float* w_reloj, const float* b_reloj, float beta_max,
                                     float log_alfa_min, const float* w_cq, const float* w_ck, int32_t cf, float* Qc,
                                     float* Kc, float* log_alfa, int64_t cap, int64_t t, const int64_t* t_dev,
                                     double* beta, void* stream) {
  ASRN_REQUIRE(h, "asrn_decode_produce_h: null pointer");
  return produce_h(h, nullptr, nullptr, nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr, 0, B, d, ln_w, ln_b, eps,
                   w_reloj, b_reloj, beta_max, log_alfa_min, w_cq, w_ck, cf, Qc, Kc, log_alfa, cap, t, t_dev, beta,
                   (hipStream_t)stream, "asrn_decode_produce_h");
}

extern "C" int asrn_decode_produce_h_ex(const float* h, const float* prev_h1, const float* prev_b2,
                                        const float* prev_z, float* prev_ring, int32_t prev_k, int32_t prev_ff,
                                        float* prev_out, const int64_t* prev_pos, void* workspace,
                                        int64_t workspace_bytes, int64_t B, int32_t d, const float* ln_w,
                                        const float* ln_b, float eps, const float* w_reloj, const float* b_reloj,
                                        float beta_max, float log_alfa_min, const float* w_cq, const float* w_ck,
                                        int32_t cf, float* Qc, float* Kc, float* log_alfa, int64_t cap, int64_t t,
                                        const int64_t* t_dev, double* beta, void* stream) {
  return produce_h(h, prev_h1, prev_b2, prev_z, prev_ring, prev_k, prev_ff, prev_out, prev_pos, workspace,
                   workspace_bytes, B, d, ln_w, ln_b, eps, w_reloj, b_reloj, beta_max, log_alfa_min, w_cq, w_ck, cf,
                   Qc, Kc, log_alfa, cap, t, t_dev, beta, (hipStream_t)stream, "asrn_decode_produce_h_ex");
}
