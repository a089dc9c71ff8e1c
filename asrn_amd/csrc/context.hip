// a0 (part): the context producer's LayerNorm and clock projection, fused (reference asrn/estable.py:153-194).
//
// Per token t, over the d features of h:
//   hh  = (h - mean) rstd ln_w + ln_b            (biased variance, rstd = 1 / sqrt(var + eps))
//   u_k = hh . w_reloj[k] + b_reloj[k]           (k = 0, 1; fp32, as the reference's IEEE branch)
//   beta = min(softplus(u_0), beta_max) -> fp64, log_alfa = max(logsigmoid(u_1) + log 2, log_alfa_min)
// hh feeds the Qc/Kc GEMM (hipBLASLt). Kept per token for the backward: (mean, rstd, u_0, u_1).
// Backward, from dhh (the Qc/Kc GEMM's input gradient) or from that GEMM's output gradient dy (ny <= 32 per token)
// and its weight Wq (ny, d), as dhh = dy Wq formed here on the matrix cores (v_mfma_f32_16x16x4_f32: lane l supplies
// A[l % 16][l / 16] and B[l / 16][l % 16] and receives D[(l / 16) * 4 + q][l % 16]), and from dbeta and dlog_alfa:
//   du_0 = dbeta softplus'(u_0) [softplus(u_0) <= beta_max],  du_1 = dlog_alfa sigmoid(-u_1) [not clamped below]
//   g = dhh + du_0 w_reloj[0] + du_1 w_reloj[1],  dxhat = g ln_w
//   dh = rstd (dxhat - mean(dxhat) - xhat mean(dxhat xhat)) [+ dh_add: h's gradient through the layer's other use]
//   d ln_w = sum_t g xhat, d ln_b = sum_t g, d w_reloj[k] = sum_t du_k hh, d b_reloj[k] = sum_t du_k
// Forward: a workgroup takes 8 tokens, each wave 2 of them with both rows (float4 per lane) loaded at once. Backward:
// a workgroup takes 32 tokens, each wave 8 of them, loading 2 tokens' rows at a time; the parameter gradients are
// per-workgroup partials summed in a fixed order by a second launch (deterministic, no atomics).
#include "common.h"

namespace asrn {

constexpr int kCtxThreads = 256;
constexpr int kCtxWaves = kCtxThreads / kWave;
constexpr int kCtxTok = 32;
constexpr int kCtxTokPerWave = kCtxTok / kCtxWaves;
constexpr int kCtxBatch = 2;
constexpr int kCtxFwdTok = 8;              // forward: tokens per workgroup, one round of loads per wave
constexpr int kCtxFwdPerWave = kCtxFwdTok / kCtxWaves;
constexpr int kCtxMaxD4 = 4;    // d <= 1024

struct CtxArgs {
  const float* h; const float* lnw; const float* lnb; const float* wr; const float* br;
  int64_t BL; int d; float eps; float beta_max; float la_min;
  float* hh; float4* stats; double* beta; float* la;                      // forward
  const float* dhh; const double* dbeta; const float* dla; float* dh; float* partial;   // backward
  const float* dh_add;   // backward, optional: a gradient of h from elsewhere, added to dh
  const float* dy; int64_t ldy; int ny; const float* wq;   // backward, instead of dhh: dhh = dy Wq
};

__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float logsigmoid_f(float x) { return fminf(x, 0.f) - log1pf(expf(-fabsf(x))); }

__device__ __forceinline__ float dot4(float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }

template <int D4>
__global__ __launch_bounds__(kCtxThreads) void k_ctx_fwd(CtxArgs a) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  const float inv_d = 1.f / (float)a.d;
  const int64_t tw = (int64_t)blockIdx.x * kCtxFwdTok + wave * kCtxFwdPerWave;
  for (int b = 0; b < kCtxFwdPerWave; b += kCtxBatch) {
    float4 hv[kCtxBatch][D4];
    float s[kCtxBatch];
#pragma unroll
    for (int u = 0; u < kCtxBatch; ++u) {
      const int64_t t = tw + b + u;
      s[u] = 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        hv[u][k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < a.BL && q < d4) {
          hv[u][k] = ((const float4*)(a.h + t * a.d))[q];
          s[u] += (hv[u][k].x + hv[u][k].y) + (hv[u][k].z + hv[u][k].w);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kCtxBatch; ++u) {
      const int64_t t = tw + b + u;
      if (t >= a.BL) break;
      const float mean = wave_sum_u(s[u]) * inv_d;
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (q < d4) {
          const float4 c = make_float4(hv[u][k].x - mean, hv[u][k].y - mean, hv[u][k].z - mean, hv[u][k].w - mean);
          v += dot4(c, c);
        }
      }
      const float rstd = rsqrtf(wave_sum_u(v) * inv_d + a.eps);
      float u0 = 0.f, u1 = 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (q < d4) {
          const float4 w = ((const float4*)a.lnw)[q], bb = ((const float4*)a.lnb)[q];
          const float4 y = make_float4((hv[u][k].x - mean) * rstd * w.x + bb.x, (hv[u][k].y - mean) * rstd * w.y + bb.y,
                                       (hv[u][k].z - mean) * rstd * w.z + bb.z, (hv[u][k].w - mean) * rstd * w.w + bb.w);
          ((float4*)(a.hh + t * a.d))[q] = y;
          u0 += dot4(y, ((const float4*)a.wr)[q]);
          u1 += dot4(y, ((const float4*)(a.wr + a.d))[q]);
        }
      }
      u0 = wave_sum_u(u0) + a.br[0];
      u1 = wave_sum_u(u1) + a.br[1];
      if (lane == 0) {
        a.stats[t] = make_float4(mean, rstd, u0, u1);
        float be = softplus_f(u0);
        if (a.beta_max >= 0.f) be = fminf(be, a.beta_max);
        a.beta[t] = (double)be;
        a.la[t] = fmaxf(logsigmoid_f(u1) + 0.69314718055994530942f, a.la_min);
      }
    }
  }
}

// PROJ: dhh = dy Wq for the workgroup's kCtxTok tokens, formed before the loop as a (32 x 32) by (32 x 4 D4 kWave)
// product on the matrix cores: Wq (ny <= 32 rows, zero-padded to 32 rows and 4 D4 kWave columns) and the tokens' dy
// rows staged in LDS, wave w taking the column blocks w, w + 4, ... for both 16-token blocks (K = 8 steps of 4), and
// the dhh tile written back over the stage for the token loop. The stage shares its LDS with the end's partial rows.
constexpr int kProjRows = 32;
typedef float ctx_floatx4 __attribute__((ext_vector_type(4)));
template <int D4, bool PROJ>
__global__ __launch_bounds__(kCtxThreads, (PROJ && D4 == 1) ? 4 : 1) void k_ctx_bwd(CtxArgs a) {   // PROJ, d <= 256: 4 waves per SIMD
  constexpr int kW = 4 * D4 * kWave;             // padded row width of Wq and the dhh tile
  // LDS row strides chosen so that a wave's 64 lanes fall in distinct banks: the B reads (4 rows x 16 columns), the
  // A reads (16 rows x 4 columns) and the output writes (4 rows x 16 columns, rows 4 apart)
  constexpr int kWs = kW + 16, kDs = kProjRows + 4, kTs = kW + 4;
  constexpr int kRed = kCtxWaves * (4 * 4 * D4 * kWave + 2);
  constexpr int kStage = PROJ ? kProjRows * kWs + kCtxTok * kDs : 0;
  constexpr int kTile = PROJ ? kCtxTok * kTs : 0;
  constexpr int kLds = kRed > kStage ? (kRed > kTile ? kRed : kTile) : (kStage > kTile ? kStage : kTile);
  __shared__ float lds[kLds];
  float (*red)[4 * 4 * D4 * kWave + 2] = reinterpret_cast<float (*)[4 * 4 * D4 * kWave + 2]>(lds);
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int d4 = a.d >> 2;
  const float inv_d = 1.f / (float)a.d;
  const int64_t tw = (int64_t)blockIdx.x * kCtxTok + wave * kCtxTokPerWave;
  float4 gw[D4], gb[D4], gr0[D4], gr1[D4];
#pragma unroll
  for (int k = 0; k < D4; ++k) gw[k] = gb[k] = gr0[k] = gr1[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  float gbr0 = 0.f, gbr1 = 0.f;
  if constexpr (PROJ) {
    float* wqs = lds;                              // Wq: row o at o * kWs
    float* dys = lds + kProjRows * kWs;            // dy: token row at tk * kDs
    for (int i = threadIdx.x; i < kProjRows * (kW / 4); i += kCtxThreads) {
      const int o = i / (kW / 4), q = i - o * (kW / 4);
      reinterpret_cast<float4*>(wqs + o * kWs)[q] = (o < a.ny && q < d4) ? ((const float4*)(a.wq + (int64_t)o * a.d))[q]
                                                                         : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int i = threadIdx.x; i < kCtxTok * kProjRows; i += kCtxThreads) {
      const int tk = i / kProjRows, o = i - tk * kProjRows;
      const int64_t t = (int64_t)blockIdx.x * kCtxTok + tk;
      dys[tk * kDs + o] = (t < a.BL && o < a.ny) ? a.dy[t * a.ldy + o] : 0.f;
    }
    __syncthreads();
    constexpr int kNb = kW / 16 / kCtxWaves;       // column blocks of 16 per wave
    const int r16 = lane & 15, k4 = lane >> 4;
    ctx_floatx4 acc[2][kNb];
#pragma unroll
    for (int j = 0; j < kNb; ++j) acc[0][j] = acc[1][j] = ctx_floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kProjRows / 4; ++ks) {
      const int k = ks * 4 + k4;
      const float a0 = dys[r16 * kDs + k], a1 = dys[(16 + r16) * kDs + k];
#pragma unroll
      for (int j = 0; j < kNb; ++j) {
        const float b = wqs[k * kWs + (wave + kCtxWaves * j) * 16 + r16];
        acc[0][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b, acc[1][j], 0, 0, 0);
      }
    }
    __syncthreads();                               // every wave has read the stage
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int j = 0; j < kNb; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          lds[(mb * 16 + k4 * 4 + q) * kTs + (wave + kCtxWaves * j) * 16 + r16] = acc[mb][j][q];
    __syncthreads();
  }
  constexpr int BB = kCtxBatch;                  // tokens whose rows are loaded together
  for (int b = 0; b < kCtxTokPerWave; b += BB) {
    float4 hv[BB][D4], gv[BB][D4], av[BB][D4];
    float4 st[BB];
    float db[BB], dl[BB];
#pragma unroll
    for (int u = 0; u < BB; ++u) {
      const int64_t t = tw + b + u;
      const bool ok = t < a.BL;
      st[u] = ok ? a.stats[t] : make_float4(0.f, 1.f, 0.f, 0.f);
      db[u] = ok ? (float)a.dbeta[t] : 0.f;
      dl[u] = ok ? a.dla[t] : 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (ok && q < d4) {
          hv[u][k] = ((const float4*)(a.h + t * a.d))[q];
          if constexpr (PROJ) gv[u][k] = reinterpret_cast<const float4*>(lds + (wave * kCtxTokPerWave + b + u) * kTs)[q];
          else gv[u][k] = ((const float4*)(a.dhh + t * a.d))[q];
          av[u][k] = a.dh_add ? ((const float4*)(a.dh_add + t * a.d))[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < BB; ++u) {
      const int64_t t = tw + b + u;
      if (t >= a.BL) break;
      const float mean = st[u].x, rstd = st[u].y, u0 = st[u].z, u1 = st[u].w;
      const bool pass0 = !(a.beta_max >= 0.f && softplus_f(u0) > a.beta_max);
      const bool pass1 = !(logsigmoid_f(u1) + 0.69314718055994530942f < a.la_min);
      const float sp = u0 > 20.f ? 1.f : 1.f / (1.f + expf(-u0));
      const float du0 = pass0 ? db[u] * sp : 0.f;
      const float du1 = pass1 ? dl[u] / (1.f + expf(u1)) : 0.f;
      float4 xh[D4], g[D4];
      float m1 = 0.f, m2 = 0.f;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (q < d4) {
          const float4 w = ((const float4*)a.lnw)[q];
          const float4 r0 = ((const float4*)a.wr)[q], r1 = ((const float4*)(a.wr + a.d))[q];
          xh[k] = make_float4((hv[u][k].x - mean) * rstd, (hv[u][k].y - mean) * rstd, (hv[u][k].z - mean) * rstd,
                              (hv[u][k].w - mean) * rstd);
          g[k] = make_float4(gv[u][k].x + du0 * r0.x + du1 * r1.x, gv[u][k].y + du0 * r0.y + du1 * r1.y,
                             gv[u][k].z + du0 * r0.z + du1 * r1.z, gv[u][k].w + du0 * r0.w + du1 * r1.w);
          const float4 dx = make_float4(g[k].x * w.x, g[k].y * w.y, g[k].z * w.z, g[k].w * w.w);
          m1 += (dx.x + dx.y) + (dx.z + dx.w);
          m2 += dot4(dx, xh[k]);
          // parameter partials
          const float4 bb = ((const float4*)a.lnb)[q];
          const float4 hh = make_float4(xh[k].x * w.x + bb.x, xh[k].y * w.y + bb.y, xh[k].z * w.z + bb.z,
                                        xh[k].w * w.w + bb.w);
          gw[k].x += g[k].x * xh[k].x; gw[k].y += g[k].y * xh[k].y; gw[k].z += g[k].z * xh[k].z;
          gw[k].w += g[k].w * xh[k].w;
          gb[k].x += g[k].x; gb[k].y += g[k].y; gb[k].z += g[k].z; gb[k].w += g[k].w;
          gr0[k].x += du0 * hh.x; gr0[k].y += du0 * hh.y; gr0[k].z += du0 * hh.z; gr0[k].w += du0 * hh.w;
          gr1[k].x += du1 * hh.x; gr1[k].y += du1 * hh.y; gr1[k].z += du1 * hh.z; gr1[k].w += du1 * hh.w;
        }
      }
      m1 = wave_sum_u(m1) * inv_d;
      m2 = wave_sum_u(m2) * inv_d;
#pragma unroll
      for (int k = 0; k < D4; ++k) {
        const int q = lane + kWave * k;
        if (q < d4) {
          const float4 w = ((const float4*)a.lnw)[q];
          ((float4*)(a.dh + t * a.d))[q] = make_float4(rstd * (g[k].x * w.x - m1 - xh[k].x * m2) + av[u][k].x,
                                                       rstd * (g[k].y * w.y - m1 - xh[k].y * m2) + av[u][k].y,
                                                       rstd * (g[k].z * w.z - m1 - xh[k].z * m2) + av[u][k].z,
                                                       rstd * (g[k].w * w.w - m1 - xh[k].w * m2) + av[u][k].w);
        }
      }
      gbr0 += du0;
      gbr1 += du1;
    }
  }
  // workgroup partial row: [d ln_w | d ln_b | d w_reloj[0] | d w_reloj[1] | d b_reloj (2)], the waves in order
  if constexpr (PROJ) __syncthreads();           // every wave is past the stage before the partial rows reuse it
  float* mine = red[wave];
#pragma unroll
  for (int k = 0; k < D4; ++k) {
    const int q = lane + kWave * k;
    const float4 src[4] = {gw[k], gb[k], gr0[k], gr1[k]};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      float* o = mine + m * 4 * D4 * kWave + 4 * q;
      o[0] = src[m].x;
      o[1] = src[m].y;
      o[2] = src[m].z;
      o[3] = src[m].w;
    }
  }
  if (lane == 0) {
    mine[4 * 4 * D4 * kWave] = gbr0;
    mine[4 * 4 * D4 * kWave + 1] = gbr1;
  }
  __syncthreads();
  const int cols = 4 * a.d + 2;
  float* prow = a.partial + (int64_t)blockIdx.x * cols;
  for (int c = threadIdx.x; c < cols; c += kCtxThreads) {
    const int m = c < 4 * a.d ? c / a.d : 4;
    const int src = m < 4 ? m * 4 * D4 * kWave + (c - m * a.d) : 4 * 4 * D4 * kWave + (c - 4 * a.d);
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kCtxWaves; ++w) v += red[w][src];
    prow[c] = v;
  }
}

static int64_t ctx_groups(int64_t BL) { return BL > 0 ? (BL + kCtxTok - 1) / kCtxTok : 1; }
static int64_t ctx_fwd_groups(int64_t BL) { return (BL + kCtxFwdTok - 1) / kCtxFwdTok; }

static int ctx_check(const CtxArgs& a, const char* what) {
  ASRN_REQUIRE(a.BL >= 0, "%s: bad sizes", what);
  ASRN_REQUIRE(a.d > 0 && a.d % 4 == 0 && a.d <= 4 * kCtxMaxD4 * kWave, "%s: d=%d must be a multiple of 4, <= %d",
               what, a.d, 4 * kCtxMaxD4 * kWave);
  ASRN_REQUIRE(a.eps > 0.f, "%s: eps must be positive", what);
  ASRN_REQUIRE(ctx_groups(a.BL) < (int64_t(1) << 31), "%s: too many tokens", what);
  return 0;
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_context_fwd(const float* h, const float* ln_w, const float* ln_b, const float* w_reloj,
                                const float* b_reloj, int64_t BL, int32_t d, float eps, float beta_max,
                                float log_alfa_min, float* hh, float* stats, double* beta, float* log_alfa,
                                void* stream) {
  CtxArgs a{};
  a.h = h; a.lnw = ln_w; a.lnb = ln_b; a.wr = w_reloj; a.br = b_reloj; a.BL = BL; a.d = d; a.eps = eps;
  a.beta_max = beta_max; a.la_min = log_alfa_min; a.hh = hh; a.stats = (float4*)stats; a.beta = beta; a.la = log_alfa;
  if (ctx_check(a, "asrn_context_fwd")) return 1;
  if (BL == 0) return 0;
  ASRN_REQUIRE(ctx_fwd_groups(BL) < (int64_t(1) << 31), "asrn_context_fwd: too many tokens");
  const dim3 grid((unsigned)ctx_fwd_groups(BL)), block(kCtxThreads);
  hipStream_t st = (hipStream_t)stream;
  switch ((d + 4 * kWave - 1) / (4 * kWave)) {
    case 1: hipLaunchKernelGGL(k_ctx_fwd<1>, grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL(k_ctx_fwd<2>, grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL(k_ctx_fwd<3>, grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL(k_ctx_fwd<4>, grid, block, 0, st, a); break;
  }
  return check_launch("asrn_context_fwd");
}

extern "C" int64_t asrn_context_bwd_workspace(int64_t BL, int32_t d) {
  return ctx_groups(BL) * (4 * (int64_t)d + 2) * (int64_t)sizeof(float);
}

extern "C" int asrn_context_bwd(const float* h, const float* ln_w, const float* ln_b, const float* w_reloj,
                                const float* stats, int64_t BL, int32_t d, float beta_max, float log_alfa_min,
                                const float* dhh, const float* dy, int64_t ldy, int32_t ny, const float* wq,
                                const double* dbeta, const float* dlog_alfa, const float* dh_add, float* dh,
                                float* dparams, void* workspace, int64_t workspace_bytes, void* stream) {
  CtxArgs a{};
  a.h = h; a.lnw = ln_w; a.lnb = ln_b; a.wr = w_reloj; a.BL = BL; a.d = d; a.eps = 1.f; a.beta_max = beta_max;
  a.la_min = log_alfa_min; a.stats = (float4*)stats; a.dhh = dhh; a.dbeta = dbeta; a.dla = dlog_alfa; a.dh = dh;
  a.dh_add = dh_add; a.partial = (float*)workspace;
  a.dy = dy; a.ldy = ldy; a.ny = ny; a.wq = wq;
  if (ctx_check(a, "asrn_context_bwd")) return 1;
  ASRN_REQUIRE((dhh == nullptr) != (dy == nullptr), "asrn_context_bwd: give exactly one of dhh and dy");
  ASRN_REQUIRE(dy == nullptr || (wq != nullptr && ny >= 1 && ny <= kProjRows && ldy >= ny && d <= 2 * 4 * kWave),
               "asrn_context_bwd: dy needs Wq, 1 <= ny=%d <= %d, ldy=%lld >= ny and d=%d <= %d", ny, kProjRows,
               (long long)ldy, d, 2 * 4 * kWave);
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= asrn_context_bwd_workspace(BL, d),
               "asrn_context_bwd: workspace too small");
  const int groups = (int)ctx_groups(BL);
  const int cols = 4 * d + 2;
  hipStream_t st = (hipStream_t)stream;
  const int d4c = (d + 4 * kWave - 1) / (4 * kWave);
  if (dy) {
    if (d4c == 1) hipLaunchKernelGGL((k_ctx_bwd<1, true>), dim3(groups), dim3(kCtxThreads), 0, st, a);
    else hipLaunchKernelGGL((k_ctx_bwd<2, true>), dim3(groups), dim3(kCtxThreads), 0, st, a);
  } else {
    switch (d4c) {
      case 1: hipLaunchKernelGGL((k_ctx_bwd<1, false>), dim3(groups), dim3(kCtxThreads), 0, st, a); break;
      case 2: hipLaunchKernelGGL((k_ctx_bwd<2, false>), dim3(groups), dim3(kCtxThreads), 0, st, a); break;
      case 3: hipLaunchKernelGGL((k_ctx_bwd<3, false>), dim3(groups), dim3(kCtxThreads), 0, st, a); break;
      default: hipLaunchKernelGGL((k_ctx_bwd<4, false>), dim3(groups), dim3(kCtxThreads), 0, st, a); break;
    }
  }
  if (check_launch("asrn_context_bwd")) return 1;
  return group_sums((const float*)workspace, groups, cols, dparams, st);
}
