// a0 (part): the hash MLPs from their first layers' products to phi (asrn/nucleo.py:644-659), fused.
//
// The first GEMM gives, per token t, y[t] = [W_p E_t | W_a E_t | W_b E_t] (bias-free). Then, per tile of 32 tokens:
//   forward   g = [gelu(hp + b_p) | gelu(za + zb[t-1] + b_c)] into LDS (exact erf GELU; no zb term at a row's first
//             position), and phi = [g_word W2w^T + b2w | g_ctx W2c^T + b2c] on the matrix cores
//             (v_mfma_f32_16x16x4_f32), the two second layers as the two diagonal blocks they are.
//   backward  dg = [dphi_word W2w | dphi_ctx W2c] on the matrix cores; the pre-activations recomputed from y; dp =
//             dg gelu'(x) written into the first GEMM's output gradient dy (the word block, the W_a block, and the
//             W_b block one position earlier, 0 at a row's last position: each element written once); and this
//             workgroup's share of every parameter gradient: dW2w = dphi_word^T g_word and dW2c = dphi_ctx^T g_ctx
//             (matrix cores again), db2 = sum dphi, and the first-layer biases' sum dp. The per-workgroup rows are
//             summed in order by asrn_column_sums.
// v_mfma_f32_16x16x4_f32 lane layout (checked on gfx950): lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]
// and receives D[(l / 16) * 4 + q][l % 16], q = 0..3.
#include "common.h"

namespace asrn {

constexpr int kPhiThreads = 256;     // 4 waves
constexpr int kPhiMax = 64;          // the most hidden units or outputs per MLP
constexpr int kGld = 2 * kPhiMax + 1;   // LDS row stride of the g / dg tiles (odd: conflict-free column reads)
constexpr int kWld = kPhiMax + 1;       // LDS row stride of a weight block or a dphi tile
static_assert(kPhiThreads == 2 * (2 * kPhiMax), "k_phi_bwd: thread tid loads dphi column tid % 128, even or odd tokens");

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct PhiArgs {
  const float* y; int64_t ldy;         // (N, ldy): hp at [0, m), za at [m, m + mc), zb at [m + mc, m + 2 mc)
  const float* bp; const float* bc;    // first-layer biases: word (m), context (mc)
  const float* Ww; const float* bw;    // word second layer (Pw, m) and its bias (Pw)
  const float* Wc; const float* bc2;   // context second layer (Pc, mc) and its bias (Pc)
  float* phi;                          // (N, Pw + Pc)
  const float* dphi;                   // (N, Pw + Pc)
  float* dy; int64_t ldd;              // (N, ldd): columns [0, m + 2 mc) written
  float* part;                         // per workgroup: [dW2w | dW2c | db2w | db2c | db_word | db_ctx]
  int64_t B, L;
  int m, mc, Pw, Pc;
  int32_t* ids; int T, nb;             // forward, optional: the bucket ids (B T, L) of the T tables of nb columns
};

__device__ __forceinline__ float gelu_e(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }
// gelu(x) and gelu'(x) from one erf: cdf = Phi(x), gelu = x cdf, gelu' = cdf + x pdf(x)
__device__ __forceinline__ void gelu_both(float x, float* g, float* gd) {
  const float cdf = 0.5f * (1.f + erff(x * 0.70710678118654752f));
  *g = x * cdf;
  *gd = cdf + x * 0.39894228040143268f * __expf(-0.5f * x * x);
}

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// a weight block (rows x cols, row-major) into LDS as ws[r][c] (stride kWld), zero beyond it up to kPhiMax x kPhiMax;
// every thread's 16 loads are issued before any is stored
template <int THREADS = kPhiThreads, int LD = kWld>
__device__ __forceinline__ void stage_block(const float* __restrict__ W, int rows, int cols, float* ws) {
  constexpr int kPer = kPhiMax * kPhiMax / THREADS;
  float v[kPer];
#pragma unroll
  for (int x = 0; x < kPer; ++x) {
    const int e = threadIdx.x + x * THREADS, r = e / kPhiMax, c = e % kPhiMax;
    const bool ok = r < rows && c < cols;
    v[x] = W[ok ? r * cols + c : 0];
    v[x] = ok ? v[x] : 0.f;
  }
#pragma unroll
  for (int x = 0; x < kPer; ++x) {
    const int e = threadIdx.x + x * THREADS;
    ws[(e / kPhiMax) * LD + e % kPhiMax] = v[x];
  }
}

// A tile's hidden-layer inputs for NG float4 groups per thread (group e = tid + x * 256: token e / h4, columns
// 4 (e % h4) ..): y at those columns (hp for word columns, za for context ones: both at y[row][j]) and the previous
// token's zb for context columns (0 at a row's first position). All loads issued together. A thread's groups all
// share one column group, whose bias the kernels load once.
template <int NG>
struct HidYN {
  float4 ya[NG], yb[NG];
};
template <int NG, int TOK, int THREADS = kPhiThreads>
__device__ __forceinline__ void load_hidden_y(const PhiArgs& a, int64_t t0, int64_t N, int h4, HidYN<NG>& in) {
#pragma unroll
  for (int x = 0; x < NG; ++x) {
    const int e = threadIdx.x + x * THREADS;
    const int tk = e / h4, j = (e - tk * h4) * 4;
    const int64_t row = t0 + tk;
    const bool ok = tk < TOK && row < N;
    const bool prev = ok && j >= a.m && row % a.L > 0;
    const int64_t r0 = ok ? row : 0;
    in.ya[x] = *reinterpret_cast<const float4*>(a.y + r0 * a.ldy + (ok ? j : 0));
    in.yb[x] = *reinterpret_cast<const float4*>(a.y + (prev ? (r0 - 1) * a.ldy + a.mc + j : 0));
    if (!prev) in.yb[x] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
}


// The forward takes tiles of kFwdTok = 64 tokens per workgroup of 8 waves and 67 KB of LDS (two per CU, so that 512
// tiles, 32,768 tokens, are one round; 32-token tiles at three per CU left a third-full second round): the tile's
// hidden inputs (4 float4 groups a thread, its column group's bias loaded once), g = gelu into LDS, then wave w forms
// the 16-token block w & 3 of MLP w >> 2 on the matrix cores (64 MFMAs, operands read 4 k-steps at a time).
constexpr int kFwdTok = 64;
constexpr int kFwdThreads = 512;
constexpr int kFwdHid = kFwdTok * 2 * kPhiMax / 4 / kFwdThreads;     // hidden float4 groups per thread: 4
// LDS row strides. A wave's 32-bit LDS reads are served 32 lanes at a time over 32 banks (measured: the conflict
// counter follows that model). The forward's matrix-core loop reads row r16 = lane % 16 at column k4 = lane / 16 of
// the g tile and of a weight block, so a stride of 2 mod 32 words puts each 32 lanes in distinct banks (the odd
// strides 129 / 65 gave 1.86 conflict cycles per LDS instruction, these 0.24; the kernel's time did not move).
#ifndef ASRN_PHI_FWD_GLD
#define ASRN_PHI_FWD_GLD 130
#endif
#ifndef ASRN_PHI_FWD_WLD
#define ASRN_PHI_FWD_WLD 66
#endif
// The backward's matrix-core loops read a weight block and the g / dg tile at row k4 = lane / 16, column r16 = lane %
// 16, so those rows take a stride of 16 mod 32 words (2.06 -> 0.27 conflict cycles per LDS instruction; 37.0 -> 36.6
// us at cfg2). The dphi tile keeps kWld: it is read both ways.
#ifndef ASRN_PHI_BWD_GLD
#define ASRN_PHI_BWD_GLD 144
#endif
#ifndef ASRN_PHI_BWD_WLD
#define ASRN_PHI_BWD_WLD 80
#endif
constexpr int kGldB = ASRN_PHI_BWD_GLD;
constexpr int kWldW = ASRN_PHI_BWD_WLD;
static_assert(kGldB >= 2 * kPhiMax && kWldW >= kPhiMax, "rows hold a tile");
constexpr int kGldF = ASRN_PHI_FWD_GLD;
constexpr int kWldF = ASRN_PHI_FWD_WLD;
static_assert(kGldF >= 2 * kPhiMax && kWldF >= kPhiMax, "rows hold a tile");

__global__ __launch_bounds__(kFwdThreads) void k_phi_fwd(PhiArgs a) {
  __shared__ __align__(16) float gs[kFwdTok * kGldF];
  __shared__ float wsw[kPhiMax * kWldF];
  __shared__ float wsc[kPhiMax * kWldF];
  __shared__ unsigned long long smask[2][kFwdTok];  // with a.ids: each token's positive columns of each MLP
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t N = a.B * a.L, t0 = (int64_t)blockIdx.x * kFwdTok;
  const int h = a.m + a.mc, h4 = h / 4, P = a.Pw + a.Pc;
  const int r16 = lane & 15, k4 = lane >> 4;
  const int tb = wave & 3, part = wave >> 2;
  const int kn = part ? a.mc : a.m, koff = part ? a.m : 0, pn = part ? a.Pc : a.Pw;
  float bias[4];                                   // the second layer's biases of this lane's output columns
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int cw = nt * 16 + r16;
    bias[nt] = cw < pn ? (part ? a.bc2 : a.bw)[cw] : 0.f;
  }
  {
    HidYN<kFwdHid> in;
    load_hidden_y<kFwdHid, kFwdTok, kFwdThreads>(a, t0, N, h4, in);
    // every hidden group of thread tid is column group tid % h4 (h4 divides 256): its first-layer bias
    const int jb = (tid % h4) * 4;
    const float4 b1 = *reinterpret_cast<const float4*>(jb >= a.m ? a.bc + (jb - a.m) : a.bp + jb);
    stage_block<kFwdThreads, kWldF>(a.Ww, a.Pw, a.m, wsw);
    stage_block<kFwdThreads, kWldF>(a.Wc, a.Pc, a.mc, wsc);
#pragma unroll
    for (int x = 0; x < kFwdHid; ++x) {
      const int e = tid + x * kFwdThreads;
      const int tk = e / h4, j = (e - tk * h4) * 4;
      if (tk >= kFwdTok) continue;
      float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
      if (t0 + tk < N) {
        const float4 v = make_float4((in.ya[x].x + b1.x) + in.yb[x].x, (in.ya[x].y + b1.y) + in.yb[x].y,
                                     (in.ya[x].z + b1.z) + in.yb[x].z, (in.ya[x].w + b1.w) + in.yb[x].w);
        g = make_float4(gelu_e(v.x), gelu_e(v.y), gelu_e(v.z), gelu_e(v.w));
      }
      float* o = gs + tk * kGldF + j;
      if constexpr (kGldF % 4 == 0) {
        *reinterpret_cast<float4*>(o) = g;
      } else {
        o[0] = g.x; o[1] = g.y; o[2] = g.z; o[3] = g.w;
      }
    }
  }
  __syncthreads();
  // phi tile of this wave: tokens 16 tb + .., the 4 n-tiles of 16 outputs of MLP `part` over its 16 k-steps (the
  // weight blocks are zero beyond Pw x m and Pc x mc, so the padding adds nothing)
  const float* ga = gs + (tb * 16 + r16) * kGldF + koff;
  const float* wsp = part ? wsc : wsw;
  floatx4 acc[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int quarter = 0; quarter < 4; ++quarter) {  // 4 k-steps at a time: their operands read, then 16 MFMAs
    float av[4], bv[4][4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int k = (quarter * 4 + ks) * 4 + k4;
      av[ks] = k < kn ? ga[k] : 0.f;                // the tile's other columns are not this MLP's
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) bv[ks][nt] = wsp[(nt * 16 + r16) * kWldF + k];
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[nt] = mfma4(av[ks], bv[ks][nt], acc[nt]);
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int cw = nt * 16 + r16;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t row = t0 + tb * 16 + k4 * 4 + q;
      if (row < N && cw < pn) a.phi[row * P + (part ? a.Pw : 0) + cw] = acc[nt][q] + bias[nt];
    }
  }
  if (a.ids) {
    // the sign hash (strict > 0, nucleo:661-664) of the values just stored, so that the bucket sort reads T ids per
    // token instead of its phi row: ballot (nt, q) holds token k4 4 + q's columns nt 16 + r16 in lanes 16 k4 + r16
    unsigned long long mine[4] = {0ull, 0ull, 0ull, 0ull};
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned long long bal = __ballot(nt * 16 + r16 < pn && acc[nt][q] + bias[nt] > 0.f);
        mine[q] |= ((bal >> (16 * k4)) & 0xFFFFull) << (16 * nt);
      }
    if (r16 == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) smask[part][tb * 16 + k4 * 4 + q] = mine[q];
    }
    __syncthreads();
    // table tau's id: bits j of columns tau nb + j of the row [word | context]; one (token, table) per thread, the
    // tokens of a table consecutive (coalesced stores)
    for (int e = tid; e < kFwdTok * a.T; e += kFwdThreads) {
      const int tk = e % kFwdTok, tau = e / kFwdTok;
      const int64_t row = t0 + tk;
      if (row >= N) continue;
      // the row's P = Pw + Pc sign bits as 128: lo holds columns 0-63, hi 64-127 (Pw <= 64)
      const unsigned long long w = smask[0][tk], c = smask[1][tk];
      const unsigned long long lo = a.Pw < 64 ? w | (c << a.Pw) : w;
      const unsigned long long hi = a.Pw == 0 ? c : (a.Pw < 64 ? c >> (64 - a.Pw) : c);
      const int c0 = tau * a.nb;
      unsigned long long bits;
      if (c0 >= 64) bits = hi >> (c0 - 64);
      else if (c0 == 0) bits = lo;
      else bits = (lo >> c0) | (hi << (64 - c0));
      const uint32_t id = (uint32_t)(bits & ((1ull << a.nb) - 1ull));
      const int64_t b = row / a.L, l = row - b * a.L;
      a.ids[(b * a.T + tau) * a.L + l] = (int32_t)id;
    }
  }
}

// The backward loops over tiles of kBwdTok = 32 tokens (blockIdx.x, + gridDim.x, ...) in workgroups of 75 KB of LDS,
// two per CU, so that one workgroup's loads, MFMA and GELU phases overlap another's: the weight blocks are staged once,
// dg turns into g in place, the tile's hidden inputs are loaded with its dphi (their latency under the dg products),
// and the parameter gradients accumulate across the workgroup's tiles (the dW MFMA accumulators stay in registers), so
// each workgroup writes one partial row.
constexpr int kBwdTok = 32;
constexpr int kBwdHid = kBwdTok * 2 * kPhiMax / 4 / kPhiThreads;     // hidden float4 groups per thread: 4
constexpr int kBwdD = kBwdTok * 2 * kPhiMax / kPhiThreads;           // dphi loads per thread: 16
static_assert(kBwdTok == 2 * 16, "k_phi_bwd: two 16-token MFMA row blocks per tile");

__global__ __launch_bounds__(kPhiThreads, 2) void k_phi_bwd(PhiArgs a) {
  __shared__ float ws[2 * kPhiMax * kWldW];        // the two weight blocks (outputs x hidden, zero-padded to 64 x 64)
  __shared__ float dps[kBwdTok * 2 * kWld];       // the dphi tile: word at [0, kWld), context at [kWld, 2 kWld)
  __shared__ float gs[kBwdTok * kGldB];            // dg, then g = gelu(x) in place, in the tile's token rows
  __shared__ float red[kPhiThreads];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, k4 = lane >> 4;
  const int64_t N = a.B * a.L, ntiles = (N + kBwdTok - 1) / kBwdTok;
  const int h = a.m + a.mc, h4 = h / 4, P = a.Pw + a.Pc;
  float* wsw = ws;
  float* wsc = ws + kPhiMax * kWldW;
  stage_block<kPhiThreads, kWldW>(a.Ww, a.Pw, a.m, wsw);
  stage_block<kPhiThreads, kWldW>(a.Wc, a.Pc, a.mc, wsc);
  floatx4 dWacc[2][4];                            // this wave's output rows 16w .. 16w + 15 of both dW2 blocks
#pragma unroll
  for (int part = 0; part < 2; ++part)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) dWacc[part][nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float4 bsum = make_float4(0.f, 0.f, 0.f, 0.f);  // first-layer biases: this thread's column group
  // every hidden group of thread tid is column group tid % h4 (h4 divides 256): its first-layer bias
  const int jb = (tid % h4) * 4;
  const float4 bias = *reinterpret_cast<const float4*>(jb >= a.m ? a.bc + (jb - a.m) : a.bp + jb);
  // second-layer biases: every dphi load of thread tid is output column tid % 128 (of [word | context]), at the
  // tile's even tokens for tid < 128 and its odd ones above, so the thread sums them as it loads them
  float b2sum = 0.f;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t t0 = tile * kBwdTok;
    HidYN<kBwdHid> in;                            // the tile's hidden inputs, in flight with its dphi
    load_hidden_y<kBwdHid, kBwdTok>(a, t0, N, h4, in);
    {
      // thread tid reads column c = tid % 128 of tokens tid / 128 + 2 x: one 32-bit offset, stepped by 2 rows
      const int c = tid & (2 * kPhiMax - 1), tk0 = tid / (2 * kPhiMax);
      const bool ctx = c >= kPhiMax;
      const int cc = ctx ? c - kPhiMax : c;
      const bool col_ok = cc < (ctx ? a.Pc : a.Pw);
      const float* src = a.dphi + t0 * P + (ctx ? a.Pw : 0) + (col_ok ? cc : 0);
      float* dst = dps + tk0 * 2 * kWld + (ctx ? kWld + cc : cc);
#pragma unroll
      for (int r = 0; r < kBwdD / 4; ++r) {
        float v[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const int tk = tk0 + 2 * (4 * r + x);
          const bool ok = col_ok && t0 + tk < N;
          v[x] = src[ok ? (uint32_t)(tk * P) : 0u];
          v[x] = ok ? v[x] : 0.f;
        }
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          dst[2 * (4 * r + x) * 2 * kWld] = v[x];
          b2sum += v[x];
        }
      }
    }
    __syncthreads();
    // dg = dphi W2 per block: wave w takes token rows 16 (w & 1) .. + 15 of block w >> 1; A = dphi tile (tokens x
    // outputs), B = the block (outputs x hidden), K = the 64 padded outputs (zero past Pw / Pc in both operands)
    {
      const int tb = wave & 1, part = wave >> 1;
      const float* da = dps + (tb * 16 + r16) * 2 * kWld + (part ? kWld : 0);
      const float* wsp = part ? wsc : wsw;
      floatx4 acc[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int quarter = 0; quarter < 4; ++quarter) {   // 4 k-steps at a time: their operands read, then 16 MFMAs
        float av[4], bv[4][4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int k = (quarter * 4 + ks) * 4 + k4;
          av[ks] = da[k];
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) bv[ks][nt] = wsp[k * kWldW + nt * 16 + r16];
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) acc[nt] = mfma4(av[ks], bv[ks][nt], acc[nt]);
      }
      const int kn = part ? a.mc : a.m, off = part ? a.m : 0;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int col = nt * 16 + r16;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (col < kn) gs[(tb * 16 + k4 * 4 + q) * kGldB + off + col] = acc[nt][q];
      }
    }
    __syncthreads();
    // the hidden layer's backward, one float4 of one token per thread: dp = dg gelu'(x) into dy; g = gelu(x) over dg
    // in LDS; each thread keeps one column group (h4 divides 256), summing dp for the first-layer biases
#pragma unroll
    for (int x = 0; x < kBwdHid; ++x) {
      const int e = tid + x * kPhiThreads;
      const int tk = e / h4, j = (e - tk * h4) * 4;
      if (tk >= kBwdTok) continue;
      const int64_t row = t0 + tk;
      float* d = gs + tk * kGldB + j;
      float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row < N) {
        const int64_t t = row % a.L;
        const float4 xv = make_float4((in.ya[x].x + bias.x) + in.yb[x].x, (in.ya[x].y + bias.y) + in.yb[x].y,
                                      (in.ya[x].z + bias.z) + in.yb[x].z, (in.ya[x].w + bias.w) + in.yb[x].w);
        float4 gd;
        gelu_both(xv.x, &g.x, &gd.x);
        gelu_both(xv.y, &g.y, &gd.y);
        gelu_both(xv.z, &g.z, &gd.z);
        gelu_both(xv.w, &g.w, &gd.w);
        const float4 dp = make_float4(d[0] * gd.x, d[1] * gd.y, d[2] * gd.z, d[3] * gd.w);
        *reinterpret_cast<float4*>(a.dy + row * a.ldd + j) = dp;
        if (j >= a.m) {
          const int c = j - a.m;
          if (t > 0) *reinterpret_cast<float4*>(a.dy + (row - 1) * a.ldd + a.m + a.mc + c) = dp;
          if (t == a.L - 1)
            *reinterpret_cast<float4*>(a.dy + row * a.ldd + a.m + a.mc + c) = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        bsum.x += dp.x; bsum.y += dp.y; bsum.z += dp.z; bsum.w += dp.w;
      }
      d[0] = g.x; d[1] = g.y; d[2] = g.z; d[3] = g.w;
    }
    __syncthreads();
    // dW2w += dphi_word^T g_word, dW2c += dphi_ctx^T g_ctx: A = dphi^T (outputs x tokens), B = g (tokens x hidden),
    // K = the tile's 32 tokens; wave w takes output rows 16w .. 16w + 15 of both blocks
    {
      const int orow = wave * 16 + r16;
#pragma unroll
      for (int quarter = 0; quarter < 2; ++quarter) {   // 4 token steps at a time: their operands read, then 32 MFMAs
        float aw[4], ac[4], bw_[4][4], bc_[4][4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int tk = (quarter * 4 + ks) * 4 + k4;
          aw[ks] = dps[tk * 2 * kWld + orow];
          ac[ks] = dps[tk * 2 * kWld + kWld + orow];
          const float* gr = gs + tk * kGldB;
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            const int col = nt * 16 + r16;
            bw_[ks][nt] = col < a.m ? gr[col] : 0.f;
            bc_[ks][nt] = col < a.mc ? gr[a.m + col] : 0.f;
          }
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            dWacc[0][nt] = mfma4(aw[ks], bw_[ks][nt], dWacc[0][nt]);
            dWacc[1][nt] = mfma4(ac[ks], bc_[ks][nt], dWacc[1][nt]);
          }
      }
    }
    __syncthreads();                              // the next tile overwrites dps and gs
  }
  float* prow = a.part + (int64_t)blockIdx.x * (a.Pw * a.m + a.Pc * a.mc + a.Pw + a.Pc + h);
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int col = nt * 16 + r16;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int o = wave * 16 + k4 * 4 + q;
      if (o < a.Pw && col < a.m) prow[o * a.m + col] = dWacc[0][nt][q];
      if (o < a.Pc && col < a.mc) prow[a.Pw * a.m + o * a.mc + col] = dWacc[1][nt][q];
    }
  }
  float* pb = prow + a.Pw * a.m + a.Pc * a.mc;
  red[tid] = b2sum;
  __syncthreads();
  if (tid < 2 * kPhiMax) {                         // even tokens' sum + odd tokens' sum
    const bool ctx = tid >= kPhiMax;
    const int c = ctx ? tid - kPhiMax : tid;
    if (c < (ctx ? a.Pc : a.Pw)) pb[(ctx ? a.Pw : 0) + c] = red[tid] + red[tid + 2 * kPhiMax];
  }
  __syncthreads();
  // first-layer biases: threads with the same column group (tid mod h4) combine in order of tid
  float* pdb = pb + a.Pw + a.Pc;
  for (int comp = 0; comp < 4; ++comp) {
    red[tid] = comp == 0 ? bsum.x : (comp == 1 ? bsum.y : (comp == 2 ? bsum.z : bsum.w));
    __syncthreads();
    if (tid < h4) {
      float s = 0.f;
      for (int r = tid; r < kPhiThreads; r += h4) s += red[r];
      pdb[tid * 4 + comp] = s;
    }
    __syncthreads();
  }
}

static int phi_check(const PhiArgs& a, const char* what) {
  ASRN_REQUIRE(a.B >= 0 && a.L >= 0 && a.m >= 4 && a.mc >= 4 && a.m <= kPhiMax && a.mc <= kPhiMax && a.m % 4 == 0 &&
                   a.mc % 4 == 0 && a.Pw >= 1 && a.Pc >= 1 && a.Pw <= kPhiMax && a.Pc <= kPhiMax,
               "%s: m=%d, mc=%d (multiples of 4 in [4, %d]) and Pw=%d, Pc=%d (in [1, %d]) out of range", what, a.m,
               a.mc, kPhiMax, a.Pw, a.Pc, kPhiMax);
  ASRN_REQUIRE(kPhiThreads % ((a.m + a.mc) / 4) == 0, "%s: (m + mc) / 4 = %d must divide %d", what,
               (a.m + a.mc) / 4, kPhiThreads);
  ASRN_REQUIRE(a.ldy >= a.m + 2 * a.mc && a.ldy % 4 == 0 && ((uintptr_t)a.y & 15) == 0 && ((uintptr_t)a.bp & 15) == 0 &&
                   ((uintptr_t)a.bc & 15) == 0,
               "%s: y needs a row stride >= m + 2 mc (a multiple of 4); y and the first-layer biases 16-byte aligned",
               what);
  return 0;
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_hash_fwd(const float* y, int64_t ldy, const float* b_word, const float* b_ctx,
                             const float* w2_word, const float* b2_word, const float* w2_ctx, const float* b2_ctx,
                             int64_t B, int64_t L, int32_t m, int32_t mc, int32_t p_word, int32_t p_ctx, float* phi,
                             int32_t* ids, int32_t T, int32_t nb, void* stream) {
  PhiArgs a = {};
  a.y = y; a.ldy = ldy; a.bp = b_word; a.bc = b_ctx; a.Ww = w2_word; a.bw = b2_word; a.Wc = w2_ctx; a.bc2 = b2_ctx;
  a.phi = phi; a.B = B; a.L = L; a.m = m; a.mc = mc; a.Pw = p_word; a.Pc = p_ctx;
  a.ids = ids; a.T = T; a.nb = nb;
  if (phi_check(a, "asrn_hash_fwd")) return 1;
  ASRN_REQUIRE(!ids || (T >= 1 && T <= 32 && nb >= 1 && nb <= 14 && T * nb == p_word + p_ctx),
               "asrn_hash_fwd: bucket ids need T in [1, 32], nb in [1, 14] and T * nb = p_word + p_ctx (T=%d nb=%d, "
               "%d columns)", T, nb, p_word + p_ctx);
  const int64_t n = B * L;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_phi_fwd, dim3((unsigned)((n + kFwdTok - 1) / kFwdTok)), dim3(kFwdThreads), 0,
                     (hipStream_t)stream, a);
  return check_launch("asrn_hash_fwd");
}

// the backward's workgroups: at most kBwdGroups (two of 75 KB LDS fit a CU), fewer for short inputs
#ifndef ASRN_PHI_BWD_GROUPS
#define ASRN_PHI_BWD_GROUPS 512
#endif
constexpr int64_t kBwdGroups = ASRN_PHI_BWD_GROUPS;
static int64_t phi_bwd_groups(int64_t n) {
  const int64_t tiles = (n + kBwdTok - 1) / kBwdTok;
  return tiles < kBwdGroups ? tiles : kBwdGroups;
}

extern "C" int64_t asrn_hash_bwd_workspace(int64_t B, int64_t L, int32_t m, int32_t mc, int32_t p_word,
                                           int32_t p_ctx) {
  if (B < 0 || L < 0 || m < 0 || mc < 0 || p_word < 0 || p_ctx < 0) return -1;
  const int64_t groups = phi_bwd_groups(B * L);
  const int64_t cols = (int64_t)p_word * m + (int64_t)p_ctx * mc + p_word + p_ctx + m + mc;
  const int64_t part = (groups * cols * 4 + 255) / 256 * 256;
  const int64_t sums = asrn_column_sums_workspace(groups, cols);
  return sums < 0 ? -1 : part + sums;
}

extern "C" int asrn_hash_bwd(const float* y, int64_t ldy, const float* b_word, const float* b_ctx,
                             const float* w2_word, const float* w2_ctx, int64_t B, int64_t L, int32_t m, int32_t mc,
                             int32_t p_word, int32_t p_ctx, const float* dphi, float* dy, int64_t ldd, float* dparams,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  PhiArgs a = {};
  a.y = y; a.ldy = ldy; a.bp = b_word; a.bc = b_ctx; a.Ww = w2_word; a.Wc = w2_ctx; a.dphi = dphi; a.dy = dy;
  a.ldd = ldd; a.B = B; a.L = L; a.m = m; a.mc = mc; a.Pw = p_word; a.Pc = p_ctx;
  if (phi_check(a, "asrn_hash_bwd")) return 1;
  ASRN_REQUIRE(ldd >= m + 2 * mc && ldd % 4 == 0 && ((uintptr_t)dy & 15) == 0,
               "asrn_hash_bwd: dy needs a row stride >= m + 2 mc (a multiple of 4) and 16-byte aligned rows");
  const int64_t need = asrn_hash_bwd_workspace(B, L, m, mc, p_word, p_ctx);
  ASRN_REQUIRE(need >= 0 && workspace_bytes >= need && (need == 0 || workspace != nullptr) &&
                   ((uintptr_t)workspace % 256) == 0,
               "asrn_hash_bwd: needs a 256-byte aligned workspace of %lld bytes", (long long)need);
  const int64_t n = B * L;
  const int64_t groups = phi_bwd_groups(n);
  const int64_t cols = (int64_t)p_word * m + (int64_t)p_ctx * mc + p_word + p_ctx + m + mc;
  if (n == 0) {   // no tokens: every gradient is 0 (column sums over no rows)
    return asrn_column_sums(nullptr, 0, 0, cols, cols, dparams, nullptr, 0, stream);
  }
  a.part = (float*)workspace;
  hipLaunchKernelGGL(k_phi_bwd, dim3((unsigned)groups), dim3(kPhiThreads), 0, (hipStream_t)stream, a);
  if (check_launch("asrn_hash_bwd")) return 1;
  const int64_t part_bytes = (groups * cols * 4 + 255) / 256 * 256;
  return asrn_column_sums(a.part, 0, groups, cols, cols, dparams, (char*)workspace + part_bytes, need - part_bytes,
                          stream);
}
