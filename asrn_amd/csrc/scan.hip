// a9, a11, a12: the clock, the affine scan and the Hawkes and streak scans, forward and backward.
//
// One workgroup of 1024 threads per row walks the row in tiles of 4096 elements (4 consecutive per thread) with a
// carry between tiles. Inside a tile the affine maps x -> a x + b are composed per thread, scanned across the wave
// with shuffles and across the 16 waves through LDS. Loads and stores go through small functors so the Hawkes and
// streak scans gather their inputs (key order, clock differences, exp) and scatter their outputs in the same pass.
// The backward recurrence l_i = g_i + a_{i+1} l_{i+1} is the same scan run from the right.
#include "common.h"

namespace asrn {

constexpr int kScanThreads = 1024;
constexpr int kItems = 4;

// (a1, b1) then (a2, b2)  ==  (a1 a2, a2 b1 + b2)
template <typename Op>
__global__ __launch_bounds__(kScanThreads) void k_affine_scan(Op op, int64_t N) {
  __shared__ float wa[16], wb[16];
  __shared__ float carry_s;
  __shared__ float red[16];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float carry = 0.f;
  float acc = 0.f;   // per-thread accumulator for an optional reduction the functor feeds (d kappa)
  for (int64_t base = 0; base < N; base += (int64_t)kScanThreads * kItems) {
    float a[kItems], b[kItems];
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      const int64_t e = base + (int64_t)tid * kItems + u;
      if (e < N) {
        op.load(row, e, a[u], b[u]);
      } else {
        a[u] = 1.f;
        b[u] = 0.f;
      }
    }
    float A = 1.f, Bv = 0.f;
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      Bv = a[u] * Bv + b[u];
      A = A * a[u];
    }
    // inclusive wave scan of the thread maps
    float Ai = A, Bi = Bv;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float au = __shfl_up(Ai, off, 64), bu = __shfl_up(Bi, off, 64);
      if (lane >= off) {
        Bi = Ai * bu + Bi;
        Ai = au * Ai;
      }
    }
    if (lane == 63) {
      wa[wave] = Ai;
      wb[wave] = Bi;
    }
    __syncthreads();
    if (wave == 0) {
      float x = lane < 16 ? wa[lane] : 1.f, y = lane < 16 ? wb[lane] : 0.f;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const float au = __shfl_up(x, off, 64), bu = __shfl_up(y, off, 64);
        if (lane >= off) {
          y = x * bu + y;
          x = au * x;
        }
      }
      // exclusive: shift by one wave
      const float xe = __shfl_up(x, 1, 64), ye = __shfl_up(y, 1, 64);
      if (lane < 16) {
        wa[lane] = lane == 0 ? 1.f : xe;
        wb[lane] = lane == 0 ? 0.f : ye;
      }
    }
    __syncthreads();
    // exclusive map of this thread = (wave prefix) then (lanes before it in the wave)
    float Al = __shfl_up(Ai, 1, 64), Bl = __shfl_up(Bi, 1, 64);
    if (lane == 0) {
      Al = 1.f;
      Bl = 0.f;
    }
    const float Aw = wa[wave], Bw = wb[wave];
    float S = Al * (Aw * carry + Bw) + Bl;
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      S = a[u] * S + b[u];
      const int64_t e = base + (int64_t)tid * kItems + u;
      if (e < N) op.store(row, e, S, acc);
    }
    if (tid == kScanThreads - 1) carry_s = S;
    __syncthreads();
    carry = carry_s;
    __syncthreads();
  }
  if (Op::kReduce) {
    float v = wave_sum(acc);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    if (tid == 0) {
      float s = 0.f;
      for (int w = 0; w < 16; ++w) s += red[w];
      op.reduce(row, s);
    }
  }
}

// ---- plain affine scan ----------------------------------------------------------------------------------------------
struct PlainFwd {
  static constexpr bool kReduce = false;
  const float* a; const float* b; float* S; int64_t N;
  __device__ void load(int row, int64_t e, float& x, float& y) const {
    x = a[row * N + e];
    y = b[row * N + e];
  }
  __device__ void store(int row, int64_t e, float s, float&) const { S[row * N + e] = s; }
  __device__ void reduce(int, float) const {}
};

struct PlainBwd {
  static constexpr bool kReduce = false;
  const float* a; const float* Sf; const float* g; float* ga; float* gb; int64_t N;
  __device__ void load(int row, int64_t e, float& x, float& y) const {
    const int64_t i = N - 1 - e;
    x = i + 1 < N ? a[row * N + i + 1] : 0.f;
    y = g[row * N + i];
  }
  __device__ void store(int row, int64_t e, float lam, float&) const {
    const int64_t i = N - 1 - e;
    gb[row * N + i] = lam;
    ga[row * N + i] = i > 0 ? lam * Sf[row * N + i - 1] : 0.f;
  }
  __device__ void reduce(int, float) const {}
};

// ---- Hawkes in key order (reference asrn/estable.py:313-318) --------------------------------------------------------
struct HawkesCommon {
  const int32_t* order; const uint8_t* rep; const double* Bt; const float* la; const float* kappa;
  int64_t L; int n;
  // a_i of row `row` at sorted index i, with its clock step dB_i and the validity of the clamp's gradient
  __device__ float a_at(int row, int64_t i, float* dB_out, bool* pass) const {
    const int64_t bb = row / n;
    const int j = row % n;
    if (i <= 0 || !rep[row * L + i]) {
      if (dB_out) *dB_out = 0.f;
      if (pass) *pass = false;
      return 0.f;
    }
    const int32_t t = order[row * L + i], tp = order[row * L + i - 1];
    const double diff = Bt[bb * L + t] - Bt[bb * L + tp];
    const float dB = (float)(diff < 0.0 ? 0.0 : diff);
    if (dB_out) *dB_out = dB;
    if (pass) *pass = diff >= 0.0;
    return expf(-kappa[j] * dB);
  }
  __device__ float alfa_at(int row, int64_t i) const {   // exp(log_alfa) of the element at sorted index i
    const int64_t bb = row / n;
    return expf(la[bb * L + order[row * L + i]]);
  }
};

struct HawkesFwd : HawkesCommon {
  static constexpr bool kReduce = false;
  float* hawkes; float* S_sorted;
  __device__ void load(int row, int64_t i, float& x, float& y) const {
    x = a_at(row, i, nullptr, nullptr);
    y = x != 0.f ? x * alfa_at(row, i - 1) : 0.f;
  }
  __device__ void store(int row, int64_t i, float s, float&) const {
    const int64_t bb = row / n;
    const int j = row % n;
    S_sorted[row * L + i] = s;
    hawkes[(bb * L + order[row * L + i]) * n + j] = s;
  }
  __device__ void reduce(int, float) const {}
};

struct HawkesBwd : HawkesCommon {
  static constexpr bool kReduce = true;
  const float* S_sorted; const float* dh; float* gdB; float* wa; float* dkappa;
  __device__ void load(int row, int64_t e, float& x, float& y) const {
    const int64_t i = L - 1 - e;
    const int64_t bb = row / n;
    const int j = row % n;
    x = i + 1 < L ? a_at(row, i + 1, nullptr, nullptr) : 0.f;
    y = dh[(bb * L + order[row * L + i]) * n + j];
  }
  __device__ void store(int row, int64_t e, float lam, float& acc) const {
    const int64_t i = L - 1 - e;
    const int j = row % n;
    float dB;
    bool pass;
    const float a = a_at(row, i, &dB, &pass);
    float g = 0.f, w = 0.f;
    if (a != 0.f) {
      const float ga = lam * (S_sorted[row * L + i - 1] + alfa_at(row, i - 1));   // b_i = a_i alfa_{i-1}
      const float gz = ga * a;                                                  // d a / d z = a (z = -kappa dB)
      g = pass ? -kappa[j] * gz : 0.f;
      acc += gz * -dB;
      w = lam * a;                                                              // d L / d alfa_{i-1}
    }
    gdB[row * L + i] = g;
    wa[row * L + i] = w;
  }
  __device__ void reduce(int row, float s) const { dkappa[row] = s; }
};

// per text position: dBt = sum_j (gdB_j[i] - gdB_j[i+1]) in fp64, dlog_alfa = alfa_t sum_j w_j[i+1]
__global__ void k_hawkes_bwd_finish(const int32_t* __restrict__ rank_k, const float* __restrict__ gdB,
                                    const float* __restrict__ wa, const float* __restrict__ la, int64_t B, int64_t L,
                                    int n, double* __restrict__ dBt, float* __restrict__ dla) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * L) return;
  const int64_t bb = e / L, t = e % L;
  double db = 0.0;
  float dw = 0.f;
  for (int j = 0; j < n; ++j) {
    const int64_t row = bb * n + j;
    const int64_t i = rank_k[row * L + t];
    const float g0 = gdB[row * L + i];
    const float g1 = i + 1 < L ? gdB[row * L + i + 1] : 0.f;
    db += (double)g0 - (double)g1;
    if (i + 1 < L) dw += wa[row * L + i + 1];
  }
  dBt[e] = db;
  dla[e] = dw * expf(la[e]);
}

// ---- streak over the text (reference asrn/estable.py:319-320) -------------------------------------------------------
struct StreakCommon {
  const float* vistos; const double* beta; const float* kappa_r; int64_t L; int n;
  __device__ float r_at(int row, int64_t t) const { return vistos[(row * L + t) * n + n - 1]; }
  __device__ float a_at(int row, int64_t t) const {
    return r_at(row, t) * expf(-kappa_r[0] * (float)beta[row * L + t]);
  }
};

struct StreakFwd : StreakCommon {
  static constexpr bool kReduce = false;
  float* racha;
  __device__ void load(int row, int64_t t, float& x, float& y) const {
    x = a_at(row, t);
    y = r_at(row, t);
  }
  __device__ void store(int row, int64_t t, float s, float&) const { racha[row * L + t] = s; }
  __device__ void reduce(int, float) const {}
};

struct StreakBwd : StreakCommon {
  static constexpr bool kReduce = true;
  const float* racha; const float* dr; double* dbeta; float* dkr;
  __device__ void load(int row, int64_t e, float& x, float& y) const {
    const int64_t t = L - 1 - e;
    x = t + 1 < L ? a_at(row, t + 1) : 0.f;
    y = dr[row * L + t];
  }
  __device__ void store(int row, int64_t e, float lam, float& acc) const {
    const int64_t t = L - 1 - e;
    const float ga = t > 0 ? lam * racha[row * L + t - 1] : 0.f;
    const float gz = ga * a_at(row, t);
    dbeta[row * L + t] = (double)(gz * -kappa_r[0]);
    acc += gz * -(float)beta[row * L + t];
  }
  __device__ void reduce(int row, float s) const { dkr[row] = s; }
};

// ---- clock: fp64 prefix (or suffix) sums -----------------------------------------------------------------------------
__global__ __launch_bounds__(kScanThreads) void k_clock(const double* __restrict__ x, double* __restrict__ y,
                                                        int64_t L, int reverse) {
  __shared__ double ws[16];
  __shared__ double carry_s;
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  double carry = 0.0;
  for (int64_t base = 0; base < L; base += (int64_t)kScanThreads * kItems) {
    double v[kItems];
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      const int64_t e = base + (int64_t)tid * kItems + u;
      const int64_t i = reverse ? L - 1 - e : e;
      v[u] = e < L ? x[row * L + i] : 0.0;
      s += v[u];
    }
    double inc = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double u = __shfl_up(inc, off, 64);
      if (lane >= off) inc += u;
    }
    if (lane == 63) ws[wave] = inc;
    __syncthreads();
    if (wave == 0) {
      const double w = lane < 16 ? ws[lane] : 0.0;
      double z = w;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const double u = __shfl_up(z, off, 64);
        if (lane >= off) z += u;
      }
      if (lane < 16) ws[lane] = z - w;
    }
    __syncthreads();
    double run = carry + ws[wave] + (inc - s);
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      const int64_t e = base + (int64_t)tid * kItems + u;
      run += v[u];
      const int64_t i = reverse ? L - 1 - e : e;
      if (e < L) y[row * L + i] = run;
    }
    if (tid == kScanThreads - 1) carry_s = run;
    __syncthreads();
    carry = carry_s;
    __syncthreads();
  }
}

template <typename Op>
static int launch_scan(const Op& op, int64_t rows, int64_t N, void* stream, const char* what) {
  if (rows == 0 || N == 0) return 0;
  ASRN_REQUIRE(rows < (int64_t(1) << 31), "%s: too many rows", what);
  hipLaunchKernelGGL(k_affine_scan<Op>, dim3((unsigned)rows), dim3(kScanThreads), 0, (hipStream_t)stream, op, N);
  return check_launch(what);
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_clock_scan(const double* x, double* y, int64_t B, int64_t L, int32_t reverse, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0, "asrn_clock_scan: bad sizes");
  if (B == 0 || L == 0) return 0;
  hipLaunchKernelGGL(k_clock, dim3((unsigned)B), dim3(kScanThreads), 0, (hipStream_t)stream, x, y, L, (int)reverse);
  return check_launch("asrn_clock_scan");
}

extern "C" int asrn_scan_fwd(const float* a, const float* b, float* S, int64_t rows, int64_t N, void* stream) {
  ASRN_REQUIRE(rows >= 0 && N >= 0, "asrn_scan_fwd: bad sizes");
  PlainFwd op{a, b, S, N};
  return launch_scan(op, rows, N, stream, "asrn_scan_fwd");
}

extern "C" int asrn_scan_bwd(const float* a, const float* S, const float* g, float* ga, float* gb, int64_t rows,
                             int64_t N, void* stream) {
  ASRN_REQUIRE(rows >= 0 && N >= 0, "asrn_scan_bwd: bad sizes");
  PlainBwd op{a, S, g, ga, gb, N};
  return launch_scan(op, rows, N, stream, "asrn_scan_bwd");
}

extern "C" int asrn_hawkes_fwd(const int32_t* order, const uint8_t* repeated, const double* Bt, const float* log_alfa,
                               const float* kappa, int64_t B, int64_t L, int32_t n, float* hawkes, float* S_sorted,
                               void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_hawkes_fwd: bad sizes");
  HawkesFwd op;
  op.order = order; op.rep = repeated; op.Bt = Bt; op.la = log_alfa; op.kappa = kappa; op.L = L; op.n = n;
  op.hawkes = hawkes; op.S_sorted = S_sorted;
  return launch_scan(op, B * n, L, stream, "asrn_hawkes_fwd");
}

extern "C" int64_t asrn_hawkes_bwd_workspace(int64_t B, int64_t L, int32_t n) {
  return 2 * B * L * n * (int64_t)sizeof(float) + 256;
}

extern "C" int asrn_hawkes_bwd(const int32_t* order, const uint8_t* repeated, const int32_t* rank_k, const double* Bt,
                               const float* log_alfa, const float* kappa, const float* S_sorted,
                               const float* dhawkes, int64_t B, int64_t L, int32_t n, double* dBt, float* dlog_alfa,
                               float* dkappa, void* workspace, int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_hawkes_bwd: bad sizes");
  if (B == 0 || L == 0) return 0;
  ASRN_REQUIRE(workspace_bytes >= asrn_hawkes_bwd_workspace(B, L, n), "asrn_hawkes_bwd: workspace too small");
  float* gdB = (float*)workspace;
  float* wa = gdB + B * L * n;
  HawkesBwd op;
  op.order = order; op.rep = repeated; op.Bt = Bt; op.la = log_alfa; op.kappa = kappa; op.L = L; op.n = n;
  op.S_sorted = S_sorted; op.dh = dhawkes; op.gdB = gdB; op.wa = wa; op.dkappa = dkappa;
  if (launch_scan(op, B * n, L, stream, "asrn_hawkes_bwd")) return 1;
  const int threads = 256;
  hipLaunchKernelGGL(k_hawkes_bwd_finish, dim3((unsigned)((B * L + threads - 1) / threads)), dim3(threads), 0,
                     (hipStream_t)stream, rank_k, gdB, wa, log_alfa, B, L, (int)n, dBt, dlog_alfa);
  return check_launch("asrn_hawkes_bwd/finish");
}

extern "C" int asrn_streak_fwd(const float* vistos, const double* beta, const float* kappa_r, int64_t B, int64_t L,
                               int32_t n, float* racha, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_streak_fwd: bad sizes");
  StreakFwd op;
  op.vistos = vistos; op.beta = beta; op.kappa_r = kappa_r; op.L = L; op.n = n; op.racha = racha;
  return launch_scan(op, B, L, stream, "asrn_streak_fwd");
}

extern "C" int asrn_streak_bwd(const float* vistos, const double* beta, const float* kappa_r, const float* racha,
                               const float* dracha, int64_t B, int64_t L, int32_t n, double* dbeta, float* dkappa_r,
                               void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_streak_bwd: bad sizes");
  StreakBwd op;
  op.vistos = vistos; op.beta = beta; op.kappa_r = kappa_r; op.L = L; op.n = n;
  op.racha = racha; op.dr = dracha; op.dbeta = dbeta; op.dkr = dkappa_r;
  return launch_scan(op, B, L, stream, "asrn_streak_bwd");
}
