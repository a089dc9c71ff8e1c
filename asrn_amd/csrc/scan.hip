// a9, a11, a12: the clock, the affine scan and the Hawkes and streak scans, forward and backward.
//
// Every scan here is a prefix over a monoid: maps x -> a x + b composed in fp32 (affine, Hawkes, streak) or sums in
// fp64 (clock). A row is cut into chunks of 256 Items elements (Items consecutive per thread), one 256-thread
// workgroup per chunk, so that a few rows of a few thousand elements still spread over hundreds of CUs. Two launches and
// no workgroup ever waits for another:
//   1. k_scan_totals: each chunk but the last composes its elements into one total;
//   2. k_scan_chunks: each chunk composes the totals of the chunks before it (its carry: a wave-parallel fold in a fixed
//      order), reloads its elements, scans them across the workgroup and stores through the functor.
// A row that fits one chunk needs only the second launch. So does a row of up to 4,096 elements of the scans whose
// loads are plain (kOneLaunch: the clock and the affine scan), as one chunk of a 1,024-thread workgroup with 4
// elements a thread; the Hawkes and streak scans, whose loads are dependent gathers, measured slower that way (8 to
// 32 workgroups cannot hide them: 24 -> 32 us for each backward at cfg2) and keep their 256-element chunks. Loads
// and stores go through small functors, so the Hawkes and streak scans gather their inputs (key order, clock
// differences, exp) and scatter their outputs in the same pass.
// The backward recurrence l_i = g_i + a_{i+1} l_{i+1} is the same scan run from the right. A per-row reduction the
// functor feeds (d kappa) is summed per chunk, and a third launch adds the chunk sums in a fixed order (deterministic;
// no fences or atomics between workgroups, whose agent-scope release would write back and invalidate the L2).
#include <mutex>
#include <type_traits>

#include "common.h"

namespace asrn {

constexpr int kScanThreads = 256;
constexpr int kScanWaves = kScanThreads / kWave;

// ---- the two monoids ------------------------------------------------------------------------------------------------
struct Affine {   // x -> a x + b
  using V = float;
  float a, b;
  static __device__ __forceinline__ Affine id() { return {1.f, 0.f}; }
  __device__ __forceinline__ float value() const { return b; }   // the map applied to 0
};
// x, then y
__device__ __forceinline__ Affine cat(const Affine& x, const Affine& y) { return {x.a * y.a, y.a * x.b + y.b}; }
__device__ __forceinline__ Affine shfl_up(const Affine& x, int d) {
  return {__shfl_up(x.a, d, kWave), __shfl_up(x.b, d, kWave)};
}

struct Sum64 {
  using V = double;
  double s;
  static __device__ __forceinline__ Sum64 id() { return {0.0}; }
  __device__ __forceinline__ double value() const { return s; }
};
__device__ __forceinline__ Sum64 cat(const Sum64& x, const Sum64& y) { return {x.s + y.s}; }
__device__ __forceinline__ Sum64 shfl_up(const Sum64& x, int d) { return {__shfl_up(x.s, d, kWave)}; }

// Exclusive prefix (in thread order) of each thread's element t across a workgroup of Threads, and the workgroup's
// total.
template <class M, int Threads = kScanThreads>
__device__ __forceinline__ void block_scan(const M& t, M& excl, M& total, M* lds) {
  constexpr int kWaves = Threads / kWave;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  M inc = t;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const M u = shfl_up(inc, off);
    if (lane >= off) inc = cat(u, inc);
  }
  if (lane == kWave - 1) lds[wave] = inc;
  __syncthreads();
  M before = M::id(), all = M::id();
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const M x = lds[w];
    if (w < wave) before = cat(before, x);
    all = cat(all, x);
  }
  M prev = shfl_up(inc, 1);
  if (lane == 0) prev = M::id();
  excl = cat(before, prev);
  total = all;
}

// Composition of elements [lo, hi) of v in order, by one wave (lane-contiguous runs, then an in-order lane scan).
// Every lane of the wave calls it; the result is in lane 63.
template <class M>
__device__ __forceinline__ M wave_fold(const M* v, int64_t lo, int64_t hi) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t per = (hi - lo + kWave - 1) / kWave;
  const int64_t a = lo + lane * per, b = a + per < hi ? a + per : hi;
  M x = M::id();
  for (int64_t k = a; k < b; ++k) x = cat(x, v[k]);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const M u = shfl_up(x, off);
    if (lane >= off) x = cat(u, x);
  }
  return x;
}

// 1. totals of chunks 0 .. nc-2 of every row (grid: rows x (nc - 1))
template <class Op, int Items>
__global__ __launch_bounds__(kScanThreads) void k_scan_totals(Op op, int64_t N, int nc, typename Op::M* totals) {
  using M = typename Op::M;
  __shared__ M lds[kScanWaves];
  const int row = blockIdx.x / (nc - 1), c = blockIdx.x % (nc - 1);
  const int64_t base = ((int64_t)c * kScanThreads + threadIdx.x) * Items;
  M t = M::id();
#pragma unroll
  for (int u = 0; u < Items; ++u) {
    typename Op::Aux unused;   // what only the stores need; its loads are dead here
    if (base + u < N) t = cat(t, op.load(row, base + u, unused));
  }
  M excl, total;
  block_scan(t, excl, total, lds);
  if (threadIdx.x == 0) totals[(int64_t)row * nc + c] = total;
}

// 2. every chunk of every row (grid: rows x nc): carry from the totals before it, local scan, stores. All loads, the
// ones the stores need included (the functor's Aux), are issued before the scan's barrier. With Threads = kRowThreads
// a chunk is a whole row (nc = 1): the scan's only launch.
template <class Op, int Items, int Threads = kScanThreads>
__global__ __launch_bounds__(Threads) void k_scan_chunks(Op op, int64_t N, int nc, const typename Op::M* totals,
                                                         float* partial) {
  using M = typename Op::M;
  constexpr int kWaves = Threads / kWave;
  __shared__ M lds[kWaves];
  __shared__ M carry_s;
  __shared__ float red[kWaves];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int row = blockIdx.x / nc, c = blockIdx.x % nc;
  const int64_t base = ((int64_t)c * Threads + tid) * Items;
  M e[Items];
  typename Op::Aux aux[Items];
  M t = M::id();
#pragma unroll
  for (int u = 0; u < Items; ++u) {
    e[u] = base + u < N ? op.load(row, base + u, aux[u]) : M::id();
    t = cat(t, e[u]);
  }
  if (wave == 0) {
    const M x = c > 0 ? wave_fold(totals, (int64_t)row * nc, (int64_t)row * nc + c) : M::id();
    if (lane == kWave - 1) carry_s = x;
  }
  M excl, total;
  block_scan<M, Threads>(t, excl, total, lds);   // its barrier also publishes carry_s
  M s = cat(carry_s, excl);
  float acc = 0.f;   // per-thread accumulator for the reduction the functor feeds (d kappa)
#pragma unroll
  for (int u = 0; u < Items; ++u) {
    s = cat(s, e[u]);
    if (base + u < N) op.store(row, base + u, s.value(), acc, aux[u]);
  }
  if constexpr (Op::kReduce) {
    const float v = wave_sum(acc);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    if (tid == 0) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) sum += red[w];
      if (nc == 1) op.reduce(row, sum);
      else partial[blockIdx.x] = sum;
    }
  }
}

// 3. rows of several chunks: the chunk sums of the reduction, one wave per row (lane-strided runs, then a fixed tree)
template <class Op>
__global__ __launch_bounds__(kWave) void k_scan_rows(Op op, int nc, const float* __restrict__ partial) {
  const int row = blockIdx.x, lane = threadIdx.x;
  float s = 0.f;
  for (int k = lane; k < nc; k += kWave) s += partial[(int64_t)row * nc + k];
  s = wave_sum_u(s);
  if (lane == 0) op.reduce(row, s);
}

// Functors: load(row, e, aux) gives element e's map and fills aux with what store(row, e, value, acc, aux) needs;
// element e of a backward scan is position N - 1 - e.
struct NoAux {};

// ---- plain affine scan ----------------------------------------------------------------------------------------------
struct PlainFwd {
  static constexpr bool kReduce = false;
  static constexpr bool kOneLaunch = true;
  using M = Affine;
  using Aux = NoAux;
  const float* a; const float* b; float* S; int64_t N;
  __device__ Affine load(int row, int64_t e, Aux&) const { return {a[row * N + e], b[row * N + e]}; }
  __device__ void store(int row, int64_t e, float s, float&, const Aux&) const { S[row * N + e] = s; }
  __device__ void reduce(int, float) const {}
};

struct PlainBwd {
  static constexpr bool kReduce = false;
  static constexpr bool kOneLaunch = true;
  using M = Affine;
  struct Aux { float Sprev; };
  const float* a; const float* Sf; const float* g; float* ga; float* gb; int64_t N;
  __device__ Affine load(int row, int64_t e, Aux& x) const {
    const int64_t i = N - 1 - e;
    x.Sprev = i > 0 ? Sf[row * N + i - 1] : 0.f;
    return {i + 1 < N ? a[row * N + i + 1] : 0.f, g[row * N + i]};
  }
  __device__ void store(int row, int64_t e, float lam, float&, const Aux& x) const {
    const int64_t i = N - 1 - e;
    gb[row * N + i] = lam;
    ga[row * N + i] = i > 0 ? lam * x.Sprev : 0.f;
  }
  __device__ void reduce(int, float) const {}
};

// ---- Hawkes in key order (reference asrn/estable.py:313-318) --------------------------------------------------------
// Row (b, j) at sorted index i: dB_i = fp32(max(0, Bt[o_i] - Bt[o_{i-1}])), a_i = repeated_i exp(-kappa_j dB_i)
// (0 at i = 0), alfa_i = exp(log_alfa[o_i]).
struct HawkesCommon {
  const int32_t* order; const uint8_t* rep; const double* Bt; const float* la; const float* kappa;
  int64_t L; int n;
  __device__ __forceinline__ float step(int j, double diff, float* dB, bool* pass) const {
    *dB = (float)(diff < 0.0 ? 0.0 : diff);
    *pass = diff >= 0.0;                         // the clamp passes the gradient
    return expf(-kappa[j] * *dB);
  }
};

struct HawkesFwd : HawkesCommon {
  static constexpr bool kReduce = false;
  static constexpr bool kOneLaunch = false;
  using M = Affine;
  struct Aux { int32_t t; };
  float* hawkes; float* S_sorted;
  // (a_i, a_i alfa_{i-1})
  __device__ Affine load(int row, int64_t i, Aux& x) const {
    const int64_t bb = row / n, r0 = (int64_t)row * L;
    const int j = row % n;
    const int32_t t = order[r0 + i];
    x.t = t;
    float a = 0.f, b = 0.f;
    if (i > 0 && rep[r0 + i]) {
      const int32_t tp = order[r0 + i - 1];
      float dB;
      bool pass;
      a = step(j, Bt[bb * L + t] - Bt[bb * L + tp], &dB, &pass);
      b = a != 0.f ? a * expf(la[bb * L + tp]) : 0.f;
    }
    return {a, b};
  }
  __device__ void store(int row, int64_t i, float s, float&, const Aux& x) const {
    const int64_t bb = row / n;
    const int j = row % n;
    S_sorted[(int64_t)row * L + i] = s;
    hawkes[(bb * L + x.t) * n + j] = s;
  }
  __device__ void reduce(int, float) const {}
};

struct HawkesBwd : HawkesCommon {
  static constexpr bool kReduce = true;
  static constexpr bool kOneLaunch = false;
  using M = Affine;
  struct Aux { float a, dB, Sprev, alfa; bool pass; };
  const float* S_sorted; const float* dh; float* gdB; float* wa; float* dkappa;
  // (a_{i+1}, dhawkes at i); aux: a_i, dB_i, lambda_{i-1}, alfa_{i-1}
  __device__ Affine load(int row, int64_t e, Aux& x) const {
    const int64_t i = L - 1 - e;
    const int64_t bb = row / n, r0 = (int64_t)row * L;
    const int j = row % n;
    const int32_t t = order[r0 + i];
    const double Bi = Bt[bb * L + t];
    float an = 0.f;
    if (i + 1 < L && rep[r0 + i + 1]) {
      float dB;
      bool pass;
      an = step(j, Bt[bb * L + order[r0 + i + 1]] - Bi, &dB, &pass);
    }
    x.a = 0.f;
    x.dB = 0.f;
    x.pass = false;
    x.Sprev = 0.f;
    x.alfa = 0.f;
    if (i > 0 && rep[r0 + i]) {
      const int32_t tp = order[r0 + i - 1];
      x.a = step(j, Bi - Bt[bb * L + tp], &x.dB, &x.pass);
      x.Sprev = S_sorted[r0 + i - 1];
      x.alfa = expf(la[bb * L + tp]);
    }
    return {an, dh[(bb * L + t) * n + j]};
  }
  __device__ void store(int row, int64_t e, float lam, float& acc, const Aux& x) const {
    const int64_t i = L - 1 - e;
    const int j = row % n;
    float g = 0.f, w = 0.f;
    if (x.a != 0.f) {
      const float ga = lam * (x.Sprev + x.alfa);   // b_i = a_i alfa_{i-1}
      const float gz = ga * x.a;                   // d a / d z = a (z = -kappa dB)
      g = x.pass ? -kappa[j] * gz : 0.f;
      acc += gz * -x.dB;
      w = lam * x.a;                               // d L / d alfa_{i-1}
    }
    gdB[(int64_t)row * L + i] = g;
    wa[(int64_t)row * L + i] = w;
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
  static constexpr bool kOneLaunch = false;
  using M = Affine;
  using Aux = NoAux;
  float* racha;
  __device__ Affine load(int row, int64_t t, Aux&) const { return {a_at(row, t), r_at(row, t)}; }
  __device__ void store(int row, int64_t t, float s, float&, const Aux&) const { racha[row * L + t] = s; }
  __device__ void reduce(int, float) const {}
};

struct StreakBwd : StreakCommon {
  static constexpr bool kReduce = true;
  static constexpr bool kOneLaunch = false;
  using M = Affine;
  struct Aux { float a, rprev, beta; };
  const float* racha; const float* dr; double* dbeta; float* dkr;
  __device__ Affine load(int row, int64_t e, Aux& x) const {
    const int64_t t = L - 1 - e;
    x.a = a_at(row, t);
    x.rprev = t > 0 ? racha[row * L + t - 1] : 0.f;
    x.beta = (float)beta[row * L + t];
    return {t + 1 < L ? a_at(row, t + 1) : 0.f, dr[row * L + t]};
  }
  __device__ void store(int row, int64_t e, float lam, float& acc, const Aux& x) const {
    const int64_t t = L - 1 - e;
    const float ga = t > 0 ? lam * x.rprev : 0.f;
    const float gz = ga * x.a;
    dbeta[row * L + t] = (double)(gz * -kappa_r[0]);
    acc += gz * -x.beta;
  }
  __device__ void reduce(int row, float s) const { dkr[row] = s; }
};

// ---- clock: fp64 prefix (or suffix) sums -----------------------------------------------------------------------------
// round32: each stored prefix sum rounded to fp32 (held in fp64) while the running sum stays fp64: the unprotected
// layer's fp32 clock, which the reference gets from an fp32 cumsum that accumulates in double on the CPU
struct ClockOp {
  static constexpr bool kReduce = false;
  static constexpr bool kOneLaunch = true;
  using M = Sum64;
  using Aux = NoAux;
  const double* x; double* y; int64_t L; int reverse; int round32;
  __device__ Sum64 load(int row, int64_t e, Aux&) const { return {x[row * L + (reverse ? L - 1 - e : e)]}; }
  __device__ void store(int row, int64_t e, double v, float&, const Aux&) const {
    y[row * L + (reverse ? L - 1 - e : e)] = round32 ? (double)(float)v : v;
  }
  __device__ void reduce(int, float) const {}
};

// ---- two scans of one monoid and row length in the same launches ------------------------------------------------------
// Rows [0, ra) are A's, the rest B's (a workgroup's rows are of one kind, so the branch is uniform): the repetition
// branch's Hawkes rows (B n) and streak rows (B) share their totals, chunk and row-sum launches.
template <class A, class B>
struct Both {
  static_assert(std::is_same<typename A::M, typename B::M>::value, "the two scans must compose the same monoid");
  static constexpr bool kReduce = A::kReduce || B::kReduce;
  static constexpr bool kOneLaunch = false;
  using M = typename A::M;
  struct Aux { typename A::Aux a; typename B::Aux b; };
  A a; B b; int ra;
  __device__ M load(int row, int64_t e, Aux& x) const {
    return row < ra ? a.load(row, e, x.a) : b.load(row - ra, e, x.b);
  }
  __device__ void store(int row, int64_t e, typename M::V v, float& acc, const Aux& x) const {
    if (row < ra) a.store(row, e, v, acc, x.a);
    else b.store(row - ra, e, v, acc, x.b);
  }
  __device__ void reduce(int row, float s) const {
    if (row < ra) a.reduce(row, s);
    else b.reduce(row - ra, s);
  }
};

// ---- launch ---------------------------------------------------------------------------------------------------------
constexpr int64_t kOneChunk = (int64_t)kScanThreads * 4;   // rows up to this length take one chunk and no workspace
constexpr int kRowThreads = 1024;
constexpr int64_t kOneRow = (int64_t)kRowThreads * 4;      // longer rows up to this: one 1024-thread workgroup a row
constexpr int64_t kAlign = 256;
constexpr int64_t kScanStaticScratchBytes = int64_t(4) << 20;   // asrn_scan_fwd_static's chunk totals
constexpr int kMaxScratchDevices = 64;

static int64_t round_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Items per thread: one chunk for a short row; otherwise as many elements per thread as still leaves ~1000 chunks.
// (One 256-thread chunk per row of up to 4096, 16 per thread, measured slower than two launches over 256-element
// chunks: the per-thread chain of gathers, not the launch, is what costs.)
static int items_for(int64_t rows, int64_t N) {
  if (N <= kOneChunk) return N <= kScanThreads ? 1 : (N <= 2 * kScanThreads ? 2 : 4);
  const int64_t total = rows * N;
  return total >= 1024 * kScanThreads * 4 ? 4 : (total >= 1024 * kScanThreads * 2 ? 2 : 1);
}

template <int Items, typename Op>
static void launch_items(const Op& op, int64_t rows, int64_t N, char* ws, hipStream_t stream) {
  using M = typename Op::M;
  const int64_t nc = (N + (int64_t)kScanThreads * Items - 1) / ((int64_t)kScanThreads * Items);
  M* totals = nullptr;
  float* partial = nullptr;
  if (nc > 1) {
    totals = (M*)ws;
    partial = (float*)(ws + round_up(rows * nc * (int64_t)sizeof(M)));
    hipLaunchKernelGGL((k_scan_totals<Op, Items>), dim3((unsigned)(rows * (nc - 1))), dim3(kScanThreads), 0, stream,
                       op, N, (int)nc, totals);
  }
  hipLaunchKernelGGL((k_scan_chunks<Op, Items>), dim3((unsigned)(rows * nc)), dim3(kScanThreads), 0, stream, op, N,
                     (int)nc, (const M*)totals, partial);
  if (Op::kReduce && nc > 1)
    hipLaunchKernelGGL((k_scan_rows<Op>), dim3((unsigned)rows), dim3(kWave), 0, stream, op, (int)nc,
                       (const float*)partial);
}

// The chunk totals a scan of this op and size needs: none where it runs as one launch (a short row, or a row of up
// to kOneRow for the ops whose loads are plain), else asrn_scan_workspace's bound.
template <typename Op>
static int64_t scan_need(int64_t rows, int64_t N) {
  if (Op::kOneLaunch && N > kOneChunk && N <= kOneRow) return 0;
  return asrn_scan_workspace(rows, N);
}

template <typename Op>
static int launch_scan(const Op& op, int64_t rows, int64_t N, void* ws, int64_t wsb, void* stream, const char* what) {
  if (rows == 0 || N == 0) return 0;
  const int64_t need = scan_need<Op>(rows, N);
  ASRN_REQUIRE(need >= 0, "%s: rows x chunks must stay below 2^31", what);
  ASRN_REQUIRE(need == 0 || (ws != nullptr && wsb >= need), "%s: workspace too small (%lld bytes needed)", what,
               (long long)need);
  hipStream_t st = (hipStream_t)stream;
  if (Op::kOneLaunch && N > kOneChunk && N <= kOneRow) {   // one launch: a workgroup per row, 4 elements a thread
    hipLaunchKernelGGL((k_scan_chunks<Op, 4, kRowThreads>), dim3((unsigned)rows), dim3(kRowThreads), 0, st, op, N, 1,
                       (const typename Op::M*)nullptr, (float*)nullptr);
    return check_launch(what);
  }
  const int items = items_for(rows, N);
  if (items == 1) launch_items<1>(op, rows, N, (char*)ws, st);
  else if (items == 2) launch_items<2>(op, rows, N, (char*)ws, st);
  else launch_items<4>(op, rows, N, (char*)ws, st);
  return check_launch(what);
}

}  // namespace asrn

using namespace asrn;

extern "C" int64_t asrn_scan_workspace(int64_t rows, int64_t N) {
  if (rows <= 0 || N <= kOneChunk) return 0;
  const int64_t nc = (N + kScanThreads - 1) / kScanThreads;   // chunks at one element per thread: an upper bound
  if (rows >= (int64_t(1) << 31) / nc) return -1;
  return round_up(rows * nc * 8) + round_up(rows * nc * 4);
}

extern "C" int asrn_clock_scan(const double* x, double* y, int64_t B, int64_t L, int32_t mode, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0, "asrn_clock_scan: bad sizes");
  ASRN_REQUIRE(mode >= 0 && mode <= 2, "asrn_clock_scan: mode=%d must be 0 (prefix sums), 1 (suffix sums) or 2 "
               "(prefix sums rounded to fp32)", mode);
  ClockOp op{x, y, L, mode == 1 ? 1 : 0, mode == 2 ? 1 : 0};
  return launch_scan(op, B, L, workspace, workspace_bytes, stream, "asrn_clock_scan");
}

extern "C" int asrn_scan_fwd(const float* a, const float* b, float* S, int64_t rows, int64_t N, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(rows >= 0 && N >= 0, "asrn_scan_fwd: bad sizes");
  PlainFwd op{a, b, S, N};
  return launch_scan(op, rows, N, workspace, workspace_bytes, stream, "asrn_scan_fwd");
}

// ---- the affine scan without a caller workspace ------------------------------------------------------------------
// The chunk totals go to a file-scope device array instead of a caller's workspace; every GPU the library runs on
// holds its own copy until the process ends. On the host the array's name is only a stand-in: the device address
// comes from hipGetSymbolAddress, taken once per device with that device current, and only that address is passed
// to kernels. Every call on one GPU shares the array, so calls that overlap on one GPU (on different streams) race.
static __device__ __align__(256) char scratch[kScanStaticScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_addr[kMaxScratchDevices] = {};

static int scratch_address(void** out, const char* what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail("%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  ASRN_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "%s: device %d beyond the %d the library tracks", what, dev,
               kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev, hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return 0;
}

extern "C" int64_t asrn_scan_static_scratch_bytes(void) { return kScanStaticScratchBytes; }

extern "C" int asrn_scan_fwd_static(const float* a, const float* b, float* S, int64_t rows, int64_t N, void* stream) {
  const char* what = "asrn_scan_fwd_static";
  ASRN_REQUIRE(rows >= 0 && N >= 0, "%s: bad sizes", what);
  const int64_t need = scan_need<PlainFwd>(rows, N);    // 0 where the scan runs as one launch
  ASRN_REQUIRE(need >= 0 && need <= kScanStaticScratchBytes,
               "%s: rows=%lld, N=%lld need %lld bytes of chunk totals, beyond the library's %lld-byte static scratch "
               "(call asrn_scan_fwd with a workspace instead)", what, (long long)rows, (long long)N, (long long)need,
               (long long)kScanStaticScratchBytes);
  void* ws = nullptr;
  if (need > 0 && scratch_address(&ws, what)) return 1;
  PlainFwd op{a, b, S, N};
  return launch_scan(op, rows, N, ws, need, stream, what);
}

extern "C" int asrn_scan_bwd(const float* a, const float* S, const float* g, float* ga, float* gb, int64_t rows,
                             int64_t N, void* workspace, int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(rows >= 0 && N >= 0, "asrn_scan_bwd: bad sizes");
  PlainBwd op{a, S, g, ga, gb, N};
  return launch_scan(op, rows, N, workspace, workspace_bytes, stream, "asrn_scan_bwd");
}

extern "C" int asrn_hawkes_fwd(const int32_t* order, const uint8_t* repeated, const double* Bt, const float* log_alfa,
                               const float* kappa, int64_t B, int64_t L, int32_t n, float* hawkes, float* S_sorted,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_hawkes_fwd: bad sizes");
  HawkesFwd op;
  op.order = order; op.rep = repeated; op.Bt = Bt; op.la = log_alfa; op.kappa = kappa; op.L = L; op.n = n;
  op.hawkes = hawkes; op.S_sorted = S_sorted;
  return launch_scan(op, B * n, L, workspace, workspace_bytes, stream, "asrn_hawkes_fwd");
}

extern "C" int64_t asrn_hawkes_bwd_workspace(int64_t B, int64_t L, int32_t n) {
  const int64_t scan = asrn_scan_workspace(B * n, L);
  if (scan < 0) return -1;
  return round_up(2 * B * L * n * (int64_t)sizeof(float)) + scan;
}

extern "C" int asrn_hawkes_bwd(const int32_t* order, const uint8_t* repeated, const int32_t* rank_k, const double* Bt,
                               const float* log_alfa, const float* kappa, const float* S_sorted,
                               const float* dhawkes, int64_t B, int64_t L, int32_t n, double* dBt, float* dlog_alfa,
                               float* dkappa, void* workspace, int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_hawkes_bwd: bad sizes");
  if (B == 0 || L == 0) return 0;
  const int64_t need = asrn_hawkes_bwd_workspace(B, L, n);
  ASRN_REQUIRE(need >= 0, "asrn_hawkes_bwd: rows x chunks must stay below 2^31");
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "asrn_hawkes_bwd: workspace too small");
  float* gdB = (float*)workspace;
  float* wa = gdB + B * L * n;
  char* scan_ws = (char*)workspace + round_up(2 * B * L * n * (int64_t)sizeof(float));
  HawkesBwd op;
  op.order = order; op.rep = repeated; op.Bt = Bt; op.la = log_alfa; op.kappa = kappa; op.L = L; op.n = n;
  op.S_sorted = S_sorted; op.dh = dhawkes; op.gdB = gdB; op.wa = wa; op.dkappa = dkappa;
  if (launch_scan(op, B * n, L, scan_ws, need - (scan_ws - (char*)workspace), stream, "asrn_hawkes_bwd")) return 1;
  const int threads = 256;
  hipLaunchKernelGGL(k_hawkes_bwd_finish, dim3((unsigned)((B * L + threads - 1) / threads)), dim3(threads), 0,
                     (hipStream_t)stream, rank_k, gdB, wa, log_alfa, B, L, (int)n, dBt, dlog_alfa);
  return check_launch("asrn_hawkes_bwd/finish");
}

extern "C" int asrn_streak_fwd(const float* vistos, const double* beta, const float* kappa_r, int64_t B, int64_t L,
                               int32_t n, float* racha, void* workspace, int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_streak_fwd: bad sizes");
  StreakFwd op;
  op.vistos = vistos; op.beta = beta; op.kappa_r = kappa_r; op.L = L; op.n = n; op.racha = racha;
  return launch_scan(op, B, L, workspace, workspace_bytes, stream, "asrn_streak_fwd");
}

extern "C" int asrn_streak_bwd(const float* vistos, const double* beta, const float* kappa_r, const float* racha,
                               const float* dracha, int64_t B, int64_t L, int32_t n, double* dbeta, float* dkappa_r,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_streak_bwd: bad sizes");
  StreakBwd op;
  op.vistos = vistos; op.beta = beta; op.kappa_r = kappa_r; op.L = L; op.n = n;
  op.racha = racha; op.dr = dracha; op.dbeta = dbeta; op.dkr = dkappa_r;
  return launch_scan(op, B, L, workspace, workspace_bytes, stream, "asrn_streak_bwd");
}

// The repetition branch's two scans in shared launches: Hawkes over B n rows and the streak over B rows, both of
// length L (asrn_hawkes_fwd and asrn_streak_fwd in one pass; the same results).
extern "C" int64_t asrn_repetition_workspace(int64_t B, int64_t L, int32_t n) {
  if (B < 0 || L < 0 || n < 1) return -1;
  return asrn_scan_workspace(B * (n + 1), L);
}

extern "C" int asrn_repetition_fwd(const int32_t* order, const uint8_t* repeated, const double* Bt,
                                   const float* log_alfa, const float* kappa, const float* vistos, const double* beta,
                                   const float* kappa_r, int64_t B, int64_t L, int32_t n, float* hawkes,
                                   float* S_sorted, float* racha, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_repetition_fwd: bad sizes");
  Both<HawkesFwd, StreakFwd> op;
  op.a.order = order; op.a.rep = repeated; op.a.Bt = Bt; op.a.la = log_alfa; op.a.kappa = kappa; op.a.L = L;
  op.a.n = n; op.a.hawkes = hawkes; op.a.S_sorted = S_sorted;
  op.b.vistos = vistos; op.b.beta = beta; op.b.kappa_r = kappa_r; op.b.L = L; op.b.n = n; op.b.racha = racha;
  op.ra = (int)(B * n);
  return launch_scan(op, B * (n + 1), L, workspace, workspace_bytes, stream, "asrn_repetition_fwd");
}

extern "C" int64_t asrn_repetition_bwd_workspace(int64_t B, int64_t L, int32_t n) {
  const int64_t scan = asrn_repetition_workspace(B, L, n);
  if (scan < 0) return -1;
  return round_up(2 * B * L * n * (int64_t)sizeof(float)) + scan;
}

extern "C" int asrn_repetition_bwd(const int32_t* order, const uint8_t* repeated, const int32_t* rank_k,
                                   const double* Bt, const float* log_alfa, const float* kappa, const float* S_sorted,
                                   const float* dhawkes, const float* vistos, const double* beta,
                                   const float* kappa_r, const float* racha, const float* dracha, int64_t B,
                                   int64_t L, int32_t n, double* dBt, float* dlog_alfa, float* dkappa,
                                   double* dbeta, float* dkappa_r, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1, "asrn_repetition_bwd: bad sizes");
  if (B == 0 || L == 0) return 0;
  const int64_t need = asrn_repetition_bwd_workspace(B, L, n);
  ASRN_REQUIRE(need >= 0, "asrn_repetition_bwd: rows x chunks must stay below 2^31");
  ASRN_REQUIRE(workspace != nullptr && workspace_bytes >= need, "asrn_repetition_bwd: workspace too small");
  float* gdB = (float*)workspace;
  float* wa = gdB + B * L * n;
  char* scan_ws = (char*)workspace + round_up(2 * B * L * n * (int64_t)sizeof(float));
  Both<HawkesBwd, StreakBwd> op;
  op.a.order = order; op.a.rep = repeated; op.a.Bt = Bt; op.a.la = log_alfa; op.a.kappa = kappa; op.a.L = L;
  op.a.n = n; op.a.S_sorted = S_sorted; op.a.dh = dhawkes; op.a.gdB = gdB; op.a.wa = wa; op.a.dkappa = dkappa;
  op.b.vistos = vistos; op.b.beta = beta; op.b.kappa_r = kappa_r; op.b.L = L; op.b.n = n;
  op.b.racha = racha; op.b.dr = dracha; op.b.dbeta = dbeta; op.b.dkr = dkappa_r;
  op.ra = (int)(B * n);
  if (launch_scan(op, B * (n + 1), L, scan_ws, need - (scan_ws - (char*)workspace), stream, "asrn_repetition_bwd"))
    return 1;
  const int threads = 256;
  hipLaunchKernelGGL(k_hawkes_bwd_finish, dim3((unsigned)((B * L + threads - 1) / threads)), dim3(threads), 0,
                     (hipStream_t)stream, rank_k, gdB, wa, log_alfa, B, L, (int)n, dBt, dlog_alfa);
  return check_launch("asrn_repetition_bwd/finish");
}
