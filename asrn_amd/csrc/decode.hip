// a14: the O(1) generation step's state: per-bucket rings of recent positions and the per-n-gram Hawkes memory.
//
// Rings. Every (batch row, table) has 2^nb buckets of C slots holding positions (-1: empty) and a count per bucket.
// The r-th position to enter a bucket sits in slot r % C, so the ring keeps the C most recent and the next one
// overwrites the oldest (reference nucleo:1585-1618). The prompt's rings come from its stable bucket sort: in sorted
// order a position's place inside its bucket is its index minus the bucket's first index, found by binary search on
// the sorted ids. The step's own insert is fused into the decode attention kernel (candidates.hip).
//
// Hawkes memory. Per (batch row, n-gram length j) one open-addressing table with linear probing, keyed by the
// order-preserving code of the fp64 n-gram key (-0 and +0 are one key; NaN keys, whose group starts before the text,
// never enter). A slot holds the clock of the key's last occurrence Bu (fp64) and A = lambda + alfa there (fp32), so
//     lambda(t) = exp(-kappa_j fp32(B_t - Bu)) A,   then   A <- lambda(t) + alfa_t,  Bu <- B_t,
// the recurrence of the whole-text Hawkes scan carried per key (reference nucleo:1634-1714). A table of `cap` slots
// (a power of two) is kept at least half empty, so a probe always ends at the key or at an empty slot. The step runs
// one thread per (row, j): no two threads touch one table, and no atomics are needed; the bulk load of a prompt
// inserts distinct keys per table and claims slots with compare-and-swap.
//
// The step itself (repetition.h) rounds every multiply and add explicitly; the file is also built with
// -ffp-contract=off, so the prompt's bulk load forms its A values the same way.
#include "repetition.h"

namespace asrn {

constexpr int kThreads = 256;

__global__ void k_fill_i32(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}
__global__ void k_fill_u64(uint64_t* __restrict__ p, int64_t n, uint64_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

static unsigned fill_blocks(int64_t n) {
  const int64_t b = (n + kThreads - 1) / kThreads;
  return (unsigned)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

// ---- rings from a prompt -------------------------------------------------------------------------------------------
// thread per (row, sorted index i < n): order / ids_sorted rows of n from the stable bucket sort of positions 0..n-1
__global__ void k_ring_build(const int32_t* __restrict__ order, const int32_t* __restrict__ ids_sorted, int64_t rows,
                             int64_t n, int nb, int C, int32_t* __restrict__ rings, int32_t* __restrict__ counts) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * n) return;
  const int64_t row = e / n, i = e % n;
  const int32_t* ids = ids_sorted + row * n;
  const int id = ids[i];
  int64_t lo = 0, hi = i;                        // first index of this bucket
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ids[mid] < id) lo = mid + 1; else hi = mid;
  }
  const int64_t first = lo;
  lo = i + 1;
  hi = n;                                        // one past its last index
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ids[mid] <= id) lo = mid + 1; else hi = mid;
  }
  const int64_t place = i - first, count = lo - first;
  const int64_t bucket = row * ((int64_t)1 << nb) + id;
  if (place == 0) counts[bucket] = (int32_t)count;
  if (place >= count - C) rings[bucket * C + place % C] = order[row * n + i];
}

// ---- Hawkes tables (Table and probe: repetition.h) ------------------------------------------------------------------
// insert a key that is not in the table yet (concurrent inserts of distinct keys): returns its slot
__device__ __forceinline__ int64_t claim(const Table& tb, int64_t g, uint64_t code) {
  unsigned long long* k = reinterpret_cast<unsigned long long*>(tb.keys + g * tb.cap);
  const int64_t mask = tb.cap - 1;
  int64_t s = (int64_t)(mix64(code) & (uint64_t)mask);
  for (int64_t n = 0; n < tb.cap; ++n, s = (s + 1) & mask) {
    const unsigned long long prev = atomicCAS(k + s, (unsigned long long)kEmpty, (unsigned long long)code);
    if (prev == kEmpty || prev == code) return s;
  }
  return -1;
}

// thread per (b, j, sorted index i): the last occurrence of every non-NaN key enters the table with
// Bu = Bt[t] and A = hawkes[t, j] + exp(log_alfa[t]) (reference nucleo:1656-1681)
__global__ void k_hawkes_load(const double* __restrict__ keys, const int32_t* __restrict__ order,
                              const uint8_t* __restrict__ repeated, const float* __restrict__ hawkes,
                              const double* __restrict__ Bt, const float* __restrict__ log_alfa, int64_t B, int64_t L,
                              int n, Table tb) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * n * L) return;
  const int64_t row = e / L, i = e % L;          // row = b * n + j
  const int64_t b = row / n;
  const int j = (int)(row % n);
  const bool last = i == L - 1 || !repeated[row * L + i + 1];
  if (!last) return;
  const int64_t t = order[row * L + i];
  const double key = keys[(b * L + t) * n + j];
  if (key != key) return;
  const int64_t s = claim(tb, row, table_code(key));
  if (s < 0) return;                              // unreachable: the host keeps cap >= 2 L
  tb.Bu[row * tb.cap + s] = Bt[b * L + t];
  tb.A[row * tb.cap + s] = hawkes[(b * L + t) * n + j] + expf(log_alfa[b * L + t]);
}

// thread per old slot: re-insert into a table twice as large (or any larger power of two)
__global__ void k_hawkes_grow(Table from, Table to, int64_t groups) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= groups * from.cap) return;
  const int64_t g = e / from.cap;
  const uint64_t code = from.keys[e];
  if (code == kEmpty) return;
  const int64_t s = claim(to, g, code);
  if (s < 0) return;
  to.Bu[g * to.cap + s] = from.Bu[e];
  to.A[g * to.cap + s] = from.A[e];
}

// ---- the step: clock, n-gram keys, Hawkes, streak ------------------------------------------------------------------
// thread per (b, j)
__global__ void k_repetition_step(Step a, Table tb) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= a.B * a.n) return;
  const int64_t t = step_pos(a);
  if (t < 0 || t >= a.stride) return;                            // outside the caches: nothing written
  repetition_row(a, tb, e, t);
}

// The generation loop step's embedding rows: e_t = emb[ids] (the model's nn.Embedding on the chosen tokens,
// nucleo:1805) and e_prev = emb[text[:, pos - 1]] (the previous position's token, the context MLP's second input), so
// that the loop keeps no copy of the last step's row. Ids outside [0, V) are clamped (the sampler never makes one).
__global__ void k_embed_step(const float* __restrict__ emb, int64_t V, int d4, const int64_t* __restrict__ ids,
                             const int64_t* __restrict__ text, int64_t ld_text, const int64_t* __restrict__ pos_p,
                             int64_t B, float* __restrict__ e_t, float* __restrict__ e_prev) {
  const int64_t b = blockIdx.y;
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B || q >= d4) return;
  const int64_t p = *pos_p;
  int64_t i = ids[b], j = p >= 1 ? text[b * ld_text + p - 1] : i;
  i = i < 0 ? 0 : (i >= V ? V - 1 : i);
  j = j < 0 ? 0 : (j >= V ? V - 1 : j);
  ((float4*)e_t)[b * d4 + q] = ((const float4*)emb)[i * d4 + q];
  ((float4*)e_prev)[b * d4 + q] = ((const float4*)emb)[j * d4 + q];
}

static bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_ring_build(const int32_t* order, const int32_t* ids_sorted, int64_t B, int64_t n, int32_t T,
                               int32_t nb, int32_t C, int32_t* rings, int32_t* counts, void* stream) {
  ASRN_REQUIRE(B >= 0 && n >= 0 && n < (int64_t(1) << 31) && T >= 1 && T <= 32 && nb >= 1 && nb <= 14 && C >= 1 &&
                   C <= 64,
               "asrn_ring_build: bad sizes B=%lld n=%lld T=%d nb=%d C=%d", (long long)B, (long long)n, T, nb, C);
  hipStream_t st = (hipStream_t)stream;
  const int64_t rows = B * T, buckets = rows << nb;
  if (buckets == 0) return 0;
  hipLaunchKernelGGL(k_fill_i32, dim3(fill_blocks(buckets * C)), dim3(kThreads), 0, st, rings, buckets * C, -1);
  hipLaunchKernelGGL(k_fill_i32, dim3(fill_blocks(buckets)), dim3(kThreads), 0, st, counts, buckets, 0);
  if (check_launch("asrn_ring_build/fill")) return 1;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_ring_build, dim3((unsigned)((rows * n + kThreads - 1) / kThreads)), dim3(kThreads), 0, st,
                     order, ids_sorted, rows, n, nb, C, rings, counts);
  return check_launch("asrn_ring_build");
}

extern "C" int asrn_hawkes_table_load(const double* keys, const int32_t* order, const uint8_t* repeated,
                                      const float* hawkes, const double* Bt, const float* log_alfa, int64_t B,
                                      int64_t L, int32_t n, int64_t cap, uint64_t* tab_keys, double* tab_Bu,
                                      float* tab_A, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && n >= 1 && n <= 16, "asrn_hawkes_table_load: bad sizes B=%lld L=%lld n=%d",
               (long long)B, (long long)L, n);
  ASRN_REQUIRE(pow2(cap) && cap >= 2 * L, "asrn_hawkes_table_load: cap=%lld must be a power of two >= 2 L = %lld",
               (long long)cap, (long long)(2 * L));
  hipStream_t st = (hipStream_t)stream;
  const int64_t slots = B * n * cap;
  if (slots == 0) return 0;
  hipLaunchKernelGGL(k_fill_u64, dim3(fill_blocks(slots)), dim3(kThreads), 0, st, tab_keys, slots, kEmpty);
  if (check_launch("asrn_hawkes_table_load/fill")) return 1;
  if (L == 0) return 0;
  Table tb = {tab_keys, tab_Bu, tab_A, cap};
  hipLaunchKernelGGL(k_hawkes_load, dim3((unsigned)((B * n * L + kThreads - 1) / kThreads)), dim3(kThreads), 0, st,
                     keys, order, repeated, hawkes, Bt, log_alfa, B, L, n, tb);
  return check_launch("asrn_hawkes_table_load");
}

extern "C" int asrn_hawkes_table_grow(const uint64_t* old_keys, const double* old_Bu, const float* old_A,
                                      int64_t groups, int64_t old_cap, uint64_t* new_keys, double* new_Bu,
                                      float* new_A, int64_t new_cap, void* stream) {
  ASRN_REQUIRE(groups >= 0 && pow2(old_cap) && pow2(new_cap) && new_cap >= old_cap,
               "asrn_hawkes_table_grow: capacities %lld -> %lld must be powers of two, growing", (long long)old_cap,
               (long long)new_cap);
  hipStream_t st = (hipStream_t)stream;
  if (groups == 0) return 0;
  hipLaunchKernelGGL(k_fill_u64, dim3(fill_blocks(groups * new_cap)), dim3(kThreads), 0, st, new_keys,
                     groups * new_cap, kEmpty);
  if (check_launch("asrn_hawkes_table_grow/fill")) return 1;
  Table from = {const_cast<uint64_t*>(old_keys), const_cast<double*>(old_Bu), const_cast<float*>(old_A), old_cap};
  Table to = {new_keys, new_Bu, new_A, new_cap};
  hipLaunchKernelGGL(k_hawkes_grow, dim3((unsigned)((groups * old_cap + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     st, from, to, groups);
  return check_launch("asrn_hawkes_table_grow");
}

extern "C" int asrn_embed_step(const float* emb, int64_t V, int32_t d, const int64_t* ids, const int64_t* text,
                               int64_t ld_text, const int64_t* pos, int64_t B, float* e_t, float* e_prev,
                               void* stream) {
  ASRN_REQUIRE(V >= 1 && d >= 4 && d % 4 == 0 && B >= 0 && B <= 65535 && ld_text >= 1,
               "asrn_embed_step: bad sizes V=%lld d=%d B=%lld", (long long)V, d, (long long)B);
  ASRN_REQUIRE(emb && ids && text && pos && e_t && e_prev, "asrn_embed_step: null pointer");
  for (const void* q : {(const void*)emb, (const void*)e_t, (const void*)e_prev})
    ASRN_REQUIRE(((uintptr_t)q & 15) == 0, "asrn_embed_step: rows are copied as float4: 16-byte alignment");
  if (B == 0) return 0;
  const int d4 = d / 4;
  hipLaunchKernelGGL(k_embed_step, dim3((unsigned)((d4 + 255) / 256), (unsigned)B), dim3(256), 0,
                     (hipStream_t)stream, emb, V, d4, ids, text, ld_text, pos, B, e_t, e_prev);
  return check_launch("asrn_embed_step");
}

extern "C" int asrn_repetition_step(const float* sig, double* Bt, const float* log_alfa, const double* beta_t,
                                    const double* coef, const float* kappa, const float* kappa_r, int64_t B,
                                    int64_t stride, int64_t t, const int64_t* t_dev, int32_t n, int64_t cap,
                                    uint64_t* tab_keys,
                                    double* tab_Bu, float* tab_A, float* racha, float* vistos, float* hawkes,
                                    int32_t reloj32, void* stream) {
  ASRN_REQUIRE(B >= 0 && n >= 1 && n <= 16 && t >= 0 && t < stride,
               "asrn_repetition_step: bad sizes B=%lld n=%d t=%lld stride=%lld", (long long)B, n, (long long)t,
               (long long)stride);
  ASRN_REQUIRE(pow2(cap) && cap >= 2 * (t + 1),
               "asrn_repetition_step: table capacity %lld must be a power of two >= 2 (t + 1) = %lld: grow it first",
               (long long)cap, (long long)(2 * (t + 1)));
  if (B == 0) return 0;
  Step a = {sig, Bt, log_alfa, beta_t, coef, kappa, kappa_r, B, stride, t, n, racha, vistos, hawkes, t_dev,
            reloj32 ? 1 : 0};
  Table tb = {tab_keys, tab_Bu, tab_A, cap};
  hipLaunchKernelGGL(k_repetition_step, dim3((unsigned)((B * n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, a, tb);
  return check_launch("asrn_repetition_step");
}
