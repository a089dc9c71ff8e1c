// Token choice for the generation loop, on the device, and the n-gram sets it consults.
//
// n-gram sets: per text row, an open-addressing table of 64-bit keys; a key packs the n token ids of an n-gram, w bits
// apiece, the oldest token in the lowest bits. w is asrn_sample_bits(V), the smallest width whose all-ones field is
// above every token id, so no key is the all-ones word that marks an empty slot. When n w > 64 (4-grams of a
// vocabulary of 65,536 or more, 5-grams of 50,304) the key is instead a 64-bit hash of the n ids (SplitMix64 steps,
// all ones mapped to all ones minus one): two distinct n-grams then share a key with probability 2^-64 per pair, about
// 2^-33 for a row of 65,536 n-grams. Inserting is then one 64-bit
// compare-and-swap that claims and publishes the key at once: concurrent inserts of one n-gram meet in one slot, and
// no thread ever waits on another. Beside it, a table of contexts (the n-gram minus its last token) holds each
// context's distinct successors, up to kSucc of them inline with a count: a successor is appended only by the insert
// that added its n-gram, so the list has no repeats, and a context whose count passes kSucc is answered by probing
// every token instead. Tables hold at most half their slots, so probes stay short, and every probe loop ends within
// `cap` steps.
//
// asrn_sample: one workgroup per text row makes the reference's whole per-token decision of escribir
// (asrn/nucleo.py:2017-2036) with no host round trip:
//   the repetition penalty over the last `window` tokens and the n-gram bans (_frenar, nucleo:1909-1918), with the
//   fallback to the plain logits when the bans leave nothing (nucleo:2020-2021); the quote mask (_Ngramas.siguientes,
//   nucleo:1877-1889); temperature, top-k and top-p (_muestrear, nucleo:1946-1962: the k-th largest logit and the
//   top-p cut are found by radix selection over the values' bits, with counts and fixed-point masses in LDS, each
//   wavefront adding once per distinct bin, instead of a sort); the softmax and the quote-mass correction
//   (_conservar_cita, nucleo:1933-1943); one draw by inverse CDF with a counter-based uniform (seed, row, position);
//   the stop token (nucleo:2026-2028); then the token is written into the text and its n-grams into the sets
//   (_Ngramas.agregar, nucleo:1872-1875).
// Every reduction runs in a fixed order: the same inputs and seed give the same token.
#include <climits>
#include <cstdint>

#include "common.h"

namespace asrn {
namespace {

constexpr unsigned long long kEmptySlot = ~0ull;
constexpr int kSampleThreads = 1024;
constexpr int kTiesPerThread = 4;         // greedy: tokens at the maximum a thread keeps
constexpr int kSampleWaves = kSampleThreads / kWave;
constexpr int kSucc = 8;                         // successors held inline per context
constexpr int kMaxCand = 4096;                   // tokens past the top-k cut handled in LDS
static_assert(kTiesPerThread * kSampleThreads <= kMaxCand, "a thread's ties are parked in the candidate list");
constexpr double kMassScale = 1099511627776.0;   // 2^40: fixed-point probability masses (sums stay below 2^63)

// SplitMix64's output function (G. Steele, D. Lea, C. Flood, "Fast splittable pseudorandom number generators",
// OOPSLA 2014): a bijective 64-bit mixer, used for slot hashes and for the counter-based uniforms.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  x ^= x >> 31;
  return x;
}

struct TupleSet {
  unsigned long long* slots;   // (rows, cap) n-gram keys; nullptr: the set is not used
  unsigned long long* ctx;     // (rows, cap) context keys
  int32_t* count;              // (rows, cap) distinct successors per context
  int32_t* succ;               // (rows, cap, kSucc) the first kSucc of them
  int64_t cap;                 // power of two
  int32_t n;                   // tokens per n-gram
};

__device__ __forceinline__ int64_t slot_of(const unsigned long long* t, int64_t cap, uint64_t key) {
  const uint64_t m = (uint64_t)cap - 1;
  uint64_t i = mix64(key) & m;
  for (int64_t p = 0; p < cap; ++p) {
    const unsigned long long v = t[i];
    if (v == key) return (int64_t)i;
    if (v == kEmptySlot) return -1;
    i = (i + 1) & m;
  }
  return -1;
}

// the slot holding `key` after the call, and whether this call put it there (-1: the table is full)
__device__ __forceinline__ int64_t slot_add(unsigned long long* t, int64_t cap, uint64_t key, bool* nuevo) {
  const uint64_t m = (uint64_t)cap - 1;
  uint64_t i = mix64(key) & m;
  for (int64_t p = 0; p < cap; ++p) {
    const unsigned long long prev = atomicCAS(t + i, kEmptySlot, (unsigned long long)key);
    if (prev == kEmptySlot || prev == key) {
      *nuevo = prev == kEmptySlot;
      return (int64_t)i;
    }
    i = (i + 1) & m;
  }
  *nuevo = false;
  return -1;
}

// the slot holding `key` (*found) or the empty slot where it goes; -1 if the table is full (plain loads: for the one
// thread that owns a row's tables)
__device__ __forceinline__ int64_t slot_find(const unsigned long long* t, int64_t cap, uint64_t key, bool* found) {
  const uint64_t m = (uint64_t)cap - 1;
  uint64_t i = mix64(key) & m;
  for (int64_t p = 0; p < cap; ++p) {
    const unsigned long long v = t[i];
    if (v == key || v == kEmptySlot) {
      *found = v == key;
      return (int64_t)i;
    }
    i = (i + 1) & m;
  }
  *found = false;
  return -1;
}

__device__ __forceinline__ bool set_has(const TupleSet& s, int64_t row, uint64_t key) {
  return slot_of(s.slots + row * s.cap, s.cap, key) >= 0;
}

// Keys of n-grams of a set with n tokens of w bits: a running state over the tokens, oldest first. Packed (n w <= 64):
// the state is the key so far, token j at bit w j. Hashed: the state is a 64-bit hash chain. key_of finishes a state
// (the context of an n-gram is its first n - 1 tokens, finished the same way for the context table).
struct KeyForm {
  int w;
  bool hashed;
  __device__ __forceinline__ uint64_t start() const { return hashed ? 0x243f6a8885a308d3ull : 0ull; }
  __device__ __forceinline__ uint64_t step(uint64_t st, int j, int64_t x) const {
    return hashed ? mix64(st ^ ((uint64_t)x + 0x9e3779b97f4a7c15ull)) : st | ((uint64_t)x << (w * j));
  }
  __device__ __forceinline__ uint64_t key_of(uint64_t st) const {
    return hashed && st == kEmptySlot ? kEmptySlot - 1 : st;
  }
};
__device__ __forceinline__ KeyForm key_form(int n, int w) { return {w, (int64_t)n * w > 64}; }

// the state after tokens x[0..n-1]
__device__ __forceinline__ uint64_t pack(const KeyForm& f, const int64_t* x, int n) {
  uint64_t k = f.start();
  for (int j = 0; j < n; ++j) k = f.step(k, j, x[j]);
  return k;
}

// the n-gram x[0..n-1] into row `row`'s set and, when new, its last token into its context's successors
__device__ __forceinline__ void ngram_add(const TupleSet& s, int64_t row, const int64_t* x, int w) {
  const KeyForm f = key_form(s.n, w);
  const uint64_t st = pack(f, x, s.n - 1);
  const uint64_t ctx = f.key_of(st);
  const uint64_t key = f.key_of(f.step(st, s.n - 1, x[s.n - 1]));
  bool nuevo;
  if (slot_add(s.slots + row * s.cap, s.cap, key, &nuevo) < 0 || !nuevo) return;
  const int64_t c = slot_add(s.ctx + row * s.cap, s.cap, ctx, &nuevo);
  if (c < 0) return;
  const int64_t e = row * s.cap + c;
  const int k = atomicAdd(s.count + e, 1);
  if (k < kSucc) s.succ[e * kSucc + k] = (int32_t)x[s.n - 1];
}

// Where the context text[pos - n + 1 .. pos - 1] sits in row b's context table: its slot (or the empty slot where it
// goes; -1 when not probed or the table is full), whether it is there, and its successor count. The step's lookup
// finds it and the step's insert of the n-gram ending at pos, whose context it is, reuses it: only the thread that
// does both touches row b's tables during the step.
struct CtxAt {
  int64_t slot = -1;
  bool found = false;
  int count = 0;
};

// ngram_add for the generation step's new n-gram x[0..n-1] (x[n-1] the token just written), by the one thread that owns
// row `row`'s tables during the step: plain loads and stores instead of atomics, and the context's place from the
// step's lookup (`at`; probed here when the lookup did not run). The tables end as ngram_add leaves them.
__device__ __forceinline__ void ngram_put(const TupleSet& s, int64_t row, const int64_t* x, int w, CtxAt at) {
  const KeyForm f = key_form(s.n, w);
  const uint64_t st = pack(f, x, s.n - 1);
  const uint64_t ctx = f.key_of(st);
  const uint64_t key = f.key_of(f.step(st, s.n - 1, x[s.n - 1]));
  unsigned long long* slots = s.slots + row * s.cap;
  bool found;
  const int64_t i = slot_find(slots, s.cap, key, &found);
  if (i < 0 || found) return;
  slots[i] = key;
  if (at.slot < 0) {
    at.slot = slot_find(s.ctx + row * s.cap, s.cap, ctx, &at.found);
    if (at.slot < 0) return;
    at.count = at.found ? s.count[row * s.cap + at.slot] : 0;
  }
  const int64_t e = row * s.cap + at.slot;
  if (!at.found) s.ctx[e] = ctx;
  s.count[e] = at.count + 1;
  if (at.count < kSucc) s.succ[e * kSucc + at.count] = (int32_t)x[s.n - 1];
}

__global__ void k_set_build(const int64_t* __restrict__ x, int64_t ldx, int64_t rows, int64_t L, TupleSet s, int w) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * L) return;
  const int64_t b = i / L, t = i - b * L;
  if (t < s.n - 1) return;
  ngram_add(s, b, x + b * ldx + t - (s.n - 1), w);
}

// ---- block reductions over the 1024 threads (fixed order: deterministic) ----------------------------------------

struct Red {
  float f[kSampleWaves];
};

__device__ __forceinline__ float block_sum(float v, Red& r) {
  v = wave_sum_u(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (lane_id() == 0) r.f[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kSampleWaves; ++i) s += r.f[i];
  return s;
}

__device__ __forceinline__ float block_max(float v, Red& r) {
  v = wave_max_u(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (lane_id() == 0) r.f[w] = v;
  __syncthreads();
  float s = r.f[0];
#pragma unroll
  for (int i = 1; i < kSampleWaves; ++i) s = fmaxf(s, r.f[i]);
  return s;
}

__device__ __forceinline__ uint32_t block_isum(uint32_t v, Red& r, unsigned int* slot) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  __syncthreads();
  if (threadIdx.x == 0) *slot = 0u;
  __syncthreads();
  if (lane_id() == 0 && v != 0u) atomicAdd(slot, v);
  __syncthreads();
  return *slot;
}

// The top-p cut's ties, as the reference's rule gives them (_muestrear: the row sorted descending, a token kept while
// the mass before it stays below top_p; ties in token order, a stable sort's): of the m tokens whose probability
// equals the boundary value tau, the first K by token index stay, K = how many j = 0, 1, ... have acc + j m_tau <
// target in the masses' fixed point (acc: the mass above tau, m_tau: tau's own mass), at least 1. Returns K, or 0 when
// all m stay.
__device__ __forceinline__ unsigned long long top_p_ties_kept(unsigned long long acc, double target, float tau,
                                                              unsigned int m) {
  const unsigned long long mt = (unsigned long long)rint((double)tau * kMassScale);
  const unsigned long long tg = (unsigned long long)target;
  if (mt == 0ull || m == 0u) return 0ull;
  const unsigned long long need = tg > acc ? tg - acc : 0ull;
  // K = ceil(need / mt) (both below 2^41: the quotient in double, then corrected to the exact ceiling)
  unsigned long long K = (unsigned long long)ceil((double)need / (double)mt);
  while (K > 0ull && (K - 1ull) * mt >= need) --K;
  while (K * mt < need) ++K;
  if (K == 0ull) K = 1ull;
  return K >= (unsigned long long)m ? 0ull : K;
}

// the largest token index among the first K tied tokens: the least v with K ties at or below it, by bisection over
// [0, V) with count_below(v) = the workgroup's count of tied tokens below index v (every thread calls this together)
template <class F>
__device__ int64_t top_p_tie_limit(unsigned long long K, int64_t V, F&& count_below) {
  if (K == 0ull) return INT64_MAX;
  int64_t lo = 0, hi = V - 1;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if ((unsigned long long)count_below(mid + 1) >= K) hi = mid; else lo = mid + 1;
  }
  return lo;
}

// this thread's count of the row's tokens below index lim whose kept probability (x / T at or above the top-k cut,
// softmax over the kept) equals tau; out of line, as only a top-p cut through tied tokens needs it
__device__ __noinline__ uint32_t ties_below(const float* row, int64_t V, int64_t lim, float tden, float corte, float m3,
                                            float S3, float tau) {
  uint32_t c = 0u;
  for (int64_t v = threadIdx.x; v < V && v < lim; v += kSampleThreads) {
    const float l = row[v] / tden;
    if (!(l < corte) && expf(l - m3) / S3 == tau) ++c;
  }
  return c;
}

// histogram adds aggregated over the wavefront: one LDS atomic per distinct bin among the valid lanes (every lane of
// the wavefront must call it together)
__device__ __forceinline__ void hist_count(unsigned int* h, uint32_t bin, bool valid) {
  uint64_t todo = __ballot(valid);
  while (todo) {
    const int leader = __ffsll((unsigned long long)todo) - 1;
    const uint32_t lb = (uint32_t)__builtin_amdgcn_readlane((int)bin, leader);
    const uint64_t same = __ballot(valid && bin == lb) & todo;
    if (lane_id() == leader) atomicAdd(h + lb, (unsigned int)__popcll(same));
    todo &= ~same;
  }
}

__device__ __forceinline__ void hist_mass(unsigned int* h, unsigned long long* hm, uint32_t bin, bool valid,
                                          unsigned long long q) {
  uint64_t todo = __ballot(valid);
  while (todo) {
    const int leader = __ffsll((unsigned long long)todo) - 1;
    const uint32_t lb = (uint32_t)__builtin_amdgcn_readlane((int)bin, leader);
    const uint64_t same = __ballot(valid && bin == lb) & todo;
    unsigned long long part = ((same >> lane_id()) & 1ull) ? q : 0ull;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
    if (lane_id() == leader) {
      atomicAdd(h + lb, (unsigned int)__popcll(same));
      atomicAdd(hm + lb, part);
    }
    todo &= ~same;
  }
}

// float -> unsigned key with the same order (NaN above +inf)
__device__ __forceinline__ uint32_t ordered(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_ordered(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct SampleArgs {
  const float* lg;
  int64_t ldl;
  float* work;                 // (B, V): the logits after penalty and bans
  uint32_t* quote_bits;        // (B, ceil(V / 32)), used when a context has more than kSucc successors
  float* prob_out;             // (B, V) or nullptr: the final probabilities
  float* logits_out;           // (B, steps, V) or nullptr: the logits as they came, at step pos - L0
  int64_t steps;
  int64_t* text;
  int64_t ld_text;
  const int64_t* pos_dev;
  int64_t pos_max;
  int64_t L0;
  int64_t* tokens;
  uint8_t* done;
  int32_t* stop_step;
  TupleSet quote, ban;
  int32_t w;
  int64_t V;
  float temperature, top_p, penalty;
  int32_t top_k, window;
  int64_t stop_token;
  uint64_t seed;
  int32_t greedy_parts;        // k_greedy_part ran before: its slices' results are in each row's `work`
};

// The greedy pre-pass (a greedy row with no penalty, no recorded logits and no probabilities out): kGreedySlices
// workgroups per row, each over a contiguous slice of V / kGreedySlices logits, find the maximum of x / T there, how
// many tokens reach it, the smallest of them and whether any x / T is NaN, so that the row's one workgroup in k_sample
// combines kGreedySlices results instead of reading the row: one CU per row makes that pass VALU-bound (about 60
// instructions a token, 50,304 tokens). A row with one finite maximum then takes it (its probability is 1, whatever
// the top-p cut and the quote correction); ties, NaN or an all -inf row run the full pass as before.
constexpr int kGreedySlices = 16;
constexpr int kGreedyThreads = 256;

// The successors of the context text[pos - n + 1 .. pos - 1] in row b's set: *n_list < 0 when the context has more
// than kSucc of them (then the caller probes every token); list[0 .. *n_list) otherwise. One thread calls it.
__device__ __forceinline__ void successors(const TupleSet& s, int64_t b, const int64_t* text, int64_t pos, int w,
                                           int* list, int* n_list, CtxAt* at) {
  const KeyForm f = key_form(s.n, w);
  const uint64_t ctx = f.key_of(pack(f, text + pos - (s.n - 1), s.n - 1));
  bool found;
  const int64_t c = slot_find(s.ctx + b * s.cap, s.cap, ctx, &found);
  at->slot = c;
  at->found = found;
  at->count = 0;
  if (c < 0 || !found) {
    *n_list = 0;
    return;
  }
  const int64_t e = b * s.cap + c;
  const int k = s.count[e];
  at->count = k;
  if (k > kSucc) {
    *n_list = -1;
    return;
  }
  for (int i = 0; i < k; ++i) list[i] = s.succ[e * kSucc + i];
  *n_list = k;
}

// f(v, x) for this thread's strided share of a row (v = tid + k * 1024, x = row[v]), eight loads in flight
template <class F>
__device__ __forceinline__ void each(const float* row, int64_t V, F&& f) {
  for (int64_t base = threadIdx.x; base < V; base += 8 * (int64_t)kSampleThreads) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t v = base + (int64_t)j * kSampleThreads;
      t[j] = v < V ? row[v] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t v = base + (int64_t)j * kSampleThreads;
      if (v < V) f(v, t[j]);
    }
  }
}

// the same with every lane of the wavefront calling f(v, x, valid) the same number of times (for passes that use
// wavefront-wide operations)
template <class F>
__device__ __forceinline__ void each_all(const float* row, int64_t V, F&& f) {
  for (int64_t base = 0; base < V; base += 8 * (int64_t)kSampleThreads) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t v = base + (int64_t)j * kSampleThreads + threadIdx.x;
      t[j] = v < V ? row[v] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t v = base + (int64_t)j * kSampleThreads + threadIdx.x;
      f(v, t[j], v < V);
    }
  }
}

// f(v, x) over the contiguous range [v0, v1) of a row, in order, eight loads in flight; f returns false to stop
template <class F>
__device__ __forceinline__ void each_range(const float* row, int64_t v0, int64_t v1, F&& f) {
  for (int64_t vb = v0; vb < v1; vb += 8) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = vb + j < v1 ? row[vb + j] : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (vb + j < v1 && !f(vb + j, t[j])) return;
  }
}

__global__ __launch_bounds__(kGreedyThreads) void k_greedy_part(SampleArgs a) {
  __shared__ float wl[kGreedyThreads / kWave];
  __shared__ int wc[kGreedyThreads / kWave], wf[kGreedyThreads / kWave], wn[kGreedyThreads / kWave];
  const int64_t b = blockIdx.x;                                 // row b, slice blockIdx.y
  const int64_t pos = *a.pos_dev;
  if (pos < 0 || pos > a.pos_max) return;                       // as k_sample: nothing is touched
  const int64_t V = a.V;
  const int64_t per = (V + kGreedySlices - 1) / kGreedySlices;
  const int64_t v0 = (int64_t)blockIdx.y * per, v1 = v0 + per < V ? v0 + per : V;
  const float* lg = a.lg + b * a.ldl;
  const float tden = fmaxf(a.temperature, 1e-6f);
  float lmax = -INFINITY;
  int cnt = 0, first = INT_MAX, nan = 0;
  for (int64_t base = v0 + threadIdx.x; base < v1; base += 4 * kGreedyThreads) {
    float t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t v = base + j * kGreedyThreads;
      t[j] = v < v1 ? lg[v] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {                               // this thread's tokens in increasing order
      const int64_t v = base + j * kGreedyThreads;
      if (v >= v1) continue;
      const float l = t[j] / tden;
      nan |= l != l;
      if (l > lmax) {
        lmax = l;
        cnt = 0;
        first = (int)v;
      }
      if (l == lmax) ++cnt;
    }
  }
  const float L = wave_max_u(lmax);
  int c = lmax == L ? cnt : 0, f = lmax == L ? first : INT_MAX;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    c += __shfl_xor(c, m, 64);
    f = min(f, __shfl_xor(f, m, 64));
    nan |= __shfl_xor(nan, m, 64);
  }
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0) {
    wl[w] = L;
    wc[w] = c;
    wf[w] = f;
    wn[w] = nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float Lb = wl[0];
    for (int i = 1; i < kGreedyThreads / kWave; ++i) Lb = fmaxf(Lb, wl[i]);
    int C = 0, F = INT_MAX, N = 0;
    for (int i = 0; i < kGreedyThreads / kWave; ++i) {
      if (wl[i] == Lb) {
        C += wc[i];
        F = min(F, wf[i]);
      }
      N |= wn[i];
    }
    float* out = a.work + b * V + 4 * (int64_t)blockIdx.y;
    out[0] = Lb;
    reinterpret_cast<int*>(out)[1] = C;
    reinterpret_cast<int*>(out)[2] = F;
    reinterpret_cast<int*>(out)[3] = N;
  }
}

__global__ __launch_bounds__(kSampleThreads) void k_sample(SampleArgs a) {
  __shared__ Red red;
  __shared__ unsigned int hist_n[256];
  __shared__ unsigned long long hist_m[256];
  __shared__ uint32_t sel[2];          // radix results: [0] digit, [1] rank left / found
  __shared__ float scan[kSampleThreads];
  __shared__ int pick[2];
  __shared__ int qlist[kSucc], blist[kSucc];
  __shared__ int nq_list, nb_list;
  __shared__ int ctok[kMaxCand];
  __shared__ float cval[kMaxCand];
  __shared__ int cscan[kSampleThreads];
  __shared__ unsigned long long tie_acc;
  __shared__ unsigned int tie_cnt;
  int64_t tie_max = INT64_MAX;                // top-p: the largest token index kept at the boundary probability
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t pos = *a.pos_dev;
  if (pos < 0 || pos > a.pos_max) return;                       // outside the text buffer: nothing is touched
  const int64_t V = a.V;
  const float* lg = a.lg + b * a.ldl;
  float* work = a.work + b * V;
  int64_t* text = a.text + b * a.ld_text;
  const int64_t step = pos - a.L0;
  const float ninf = -INFINITY;
  const int nq = a.quote.n, nb = a.ban.n;
  const bool quote = a.quote.slots && pos >= nq;
  const bool bans = a.ban.slots && pos - a.L0 >= nb;
  CtxAt qat, bat;                                               // thread 0's: reused by the insert at the end
  if (tid == 0) {
    nq_list = nb_list = 0;
    if (quote) successors(a.quote, b, text, pos, a.w, qlist, &nq_list, &qat);
    if (bans) successors(a.ban, b, text, pos, a.w, blist, &nb_list, &bat);
  }

  // Greedy rows (top_k = 1) take the maximum and its ties in one fused pass below. With no penalty and no bans the
  // row needs no changes, so that pass reads the logits themselves and `work` is never written.
  const bool greedy = a.top_k == 1 && V > 1;
  const bool direct = greedy && a.penalty == 1.f && !bans;
  const float* src = direct ? lg : work;
  // the greedy pre-pass's slices (in `work`, which a direct row does not otherwise use): one finite maximum is taken
  // as the row's one kept token, with no pass over the row here
  bool fast = false;
  if (direct && a.greedy_parts) {
    if (tid == 0) {
      const float* p = work;
      const int* ip = reinterpret_cast<const int*>(work);
      float L = p[0];
      for (int i = 1; i < kGreedySlices; ++i) L = fmaxf(L, p[4 * i]);
      int C = 0, F = INT_MAX, N = 0;
      for (int i = 0; i < kGreedySlices; ++i) {
        if (p[4 * i] == L) {
          C += ip[4 * i + 1];
          F = min(F, ip[4 * i + 2]);
        }
        N |= ip[4 * i + 3];
      }
      pick[0] = N == 0 && C == 1 && L != -INFINITY ? F : -1;
    }
    __syncthreads();
    fast = pick[0] >= 0;
    if (fast && tid == 0) ctok[0] = pick[0];
  }
  // penalty (_frenar): the logits as they came, then the tokens of the window penalized from those same values
  float* lout = (a.logits_out && step >= 0 && step < a.steps) ? a.logits_out + (b * a.steps + step) * V : nullptr;
  if (!direct) {
  each(lg, V, [&](int64_t v, float l) {
    work[v] = l;
    if (lout) lout[v] = l;
  });
  }
  __syncthreads();
  if (!direct && a.penalty != 1.f) {
    for (int j = tid; j < a.window; j += kSampleThreads) {
      const int64_t p = pos - a.window + j;
      if (p < 0) continue;
      const int64_t v = text[p];
      const float l = lg[v];
      work[v] = l > 0.f ? l / a.penalty : l * a.penalty;       // duplicates write the same value
    }
  }
  __syncthreads();
  // bans: tokens that would close an n-gram already generated (only generated tokens count)
  if (bans) {
    if (nb_list >= 0) {
      if (tid < nb_list) work[blist[tid]] = ninf;
    } else {
      const KeyForm f = key_form(nb, a.w);
      const uint64_t base = pack(f, text + pos - (nb - 1), nb - 1);
      for (int64_t v = tid; v < V; v += kSampleThreads)
        if (set_has(a.ban, b, f.key_of(f.step(base, nb - 1, v)))) work[v] = ninf;
    }
  }
  __syncthreads();
  if (!direct) {
    float finite = 0.f;
    each(work, V, [&](int64_t, float x) { finite += (x == ninf) ? 0.f : 1.f; });
    if (block_sum(finite, red) == 0.f) {                        // nothing left: the plain logits (no penalty either)
      __syncthreads();
      each(lg, V, [&](int64_t v, float l) { work[v] = l; });
    }
  }
  __syncthreads();

  // quote mask and its mass at temperature 1 (_conservar_cita's p1)
  uint32_t* qbits = a.quote_bits + b * ((V + 31) / 32);
  const bool qprobe = quote && nq_list < 0 && !fast;
  if (qprobe) {
    const KeyForm f = key_form(nq, a.w);
    const uint64_t base = pack(f, text + pos - (nq - 1), nq - 1);
    for (int64_t wd = tid; wd < (V + 31) / 32; wd += kSampleThreads) {
      uint32_t bits = 0;
      for (int i = 0; i < 32; ++i) {
        const int64_t v = wd * 32 + i;
        if (v < V && set_has(a.quote, b, f.key_of(f.step(base, nq - 1, v)))) bits |= 1u << i;
      }
      qbits[wd] = bits;
    }
    __syncthreads();
  }
  const int nql = quote && !qprobe ? nq_list : 0;
  auto in_quote = [&](int64_t v) {
    if (!quote) return false;
    if (qprobe) return ((qbits[v >> 5] >> (v & 31)) & 1u) != 0u;
    for (int i = 0; i < nql; ++i)
      if (qlist[i] == v) return true;
    return false;
  };
  float mass_p = 0.f;
  const bool need_mass = quote && (qprobe || nql > 0);
  const float tden = fmaxf(a.temperature, 1e-6f);
  float corte = ninf;
  // greedy: one pass gives the quote mass at temperature 1 (a running maximum with its sums rescaled), the maximum
  // of x / T and each thread's tokens at that maximum (the kept set), in the order the list gather below uses
  bool listed = fast;
  int ncand = fast ? 1 : 0;
  if (greedy && !fast) {
    float m = ninf, sm = 0.f, cm = 0.f, lmax = ninf;
    int cnt = 0;
    bool nan = false;                                            // NaN logits: the passes below keep them as they did
    int* mine = (int*)cval + tid * kTiesPerThread;              // this thread's tied tokens, ascending
    each(src, V, [&](int64_t v, float x) {
      if (direct && lout) lout[v] = x;
      if (need_mass && x != ninf) {
        const bool q = qprobe && in_quote(v);
        if (x > m) {
          const float sc = m == ninf ? 0.f : expf(m - x);
          sm = sm * sc + 1.f;
          cm = cm * sc + (q ? 1.f : 0.f);
          m = x;
        } else {
          const float e = expf(x - m);
          sm += e;
          if (q) cm += e;
        }
      }
      const float l = x / tden;
      nan |= l != l;
      if (l > lmax) {
        lmax = l;
        cnt = 0;
      }
      if (l == lmax) {
        if (cnt < kTiesPerThread) mine[cnt] = (int)v;
        ++cnt;
      }
    });
    if (need_mass) {
      const float m1 = block_max(m, red);
      const float S1 = block_sum(m == ninf ? 0.f : sm * expf(m - m1), red);
      float c = qprobe ? (m == ninf ? 0.f : cm * expf(m - m1)) : 0.f;
      if (!qprobe && tid < nql) c = expf(src[qlist[tid]] - m1);
      mass_p = block_sum(c, red) / S1;
    }
    corte = block_max(lmax, red);
    const int my = lmax == corte ? cnt : 0;
    // more ties than a thread keeps, or NaN logits (degenerate rows): the count and gather passes below
    if (block_max(my > kTiesPerThread || nan ? 1.f : 0.f, red) == 0.f) {
      __syncthreads();
      cscan[tid] = my;
      __syncthreads();
      for (int off = 1; off < kSampleThreads; off <<= 1) {
        const int add = tid >= off ? cscan[tid - off] : 0;
        __syncthreads();
        cscan[tid] += add;
        __syncthreads();
      }
      ncand = cscan[kSampleThreads - 1];
      const int o = cscan[tid] - my;
      int t[kTiesPerThread];
#pragma unroll
      for (int j = 0; j < kTiesPerThread; ++j) t[j] = j < my ? mine[j] : 0;
      __syncthreads();                                             // every thread holds its ties: cval is free
#pragma unroll
      for (int j = 0; j < kTiesPerThread; ++j)
        if (j < my) {
          ctok[o + j] = t[j];
          cval[o + j] = corte;
        }
      __syncthreads();
      listed = true;
    }
    __syncthreads();
  } else if (!greedy && need_mass) {
    float m = ninf;
    each(src, V, [&](int64_t, float x) { m = fmaxf(m, x); });
    const float m1 = block_max(m, red);
    float s = 0.f, c = 0.f;
    each(src, V, [&](int64_t v, float x) {
      const float e = expf(x - m1);
      s += e;
      if (qprobe && in_quote(v)) c += e;
    });
    if (!qprobe && tid < nql) c = expf(src[qlist[tid]] - m1);
    const float S1 = block_sum(s, red);
    mass_p = block_sum(c, red) / S1;
  }

  // temperature and top-k: keep the logits >= the k-th largest
  if (!greedy && a.top_k > 0 && (int64_t)a.top_k < V) {
    uint32_t prefix = 0, mask = 0, rest = (uint32_t)a.top_k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += kSampleThreads) hist_n[i] = 0;
      __syncthreads();
      each_all(src, V, [&](int64_t, float x, bool ok) {
        const uint32_t k = ok ? ordered(x / tden) : 0u;
        hist_count(hist_n, (k >> shift) & 255u, ok && (k & mask) == prefix);
      });
      __syncthreads();
      if (tid == 0) {
        uint32_t cum = 0, d = 0;
        for (int i = 255; i >= 0; --i) {
          if (cum + hist_n[i] >= rest) { d = (uint32_t)i; break; }
          cum += hist_n[i];
        }
        sel[0] = d;
        sel[1] = rest - cum;
      }
      __syncthreads();
      prefix |= sel[0] << shift;
      mask |= 255u << shift;
      rest = sel[1];
      __syncthreads();
    }
    corte = from_ordered(prefix);
  }
  auto kept_k = [&](float l) { return !(l < corte); };

  // Few tokens past the top-k cut: they are gathered into LDS in a fixed order (thread, then stride) and the rest of
  // the decision (top-p, the softmax, the quote-mass correction, the draw) runs on them alone. More than kMaxCand
  // (ties at the cut): the full-row passes below.
  bool lista = listed;
  if (!listed && a.top_k > 0 && (int64_t)a.top_k < V) {
    int cnt = 0;
    each(src, V, [&](int64_t, float x) { cnt += kept_k(x / tden) ? 1 : 0; });
    __syncthreads();
    cscan[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < kSampleThreads; off <<= 1) {
      const int add = tid >= off ? cscan[tid - off] : 0;
      __syncthreads();
      cscan[tid] += add;
      __syncthreads();
    }
    ncand = cscan[kSampleThreads - 1];
    lista = ncand <= kMaxCand;
    if (lista) {
      int o = cscan[tid] - cnt;
      each(src, V, [&](int64_t v, float x) {
        const float l = x / tden;
        if (kept_k(l)) {
          ctok[o] = (int)v;
          cval[o] = l;
          ++o;
        }
      });
      __syncthreads();
    }
  }
  if (lista && ncand == 1 && !a.prob_out) {
    // one token kept (a greedy row's maximum): its probability is 1 whatever the top-p cut and the quote correction,
    // so the draw picks it
    if (tid == 0) {
      pick[0] = ctok[0];
      pick[1] = -1;
    }
    __syncthreads();
  } else if (lista) {
    float m = ninf;
    for (int i = tid; i < ncand; i += kSampleThreads) m = fmaxf(m, cval[i]);
    const float m3 = block_max(m, red);
    float tau = -1.f, S3 = 1.f;
    if (a.top_p < 1.f) {
      float s = 0.f;
      for (int i = tid; i < ncand; i += kSampleThreads) s += expf(cval[i] - m3);
      S3 = block_sum(s, red);
      const double target = ceil((double)a.top_p * kMassScale);
      uint32_t prefix = 0, mask = 0;
      unsigned long long acc = 0;
      bool found = true;
      for (int shift = 24; shift >= 0 && found; shift -= 8) {
        for (int i = tid; i < 256; i += kSampleThreads) {
          hist_n[i] = 0;
          hist_m[i] = 0;
        }
        __syncthreads();
        for (int base = 0; base < ncand; base += kSampleThreads) {
          const int i = base + tid;
          const bool ok = i < ncand;
          const float p = ok ? expf(cval[i] - m3) / S3 : 0.f;
          const uint32_t k = __float_as_uint(p);
          hist_mass(hist_n, hist_m, (k >> shift) & 255u, ok && (k & mask) == prefix,
                    (unsigned long long)rint((double)p * kMassScale));
        }
        __syncthreads();
        if (tid == 0) {
          int d = -1;
          for (int i = 255; i >= 0; --i) {
            if (hist_n[i] == 0) continue;
            if ((double)(acc + hist_m[i]) >= target) { d = i; break; }
            acc += hist_m[i];
          }
          sel[0] = d < 0 ? 0u : (uint32_t)d;
          sel[1] = d < 0 ? 0u : 1u;
        }
        __syncthreads();
        found = sel[1] != 0;
        prefix |= sel[0] << shift;
        mask |= 255u << shift;
        __syncthreads();
      }
      if (found) tau = __uint_as_float(prefix);
      const unsigned int m_tie = tau >= 0.f ? hist_n[sel[0]] : 0u;
      if (m_tie > 1u) {                           // tied tokens at the boundary: the first K by token index stay
        if (tid == 0) tie_acc = acc;
        __syncthreads();
        const unsigned long long above = tie_acc;
        tie_max = top_p_tie_limit(top_p_ties_kept(above, target, tau, m_tie), V, [&](int64_t v) {
          uint32_t c = 0u;
          for (int i = tid; i < ncand; i += kSampleThreads)
            c += (expf(cval[i] - m3) / S3 == tau && ctok[i] < v) ? 1u : 0u;
          return block_isum(c, red, &tie_cnt);
        });
      }
    }
    auto keep_i = [&](int i, float* e) {
      *e = expf(cval[i] - m3);
      const float p = *e / S3;
      return tau < 0.f || p > tau || (p == tau && ctok[i] <= tie_max);
    };
    float s4 = 0.f;
    for (int i = tid; i < ncand; i += kSampleThreads) {
      float e;
      if (keep_i(i, &e)) s4 += e;
    }
    const float S4 = block_sum(s4, red);
    float sc_q = 1.f, sc_n = 1.f;
    if (quote && (qprobe || nql > 0)) {
      float c = 0.f;
      for (int i = tid; i < ncand; i += kSampleThreads) {
        float e;
        if (in_quote(ctok[i]) && keep_i(i, &e)) c += e / S4;
      }
      const float mass_q = block_sum(c, red);
      if (mass_q > 0.f && mass_q < 1.f) {
        sc_q = mass_p / fmaxf(mass_q, 1e-30f);
        sc_n = (1.f - mass_p) / fmaxf(1.f - mass_q, 1e-30f);
      }
    }
    const bool scaled = sc_q != 1.f || sc_n != 1.f;
    auto prob_i = [&](int i) {
      float e;
      if (!keep_i(i, &e)) return 0.f;
      const float p = e / S4;
      return scaled ? p * (in_quote(ctok[i]) ? sc_q : sc_n) : p;
    };
    if (a.prob_out) {
      each(src, V, [&](int64_t v, float) { a.prob_out[b * V + v] = 0.f; });
      __syncthreads();
      for (int i = tid; i < ncand; i += kSampleThreads) a.prob_out[b * V + ctok[i]] = prob_i(i);
    }
    // the draw over the list, each thread a contiguous segment of it
    const int seg = (ncand + kSampleThreads - 1) / kSampleThreads;
    const int i0 = tid * seg < ncand ? tid * seg : ncand, i1 = i0 + seg < ncand ? i0 + seg : ncand;
    float local = 0.f;
    int last = -1;
    for (int i = i0; i < i1; ++i) {
      const float p = prob_i(i);
      local += p;
      if (p > 0.f) last = i;
    }
    __syncthreads();
    scan[tid] = local;
    if (tid < 2) pick[tid] = tid == 0 ? 0x7fffffff : -1;
    __syncthreads();
    for (int off = 1; off < kSampleThreads; off <<= 1) {
      const float add = tid >= off ? scan[tid - off] : 0.f;
      __syncthreads();
      scan[tid] += add;
      __syncthreads();
    }
    const float total = scan[kSampleThreads - 1];
    const float before = tid > 0 ? scan[tid - 1] : 0.f;
    const float after = scan[tid];
    const uint64_t r = mix64(a.seed ^ mix64((uint64_t)pos * 0x9e3779b97f4a7c15ull + (uint64_t)b));
    const float u = (float)(r >> 40) * (1.f / 16777216.f);
    const float target = u * total;
    if (local > 0.f && target >= before && target < after) {
      const float inside = target - before;
      float acc = 0.f;
      int chosen = -1;
      for (int i = i0; i < i1; ++i) {
        const float p = prob_i(i);
        acc += p;
        if (p > 0.f && acc > inside) {
          chosen = i;
          break;
        }
      }
      if (chosen < 0) chosen = last;
      if (chosen >= 0) atomicMin(&pick[0], chosen);
    }
    if (last >= 0) atomicMax(&pick[1], last);
    __syncthreads();
    if (tid == 0) {                                              // list positions -> token ids
      const int o = pick[0] != 0x7fffffff ? pick[0] : pick[1];
      pick[0] = o >= 0 ? ctok[o] : 0x7fffffff;
      pick[1] = -1;
    }
    __syncthreads();
  } else {
    // the kept logits' max (the row's max is always kept) and top-p over their softmax
    float mloc = ninf;
    each(src, V, [&](int64_t, float x) {
      const float l = x / tden;
      if (kept_k(l)) mloc = fmaxf(mloc, l);
    });
    const float m3 = block_max(mloc, red);
    float tau = -1.f;                                              // keep probabilities >= tau (all when < 0)
    float S3 = 1.f;
    if (a.top_p < 1.f) {
      float s = 0.f;
      each(src, V, [&](int64_t, float x) {
        const float l = x / tden;
        if (kept_k(l)) s += expf(l - m3);
      });
      S3 = block_sum(s, red);
      const double target = ceil((double)a.top_p * kMassScale);
      uint32_t prefix = 0, mask = 0;
      unsigned long long acc = 0;
      bool found = true;
      for (int shift = 24; shift >= 0 && found; shift -= 8) {
        for (int i = tid; i < 256; i += kSampleThreads) {
          hist_n[i] = 0;
          hist_m[i] = 0;
        }
        __syncthreads();
        each_all(src, V, [&](int64_t, float x, bool ok) {
          const float l = x / tden;
          const bool in = ok && kept_k(l);
          const float p = in ? expf(l - m3) / S3 : 0.f;
          const uint32_t k = __float_as_uint(p);
          hist_mass(hist_n, hist_m, (k >> shift) & 255u, in && (k & mask) == prefix,
                    (unsigned long long)rint((double)p * kMassScale));
        });
        __syncthreads();
        if (tid == 0) {
          // from the largest values down: the bin where the mass of everything at or above it first reaches top_p
          int d = -1;
          for (int i = 255; i >= 0; --i) {
            if (hist_n[i] == 0) continue;
            if ((double)(acc + hist_m[i]) >= target) { d = i; break; }
            acc += hist_m[i];
          }
          sel[0] = d < 0 ? 0u : (uint32_t)d;
          sel[1] = d < 0 ? 0u : 1u;
        }
        __syncthreads();
        found = sel[1] != 0;
        prefix |= sel[0] << shift;
        mask |= 255u << shift;
        __syncthreads();
      }
      if (found) tau = __uint_as_float(prefix);
      const unsigned int m_tie = tau >= 0.f ? hist_n[sel[0]] : 0u;
      if (m_tie > 1u) {                           // tied tokens at the boundary: the first K by token index stay
        if (tid == 0) tie_acc = acc;
        __syncthreads();
        const unsigned long long above = tie_acc;
        tie_max = top_p_tie_limit(top_p_ties_kept(above, target, tau, m_tie), V, [&](int64_t lim) {
          return block_isum(ties_below(src, V, lim, tden, corte, m3, S3, tau), red, &tie_cnt);
        });
      }
    }

    // final probabilities: softmax over what is kept, then the quote-mass correction
    auto keep = [&](int64_t v, float x, float* e) {
      const float l = x / tden;
      if (!kept_k(l)) return false;
      *e = expf(l - m3);
      const float p = *e / S3;
      return tau < 0.f || p > tau || (p == tau && v <= tie_max);
    };
    float S4;
    {
      float s = 0.f;
      each(src, V, [&](int64_t v, float x) {
        float e;
        if (keep(v, x, &e)) s += e;
      });
      S4 = block_sum(s, red);
    }
    float sc_q = 1.f, sc_n = 1.f;
    if (quote && (qprobe || nql > 0)) {
      float c = 0.f, e;
      if (qprobe) {
        each(src, V, [&](int64_t v, float x) {
          float ee;
          if (in_quote(v) && keep(v, x, &ee)) c += ee / S4;
        });
      } else if (tid < nql && keep(qlist[tid], src[qlist[tid]], &e)) {
        c = e / S4;
      }
      const float mass_q = block_sum(c, red);
      if (mass_q > 0.f && mass_q < 1.f) {
        sc_q = mass_p / fmaxf(mass_q, 1e-30f);
        sc_n = (1.f - mass_p) / fmaxf(1.f - mass_q, 1e-30f);
      }
    }
    const bool scaled = sc_q != 1.f || sc_n != 1.f;
    auto prob = [&](int64_t v, float x) {
      float e;
      if (!keep(v, x, &e)) return 0.f;
      const float p = e / S4;
      return scaled ? p * (in_quote(v) ? sc_q : sc_n) : p;
    };
    if (a.prob_out) each(src, V, [&](int64_t v, float x) { a.prob_out[b * V + v] = prob(v, x); });

    // the draw: inverse CDF over the tokens in index order, each thread a contiguous segment
    const int64_t seg = (V + kSampleThreads - 1) / kSampleThreads;
    const int64_t v0 = (int64_t)tid * seg < V ? (int64_t)tid * seg : V;
    const int64_t v1 = v0 + seg < V ? v0 + seg : V;
    float local = 0.f;
    int64_t last_pos = -1;
    each_range(src, v0, v1, [&](int64_t v, float x) {
      const float p = prob(v, x);
      local += p;
      if (p > 0.f) last_pos = v;
      return true;
    });
    scan[tid] = local;
    if (tid < 2) pick[tid] = tid == 0 ? 0x7fffffff : -1;
    __syncthreads();
    for (int off = 1; off < kSampleThreads; off <<= 1) {        // inclusive scan (Hillis-Steele), fixed order
      const float add = tid >= off ? scan[tid - off] : 0.f;
      __syncthreads();
      scan[tid] += add;
      __syncthreads();
    }
    // thread t owns [scan[t - 1], scan[t]): neighbouring bounds are the same numbers, so the segments tile [0, total)
    const float total = scan[kSampleThreads - 1];
    const float before = tid > 0 ? scan[tid - 1] : 0.f;
    const float after = scan[tid];
    const uint64_t r = mix64(a.seed ^ mix64((uint64_t)pos * 0x9e3779b97f4a7c15ull + (uint64_t)b));
    const float u = (float)(r >> 40) * (1.f / 16777216.f);      // 24 random bits: [0, 1)
    const float target = u * total;
    if (local > 0.f && target >= before && target < after) {
      const float inside = target - before;
      float acc = 0.f;                                             // summed from 0 in `local`'s order
      int64_t chosen = -1;
      each_range(src, v0, v1, [&](int64_t v, float x) {
        const float p = prob(v, x);
        acc += p;
        if (p > 0.f && acc > inside) {
          chosen = v;
          return false;
        }
        return true;
      });
      if (chosen < 0) chosen = last_pos;
      if (chosen >= 0) atomicMin(&pick[0], (int)chosen);
    }
    if (last_pos >= 0) atomicMax(&pick[1], (int)last_pos);
    __syncthreads();
  }

  if (tid == 0) {
    int64_t tok = pick[0] != 0x7fffffff ? pick[0] : (pick[1] >= 0 ? pick[1] : 0);
    if (a.stop_token >= 0) {
      if (a.done[b]) {
        tok = a.stop_token;
      } else if (tok == a.stop_token) {
        a.done[b] = 1;
        a.stop_step[b] = (int32_t)step;
      }
    }
    text[pos] = tok;
    a.tokens[b] = tok;
    if (a.quote.slots && pos + 1 >= nq) ngram_put(a.quote, b, text + pos - (nq - 1), a.w, qat);
    if (a.ban.slots && pos + 1 - a.L0 >= nb) ngram_put(a.ban, b, text + pos - (nb - 1), a.w, bat);
  }
}

// k_sample_reg's tied tokens at the top-p boundary (m > 1 of them; bit r of `ties`: this thread's token r 1024 + tid):
// their ids into wtok (free at that point), and the K-th smallest is the last one kept (more than 1,024 tied tokens:
// all of them stay). Out of line, so that the rare case costs the common one no registers.
template <int R>
__device__ __noinline__ int reg_tie_max(uint32_t ties, unsigned int m, unsigned long long above, double target,
                                        float tau, int* wtok, unsigned int* cnt, unsigned long long* res) {
  const int tid = threadIdx.x;
  const unsigned long long K = top_p_ties_kept(above, target, tau, m);
  if (K == 0ull || m > (unsigned int)kSampleThreads) return INT_MAX;
  __syncthreads();
  if (tid == 0) *cnt = 0u;
  __syncthreads();
  for (int r = 0; r < R; ++r)
    if ((ties >> r) & 1u) wtok[atomicAdd(cnt, 1u) & (kSampleThreads - 1)] = r * kSampleThreads + tid;
  __syncthreads();
  if (tid < (int)m) {
    const int me = wtok[tid];
    unsigned int rank = 0u;
    for (unsigned int j = 0; j < m; ++j) rank += wtok[j] < me ? 1u : 0u;
    if (rank == (unsigned int)(K - 1ull)) *res = (unsigned long long)me;
  }
  __syncthreads();
  return (int)*res;
}

// The same decision with the row held in registers: thread t owns tokens t, t + 1024, ..., t + (R - 1) * 1024, loaded
// once, so every pass after the first is arithmetic on registers (the global-memory kernel above reads the row from
// the cache in each pass, eight loads in flight per thread). Tokens the thread does not own are reached through LDS lists (window, bans, quotes). The
// draw walks the tokens in thread-major order (thread 0's R tokens, then thread 1's, ...): a fixed order, so the
// inverse CDF draws from the same distribution, with other tokens for a given uniform than the index order would.
template <int R>
__global__ __launch_bounds__(kSampleThreads) void k_sample_reg(SampleArgs a) {
  __shared__ Red red;
  __shared__ unsigned int hist_n[256];
  __shared__ unsigned long long hist_m[256];
  __shared__ uint32_t sel[2];
  __shared__ float scan[kSampleThreads];
  __shared__ int pick[2];
  __shared__ int qlist[kSucc], blist[kSucc];
  __shared__ int nq_list, nb_list;
  __shared__ int wtok[kSampleThreads];
  __shared__ unsigned long long tie_acc;
  __shared__ unsigned int tie_cnt;
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t pos = *a.pos_dev;
  if (pos < 0 || pos > a.pos_max) return;                       // outside the text buffer: nothing is touched
  const int64_t V = a.V;
  const float* lg = a.lg + b * a.ldl;
  int64_t* text = a.text + b * a.ld_text;
  const int64_t step = pos - a.L0;
  const float ninf = -INFINITY;
  const int nq = a.quote.n, nb = a.ban.n;
  const bool quote = a.quote.slots && pos >= nq;
  const bool bans = a.ban.slots && pos - a.L0 >= nb;
  CtxAt qat, bat;                                               // thread 0's: reused by the insert at the end
  if (tid == 0) {
    nq_list = nb_list = 0;
    if (quote) successors(a.quote, b, text, pos, a.w, qlist, &nq_list, &qat);
    if (bans) successors(a.ban, b, text, pos, a.w, blist, &nb_list, &bat);
  }
  auto tok_of = [&](int r) { return (int64_t)r * kSampleThreads + tid; };
  // the slot of token v when this thread owns it
  auto owned = [&](int64_t v, int* r) {
    if (v < 0 || (v & (kSampleThreads - 1)) != tid) return false;
    *r = (int)(v >> 10);
    return *r < R;
  };

  float x[R];
  float* lout = (a.logits_out && step >= 0 && step < a.steps) ? a.logits_out + (b * a.steps + step) * V : nullptr;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t v = tok_of(r);
    x[r] = v < V ? lg[v] : ninf;
    if (lout && v < V) lout[v] = x[r];
  }
  // penalty over the window's tokens, each penalized once from its own logit
  if (a.penalty != 1.f) {
    uint64_t hecho = 0;
    for (int base = 0; base < a.window; base += kSampleThreads) {
      const int j = base + tid;
      const int64_t p = pos - a.window + j;
      __syncthreads();
      wtok[tid] = (j < a.window && p >= 0) ? (int)text[p] : -1;
      __syncthreads();
      const int cnt = a.window - base < kSampleThreads ? a.window - base : kSampleThreads;
      for (int k = 0; k < cnt; ++k) {
        int rr;
        if (owned(wtok[k], &rr) && !((hecho >> rr) & 1ull)) {
          hecho |= 1ull << rr;
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (r == rr) x[r] = x[r] > 0.f ? x[r] / a.penalty : x[r] * a.penalty;
        }
      }
    }
  }
  __syncthreads();                                              // the successor lists are visible from here
  if (bans) {
    if (nb_list >= 0) {
      for (int k = 0; k < nb_list; ++k) {
        int rr;
        if (owned(blist[k], &rr)) {
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (r == rr) x[r] = ninf;
        }
      }
    } else {
      const KeyForm f = key_form(nb, a.w);
      const uint64_t base = pack(f, text + pos - (nb - 1), nb - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t v = tok_of(r);
        if (v < V && set_has(a.ban, b, f.key_of(f.step(base, nb - 1, v)))) x[r] = ninf;
      }
    }
  }
  {
    float finite = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) finite += (tok_of(r) < V && x[r] != ninf) ? 1.f : 0.f;
    if (block_sum(finite, red) == 0.f) {                        // nothing left: the plain logits (no penalty either)
#pragma unroll
      for (int r = 0; r < R; ++r) x[r] = tok_of(r) < V ? lg[tok_of(r)] : ninf;
    }
  }

  // quote flags (bit r: token tok_of(r) closes an n-gram of the text) and the quote mass at temperature 1
  uint64_t qmask = 0;
  if (quote) {
    if (nq_list >= 0) {
      for (int k = 0; k < nq_list; ++k) {
        int rr;
        if (owned(qlist[k], &rr)) qmask |= 1ull << rr;
      }
    } else {
      const KeyForm f = key_form(nq, a.w);
      const uint64_t base = pack(f, text + pos - (nq - 1), nq - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t v = tok_of(r);
        if (v < V && set_has(a.quote, b, f.key_of(f.step(base, nq - 1, v)))) qmask |= 1ull << r;
      }
    }
  }
  const bool hay_cita = quote && (nq_list != 0);
  float mass_p = 0.f;
  if (hay_cita) {
    float m = ninf;
#pragma unroll
    for (int r = 0; r < R; ++r) m = fmaxf(m, x[r]);
    const float m1 = block_max(m, red);
    float s = 0.f, c = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float e = tok_of(r) < V ? expf(x[r] - m1) : 0.f;
      s += e;
      if ((qmask >> r) & 1ull) c += e;
    }
    const float S1 = block_sum(s, red);
    mass_p = block_sum(c, red) / S1;
  }

  // temperature, then top-k by radix selection over the values' ordered bits
  const float tden = fmaxf(a.temperature, 1e-6f);
#pragma unroll
  for (int r = 0; r < R; ++r) x[r] = x[r] / tden;
  float corte = ninf;
  if (a.top_k > 0 && (int64_t)a.top_k < V) {
    uint32_t prefix = 0, mask = 0, rest = (uint32_t)a.top_k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      __syncthreads();
      for (int i = tid; i < 256; i += kSampleThreads) hist_n[i] = 0;
      __syncthreads();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t k = ordered(x[r]);
        hist_count(hist_n, (k >> shift) & 255u, tok_of(r) < V && (k & mask) == prefix);
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t cum = 0, d = 0;
        for (int i = 255; i >= 0; --i) {
          if (cum + hist_n[i] >= rest) { d = (uint32_t)i; break; }
          cum += hist_n[i];
        }
        sel[0] = d;
        sel[1] = rest - cum;
      }
      __syncthreads();
      prefix |= sel[0] << shift;
      mask |= 255u << shift;
      rest = sel[1];
    }
    corte = from_ordered(prefix);
  }
  // from here x[r] is the kept logit or -inf
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (x[r] < corte) x[r] = ninf;
  float mloc = ninf;
#pragma unroll
  for (int r = 0; r < R; ++r) mloc = fmaxf(mloc, x[r]);
  const float m3 = block_max(mloc, red);
  float tau = -1.f;
  float S3 = 1.f;
  if (a.top_p < 1.f) {
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) s += expf(x[r] - m3);
    S3 = block_sum(s, red);
    const double target = ceil((double)a.top_p * kMassScale);
    uint32_t prefix = 0, mask = 0;
    unsigned long long acc = 0;
    bool found = true;
    for (int shift = 24; shift >= 0 && found; shift -= 8) {
      __syncthreads();
      for (int i = tid; i < 256; i += kSampleThreads) {
        hist_n[i] = 0;
        hist_m[i] = 0;
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool in = x[r] != ninf;
        const float p = in ? expf(x[r] - m3) / S3 : 0.f;
        const uint32_t k = __float_as_uint(p);
        hist_mass(hist_n, hist_m, (k >> shift) & 255u, in && (k & mask) == prefix,
                  (unsigned long long)rint((double)p * kMassScale));
      }
      __syncthreads();
      if (tid == 0) {
        int d = -1;
        for (int i = 255; i >= 0; --i) {
          if (hist_n[i] == 0) continue;
          if ((double)(acc + hist_m[i]) >= target) { d = i; break; }
          acc += hist_m[i];
        }
        sel[0] = d < 0 ? 0u : (uint32_t)d;
        sel[1] = d < 0 ? 0u : 1u;
      }
      __syncthreads();
      found = sel[1] != 0;
      prefix |= sel[0] << shift;
      mask |= 255u << shift;
    }
    if (found) tau = __uint_as_float(prefix);
    if (tau >= 0.f) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (x[r] != ninf && !(expf(x[r] - m3) / S3 >= tau)) x[r] = ninf;
      const unsigned int m_tie = hist_n[sel[0]];
      if (m_tie > 1u) {                           // tied tokens at the boundary: the first K by token index stay
        if (tid == 0) tie_acc = acc;
        __syncthreads();
        const unsigned long long above = tie_acc;
        uint32_t ties = 0;
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (x[r] != ninf && expf(x[r] - m3) / S3 == tau) ties |= 1u << r;
        const int tie_max = reg_tie_max<R>(ties, m_tie, above, target, tau, wtok, &tie_cnt, &tie_acc);
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (((ties >> r) & 1u) && tok_of(r) > (int64_t)tie_max) x[r] = ninf;
      }
    }
  }

  // final probabilities in place: softmax over what is kept, then the quote-mass correction
  float s4 = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    x[r] = expf(x[r] - m3);
    s4 += x[r];
  }
  const float S4 = block_sum(s4, red);
#pragma unroll
  for (int r = 0; r < R; ++r) x[r] = x[r] / S4;
  if (hay_cita) {
    float c = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if ((qmask >> r) & 1ull) c += x[r];
    const float mass_q = block_sum(c, red);
    if (mass_q > 0.f && mass_q < 1.f) {
      const float sc_q = mass_p / fmaxf(mass_q, 1e-30f), sc_n = (1.f - mass_p) / fmaxf(1.f - mass_q, 1e-30f);
#pragma unroll
      for (int r = 0; r < R; ++r) x[r] = x[r] * (((qmask >> r) & 1ull) ? sc_q : sc_n);
    }
  }
  if (a.prob_out) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tok_of(r) < V) a.prob_out[b * V + tok_of(r)] = x[r];
  }

  // the draw: inverse CDF in thread-major order
  float local = 0.f;
  int last = -1;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    local += x[r];
    if (x[r] > 0.f) last = r;
  }
  __syncthreads();
  scan[tid] = local;
  if (tid < 2) pick[tid] = tid == 0 ? 0x7fffffff : -1;
  __syncthreads();
  for (int off = 1; off < kSampleThreads; off <<= 1) {
    const float add = tid >= off ? scan[tid - off] : 0.f;
    __syncthreads();
    scan[tid] += add;
    __syncthreads();
  }
  const float total = scan[kSampleThreads - 1];
  const float before = tid > 0 ? scan[tid - 1] : 0.f;
  const float after = scan[tid];
  const uint64_t rnd = mix64(a.seed ^ mix64((uint64_t)pos * 0x9e3779b97f4a7c15ull + (uint64_t)b));
  const float u = (float)(rnd >> 40) * (1.f / 16777216.f);
  const float target = u * total;
  if (local > 0.f && target >= before && target < after) {
    const float inside = target - before;
    float acc = 0.f;
    int chosen = -1;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc += x[r];
      if (chosen < 0 && x[r] > 0.f && acc > inside) chosen = r;
    }
    if (chosen < 0) chosen = last;
    if (chosen >= 0) atomicMin(&pick[0], tid * R + chosen);     // the position in thread-major order
  }
  if (last >= 0) atomicMax(&pick[1], tid * R + last);
  __syncthreads();

  if (tid == 0) {
    const int o = pick[0] != 0x7fffffff ? pick[0] : pick[1];
    int64_t tok = o >= 0 ? (int64_t)(o % R) * kSampleThreads + o / R : 0;
    if (a.stop_token >= 0) {
      if (a.done[b]) {
        tok = a.stop_token;
      } else if (tok == a.stop_token) {
        a.done[b] = 1;
        a.stop_step[b] = (int32_t)step;
      }
    }
    text[pos] = tok;
    a.tokens[b] = tok;
    if (a.quote.slots && pos + 1 >= nq) ngram_put(a.quote, b, text + pos - (nq - 1), a.w, qat);
    if (a.ban.slots && pos + 1 - a.L0 >= nb) ngram_put(a.ban, b, text + pos - (nb - 1), a.w, bat);
  }
}

int check_set(const char* what, const TupleSet& s, int32_t w) {
  if (!s.slots) return 0;
  ASRN_REQUIRE(s.ctx && s.count && s.succ, "%s: a set needs its context, count and successor tables", what);
  ASRN_REQUIRE(s.cap >= 2 && (s.cap & (s.cap - 1)) == 0, "%s: the set's capacity %lld must be a power of two", what,
               (long long)s.cap);
  ASRN_REQUIRE(s.n >= 1 && w >= 1 && w <= 62, "%s: n=%d must be >= 1 and w=%d in [1, 62]", what, s.n, w);
  return 0;
}

}  // namespace
}  // namespace asrn

using namespace asrn;

extern "C" int32_t asrn_sample_bits(int64_t V) {
  // bits per token such that the largest id, V - 1, is below 2^w - 1: the all-ones key then never occurs
  int32_t w = 1;
  while (w < 62 && ((int64_t(1) << w) - 1) <= V - 1) ++w;
  return w;
}

extern "C" int32_t asrn_ngram_set_successors(void) { return kSucc; }

extern "C" int asrn_ngram_set_build(const int64_t* x, int64_t ldx, int64_t rows, int64_t L, int32_t n, int32_t w,
                                    uint64_t* slots, uint64_t* ctx, int32_t* count, int32_t* succ, int64_t cap,
                                    void* stream) {
  ASRN_REQUIRE(rows >= 0 && L >= 0 && ldx >= L, "asrn_ngram_set_build: bad sizes rows=%lld L=%lld ldx=%lld",
               (long long)rows, (long long)L, (long long)ldx);
  ASRN_REQUIRE(slots != nullptr, "asrn_ngram_set_build: null table");
  TupleSet s{(unsigned long long*)slots, (unsigned long long*)ctx, count, succ, cap, n};
  if (int rc = check_set("asrn_ngram_set_build", s, w)) return rc;
  ASRN_REQUIRE(L <= cap / 2, "asrn_ngram_set_build: %lld n-grams per row need a capacity of at least %lld (got %lld)",
               (long long)L, (long long)(2 * L), (long long)cap);
  const int64_t total = rows * L;
  if (total == 0) return 0;
  const int threads = 256;
  hipLaunchKernelGGL(k_set_build, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0,
                     (hipStream_t)stream, x, ldx, rows, L, s, w);
  return check_launch("asrn_ngram_set_build");
}

extern "C" int asrn_sample(const float* lg, int64_t ldl, float* work, uint32_t* quote_bits, float* prob_out,
                           float* logits_out, int64_t steps, int64_t* text, int64_t ld_text, const int64_t* pos_dev,
                           int64_t pos_max, int64_t L0, int64_t* tokens, uint8_t* done, int32_t* stop_step,
                           uint64_t* quote_slots, uint64_t* quote_ctx, int32_t* quote_count, int32_t* quote_succ,
                           int64_t quote_cap, int32_t quote_n, uint64_t* ban_slots, uint64_t* ban_ctx,
                           int32_t* ban_count, int32_t* ban_succ, int64_t ban_cap, int32_t ban_n, int32_t w, int64_t B,
                           int64_t V, float temperature, int32_t top_k, float top_p, float penalty, int32_t window,
                           int64_t stop_token, uint64_t seed, void* stream) {
  ASRN_REQUIRE(B >= 1 && V >= 1 && V <= (int64_t(1) << 31) && ldl >= V, "asrn_sample: bad sizes B=%lld V=%lld",
               (long long)B, (long long)V);
  ASRN_REQUIRE(B <= (int64_t(1) << 20), "asrn_sample: at most 2^20 rows");
  ASRN_REQUIRE(lg && work && quote_bits && text && pos_dev && tokens && done && stop_step, "asrn_sample: null pointer");
  ASRN_REQUIRE(pos_max >= 0 && pos_max < ld_text && L0 >= 0, "asrn_sample: positions up to %lld do not fit a text "
               "row of %lld", (long long)pos_max, (long long)ld_text);
  ASRN_REQUIRE(window >= 0 && top_k >= 0 && penalty > 0.f, "asrn_sample: window, top_k >= 0 and penalty > 0");
  ASRN_REQUIRE(w == asrn_sample_bits(V), "asrn_sample: w=%d must be asrn_sample_bits(V)=%d", w, asrn_sample_bits(V));
  ASRN_REQUIRE(logits_out == nullptr || steps >= 1, "asrn_sample: logits_out needs steps >= 1");
  SampleArgs a{};
  a.quote = TupleSet{(unsigned long long*)quote_slots, (unsigned long long*)quote_ctx, quote_count, quote_succ,
                     quote_cap, quote_n};
  a.ban = TupleSet{(unsigned long long*)ban_slots, (unsigned long long*)ban_ctx, ban_count, ban_succ, ban_cap, ban_n};
  if (int rc = check_set("asrn_sample (quote)", a.quote, w)) return rc;
  if (int rc = check_set("asrn_sample (bans)", a.ban, w)) return rc;
  a.lg = lg;
  a.ldl = ldl;
  a.work = work;
  a.quote_bits = quote_bits;
  a.prob_out = prob_out;
  a.logits_out = logits_out;
  a.steps = steps;
  a.text = text;
  a.ld_text = ld_text;
  a.pos_dev = pos_dev;
  a.pos_max = pos_max;
  a.L0 = L0;
  a.tokens = tokens;
  a.done = done;
  a.stop_step = stop_step;
  a.w = w;
  a.V = V;
  a.temperature = temperature;
  a.top_p = top_p;
  a.penalty = penalty;
  a.top_k = top_k;
  a.window = window;
  a.stop_token = stop_token;
  a.seed = seed;
  const dim3 grid((unsigned)B), block(kSampleThreads);
  const hipStream_t st = (hipStream_t)stream;
  static_assert(4 * kGreedySlices <= 16 * kSampleThreads, "the slices' results fit a row of the scratch");
  a.greedy_parts = V > 16 * kSampleThreads && top_k == 1 && penalty == 1.f && !logits_out && !prob_out;
  if (a.greedy_parts) {
    hipLaunchKernelGGL(k_greedy_part, dim3((unsigned)B, kGreedySlices), dim3(kGreedyThreads), 0, st, a);
    if (int rc = check_launch("asrn_sample (greedy pre-pass)")) return rc;
  }
  // rows up to 16 Ki tokens in registers (R tokens per thread: R = 16 is what fits 128 VGPRs, the budget of a
  // 1,024-thread workgroup), longer rows from global memory
  if (V <= 4 * kSampleThreads)
    hipLaunchKernelGGL(k_sample_reg<4>, grid, block, 0, st, a);
  else if (V <= 16 * kSampleThreads)
    hipLaunchKernelGGL(k_sample_reg<16>, grid, block, 0, st, a);
  else
    hipLaunchKernelGGL(k_sample, grid, block, 0, st, a);
  return check_launch("asrn_sample");
}
