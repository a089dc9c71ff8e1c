// The generation step's repetition branch for one (batch row, n-gram length): the clock advance, the n-gram key, the
// Hawkes lookup/update and the streak (reference nucleo:953-960, 1634-1714, 1826). Shared by the standalone step
// kernel (decode.hip) and the decode attention kernel that runs it beside the attention (candidates.hip). Contraction
// into fused multiply-adds is switched off inside these functions by a pragma, so the bits do not depend on the
// including file's -ffp-contract setting (the pragma is lexical: the arithmetic is written out here, since HIP's
// __dadd_rn and the like are inline functions whose operators it would not reach): the n-gram keys round each fp64
// multiply and add separately, and the Hawkes update and the streak are a multiply then an add, as in the reference.
#pragma once

#include "common.h"

namespace asrn {

constexpr uint64_t kEmpty = ~0ull;          // no non-NaN key has this code

__device__ __forceinline__ uint64_t table_code(double x) {
  if (x == 0.0) x = 0.0;
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {     // the splitmix64 finalizer
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Per (batch row, n-gram length) open-addressing tables of the Hawkes memory: keys, Bu and A are (groups, cap)
struct Table {
  uint64_t* keys; double* Bu; float* A; int64_t cap;
};

// slot of `code` in group g's table: the key's slot, or the empty slot where it goes; -1 if the table is full
__device__ __forceinline__ int64_t probe(const Table& tb, int64_t g, uint64_t code, bool* found) {
  const uint64_t* k = tb.keys + g * tb.cap;
  const int64_t mask = tb.cap - 1;
  int64_t s = (int64_t)(mix64(code) & (uint64_t)mask);
  for (int64_t n = 0; n < tb.cap; ++n, s = (s + 1) & mask) {
    const uint64_t v = k[s];
    if (v == code) {
      *found = true;
      return s;
    }
    if (v == kEmpty) {
      *found = false;
      return s;
    }
  }
  *found = false;
  return -1;
}

// The step's arguments. Caches are (B, stride) rows: sig, Bt (position t written here), log_alfa (position t given).
struct Step {
  const float* sig; double* Bt; const float* la; const double* beta_t; const double* coef; const float* kappa;
  const float* kappa_r; int64_t B, stride, t; int n;
  float* racha; float* vistos; float* hawkes;
  const int64_t* t_dev;    // optional: the position read from device memory instead of t
  int reloj32;             // the core layer's fp32 clock: Bt[t] = fp32(Bt[t-1] + beta_t), held in fp64
};

__device__ __forceinline__ int64_t step_pos(const Step& a) { return a.t_dev ? *a.t_dev : a.t; }

// The clock at position t of row b: Bt[t-1] + beta_t in fp64, or, for the core layer, as fp32 values added in fp32
// (nucleo:1826). The attention that runs beside the step forms the query's clock with this same function.
__device__ __forceinline__ double clock_at(const double* Btb, int64_t t, double beta, int reloj32) {
#pragma clang fp contract(off)
  return reloj32 ? (double)((t > 0 ? (float)Btb[t - 1] : 0.f) + (float)beta) : (t > 0 ? Btb[t - 1] : 0.0) + beta;
}

// One (b, j), e = b n + j < B n, at a position t inside the caches: no two e touch one table and no atomics are needed
__device__ __forceinline__ void repetition_row(const Step& a, const Table& tb, int64_t e, int64_t t) {
#pragma clang fp contract(off)
  const int64_t b = e / a.n;
  const int j = (int)(e % a.n);
  const double* Btb = a.Bt + b * a.stride;
  const double Bq = clock_at(Btb, t, a.beta_t[b], a.reloj32);
  if (j == 0) a.Bt[b * a.stride + t] = Bq;
  // key of the group of j + 1 pieces ending at t: sum_{k <= j} sig[t - k] c[k], NaN before the text (nucleo:175-186)
  double key = 0.0;
  for (int k = 0; k <= j; ++k) {
    const double s = t - k >= 0 ? (double)a.sig[b * a.stride + t - k] : __longlong_as_double(0x7ff8000000000000ll);
    key = key + s * a.coef[k];
  }
  float visto = 0.f, lam = 0.f;
  if (key == key) {
    bool found = false;
    const int64_t s = probe(tb, e, table_code(key), &found);
    if (s >= 0) {
      const int64_t o = e * tb.cap + s;
      if (found) {
        const float dB = (float)(Bq - tb.Bu[o]);                  // the difference in the clock's type
        lam = expf(-a.kappa[j] * dB) * tb.A[o];
        visto = 1.f;
      } else {
        tb.keys[o] = table_code(key);
      }
      tb.Bu[o] = Bq;
      tb.A[o] = lam + expf(a.la[b * a.stride + t]);
    }
  }
  a.vistos[e] = visto;
  a.hawkes[e] = lam;
  if (j == a.n - 1) {                                             // racha = r (exp(-kappa_r beta) racha + 1)
    const float g = expf(-a.kappa_r[0] * (float)a.beta_t[b]) * a.racha[b];
    a.racha[b] = visto * (g + 1.f);
  }
}

}  // namespace asrn
