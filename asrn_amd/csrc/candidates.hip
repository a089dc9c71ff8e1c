// a3 - a8: candidate attention over the recent bucket mates, forward and backward.
//
// One wavefront per token, in phases that each keep many independent loads in flight and reduce across lanes with
// DPP row rotations (no LDS round trips):
//   gather  the recent-mates index gives, per table, the token's sorted rank s and how many bucket mates sit right
//           before it (forward: the window [s - n, s)) or right after it (the backward's key pass: (s, s + n]); one
//           round of `order` loads yields every table's candidates, packed into one list in LDS grouped by table,
//           oldest first.
//   dedupe  the tables mostly return the same positions (the word tables hash the same token), so each entry is
//           matched against the earlier tables' segments and every distinct position gets one slot: the table-free
//           part of the score, the suffix match and the row gathers are done once per position.
//   score   a 32-lane half-wave reads one candidate's [phi ; Kc] row as one float4 per lane (512 B for P + cf = 128)
//           and reduces it against the query's pre-scaled [phi * scale_phi ; Qc * scale_c] in registers, 16 rows in
//           flight. Each table adds its own clock term; the exact masked softmax runs with one entry per lane.
//   gather  each distinct candidate's V row is read once by the 64 lanes with the weights summed over the tables,
//           8+ rows in flight: the table sum never leaves the kernel.
// The forward also keeps every candidate's weight att at [query][table][distance - 1]. The backward has one owner per
// output row, no atomics and no score recomputation: a query pass (ds = att (dp - D) with D = sum att*dp per (query,
// table), written next to att; query-side gradients; per-query partials of d gamma and d w_suf) and a key pass
// (key-side gradients: reads each (att, ds) pair with one 8-byte load at the slots of the queries that see the key).
#include <type_traits>

#include <cstdlib>

#include "common.h"
#include "repetition.h"

namespace asrn {

constexpr int kWavesPerBlock = 1;   // a wave's slot frees when its own query ends, and 5.9 KB of LDS a workgroup
                                    // fits 27 per CU (a 4-wave workgroup's 23.6 KB fits 6: 24 waves)
constexpr int kMaxSlots = 256;       // T * C
constexpr float kFill = -1e9f;       // the reference's "not allowed" score (asrn/nucleo.py:86)
constexpr float kLeakReach = 256.f;  // a table's best valid score within this of kFill is counted as a possible leak
constexpr int kCh = kMaxSlots / kWave;
constexpr int kRows = 8;             // rows per half-wave in flight in the feature loops

struct Cand {
  const float* phi; const float* V; const float* Qc; const float* Kc; const float* sig;
  // V rows: position p of batch row b at V + (b * L + p + vshift) * ldv (vshift 1: the layer's V[p] = W_v E[p + 1] read
  // straight from the projection of every position; the backward then writes dV at p + 1, and zeros at 0). dV has
  // V's layout: the same row stride ldv.
  int64_t ldv; int vshift;
  int64_t ldq;   // row stride of Qc and Kc (cf for dense rows; more when both are column blocks of one projection),
                 // and of dQc and dKc
  const double* Bt; const float* la; const float* w_suf; const float* gamma;
  const int32_t* order; const int32_t* win; const int32_t* rank;
  int64_t B, L;
  int d, P, cf, K, T, Tc, C;
  float sp, sc;
  // per-entry weights (B*L, T, C, 2): for the key at distance j + 1 before the query in a table, at slot j, its
  // attention weight (the forward writes it) and its ds (the backward's query pass writes it for the key pass)
  float* ent;
  // the query's deduplicated candidate list, one record per token (see RecLayout): written by the forward when not
  // null, read by the backward's query pass instead of its own gather and dedupe
  uint8_t* lists; int64_t rec;
  // forward outputs
  float* salida; float* signals;
  // backward
  const float* dsal; float* dphi; float* dV; float* dQc; float* dKc; double* dBt; float* dla; float* partials;
  // generation: per-bucket rings (B*T, 2^nb, C) of positions and their counts (B*T, 2^nb); the query position tq,
  // its bucket ids (B, T) out, and whether tq then enters the rings
  int32_t* rings; int32_t* counts; int32_t* ids_out; int nb; int64_t tq; int insert;
  const int64_t* tq_dev;   // generation, optional: the query position read from device memory instead of tq
  int32_t* done;           // generation, optional: per batch row, the column workgroups past their ring reads (0
                           // between launches): the launch then splits each row's columns over several workgroups
  // the unprotected core layer (v89 numerics): clock32 forms each score's clock term as (log_alfa_k + rate B_k) -
  // rate B_q in fp32 from the fp32 clock (held in Bt as fp64 values that fp32 represents exactly); leak, when given,
  // counts the (query, table) pairs whose best valid score is within the -1e9 fill's reach, where the reference's
  // fill gives its invalid keys weight
  int clock32; int32_t* leak;
  // ceil(2^64 / L) (0 when L = 1): a token index's batch row is the high half of its 64-bit product with this
  uint64_t Linv;
  // > 0: the XCDs take one batch row at a time, XCD x the positions [x slice, (x + 1) slice) of it (L = 8 slice)
  int64_t slice;
  // generation with the repetition step in the same launch (asrn_decode_attend_repeat): the step's arguments; the
  // query's clock is then formed from Bt[t - 1] and the step's beta (clock_at) instead of read from Bt[t]
  Step rep; Table rep_tab;
};

// i / L for 0 <= i < 2^32: the high half of i * ceil(2^64 / L) (the product exceeds i * 2^64 / L by less than
// i / L * L / 2^64 < 2^-32 <= 1 / L, which cannot carry the quotient past its floor)
__device__ __forceinline__ int64_t row_of(const Cand& a, int64_t i) {
  return a.Linv ? (int64_t)__umul64hi((uint64_t)i, a.Linv) : i;
}

// per-wave LDS scratch: one token's candidate list (entries) and its distinct positions (uniques)
constexpr int kHash = 3 * kMaxSlots / 2;   // dedupe hash slots: at most kMaxSlots distinct positions (load <= 2/3)

struct alignas(16) Scratch {
  int key[kMaxSlots];      // entry: (position << 5) | table
  uint8_t uid[kMaxSlots];  // entry -> unique (fewer than kMaxSlots = 256)
  int upos[kMaxSlots];     // unique: position
  union {
    struct {
      float ua[kMaxSlots];   // unique: base score, then (base + w_suf[ell]) + log_alfa_k; per entry in the backward
      float ub[kMaxSlots];   // unique: fp32(Bt_k - Bt_q)
      float uc[kMaxSlots];   // unique: sum over tables of att (forward, key side) or dp (query side)
    };
    struct {                 // the dedupe's hash table, dead once the uniques are numbered
      int hpos[kHash];       // position held by the slot (-1 empty)
      int hfirst[kHash];     // the first entry (table-major) with that position
    };
  };
  uint8_t uell[kMaxSlots]; // unique: suffix-match length (query side)
  int off[35];             // entries of table tau: [off[tau], off[tau + 1]) (T <= 32); table tau's window length
                           // is off[tau + 1] - off[tau]
  float bq32;              // clock32: the query's fp32 clock
  union {
    int wrank[32];         // per table: the token's sorted rank (the gather)
    float tinv[32];        // per table: 1 / softmax denominator (the forward's weights, after the gather)
  };
  float tsum[32];          // per-table sums (backward); per-table max keys (forward)
};
// 5.9 KB of LDS per wave. The backward's per-unique sums of ds reuse a per-unique array its pass no
// longer needs (uc in the query pass once dp is in registers, ub in the key pass, which has no clock differences).

// order-preserving map of finite floats and -inf to unsigned keys, and back
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_order_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup i runs on XCD i % 8), each with its own L2. Give
// each XCD a contiguous range of tokens instead, so one XCD's L2 serves one stretch of a batch row (at B = 8, one
// whole row) and candidates, which are earlier positions of the same row, hit there. The tail that does not divide
// evenly keeps the identity mapping.
// When the rows of all the batch rows that run at once outgrow the chip's 256 MB last-level cache (cfg3: 4 rows of
// 65,536 positions, 335 MB), a.slice > 0 turns the mapping row-wise instead: all eight XCDs work on one batch row at a
// time, XCD x on the x-th eighth of it, so the rows the waves gather (earlier positions of that one row) stay in the
// last-level cache that the XCDs share.
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t token_of_wave(const Cand& a) {
  const int64_t n = gridDim.x, i = blockIdx.x;
  int64_t blk = i;
  if (a.slice > 0) {
    const int64_t x = i % kXcds, j = i / kXcds;             // the j-th wave of XCD x
    if (i < a.B * a.L) {
      const int64_t b = j / a.slice;
      return b * a.L + x * a.slice + (j - b * a.slice);
    }
    return i;
  }
  const int64_t per = n / kXcds;
  if (i < per * kXcds) blk = (i % kXcds) * per + i / kXcds;
  return blk * kWavesPerBlock + (threadIdx.x >> 6);
}

// The whole-text kernels take their tokens in one table's sorted order (table ASRN_SORTED_TABLE, the last one when
// negative): the waves that run together on an XCD are then mostly mates of a few buckets, whose candidate lists
// overlap, instead of a stretch of positions whose candidates spread over the whole row, so L2 keeps their rows.
#ifndef ASRN_SORTED_MAP
#define ASRN_SORTED_MAP 1
#endif
#ifndef ASRN_SORTED_TABLE
#define ASRN_SORTED_TABLE 0
#endif
struct TokAt { int64_t b, t, tok; };   // batch row, position, b * L + t (tok < 0: past the end); wave-uniform
__device__ __forceinline__ TokAt sorted_token_of_wave(const Cand& a);

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
// rows stored as fp32 or as bf16 (B16; the value rows V and dO, and the feature rows phi, Qc, Kc): `base` points at
// element 0 of a row block, offsets count elements; a bf16 row's 4 elements load as 8 bytes and widen exactly (bf16 ->
// fp32 shifts the bits), so the results equal those from fp32 copies
template <bool B16>
__device__ __forceinline__ const float* rows_at(const float* base, int64_t elems) {
  if constexpr (B16) return reinterpret_cast<const float*>(reinterpret_cast<const uint16_t*>(base) + elems);
  else return base + elems;
}
template <bool B16>
__device__ __forceinline__ float4 ld4r(const float* base, uint32_t off) {
  if constexpr (B16) {
    const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(base) + off);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
  } else {
    return ld4(base + off);
  }
}
// 4 bf16 values (8 bytes) at element `off` of a bf16 row, as two packed pairs
__device__ __forceinline__ uint2 ld_bf16x4(const float* base, uint32_t off) {
  return *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(base) + off);
}
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// acc + <x, y> over 4 bf16 pairs: exact products, fp32 sums (v_dot2c_f32_bf16)
__device__ __forceinline__ float dot_bf16x4(uint2 x, uint2 y, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.x), __builtin_bit_cast(bf16x2, y.x), acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.y), __builtin_bit_cast(bf16x2, y.y), acc, false);
}

// 4 values stored at element `off` of an fp32 or bf16 (B16: rounded to nearest even, as a cast to bfloat16 does) row
__device__ __forceinline__ uint32_t bf16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;        // NaN stays a (quiet) NaN
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
template <bool B16>
__device__ __forceinline__ void st4r(float* base, int64_t off, const float4& v) {
  if constexpr (B16) {
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(base) + off) =
        make_uint2(bf16_bits(v.x) | (bf16_bits(v.y) << 16), bf16_bits(v.z) | (bf16_bits(v.w) << 16));
  } else {
    *reinterpret_cast<float4*>(base + off) = v;
  }
}
__device__ __forceinline__ float dot4(const float4& x, const float4& y) {
  return x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
}
__device__ __forceinline__ void fma4(float4& acc, float w, const float4& v) {
  acc.x += w * v.x; acc.y += w * v.y; acc.z += w * v.z; acc.w += w * v.w;
}
__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// The feature row a lane reads: float4 chunk c covers features x = 128 c + 4 (lane & 31) .. + 3 of [phi ; conf] (conf
// = Qc for queries, Kc for keys), pre-scaled by scale_phi / scale_c for queries. P and cf are multiples of 4, so a
// chunk never straddles the two. The per-lane base, stride and scale are fixed for a kernel: a row costs one 32-bit
// multiply and one float4 load (offsets fit 31 bits; lanes past P + cf read column 0 and are zeroed by their scale).
template <int F4>
struct FeatLanes {
  const float* base[F4];
  uint32_t stride[F4];
  float scale[F4];
};

template <int F4, bool FB16 = false>
__device__ __forceinline__ FeatLanes<F4> feat_lanes(const Cand& a, const float* conf, bool scaled) {
  FeatLanes<F4> fl;
  const int x0 = 4 * (lane_id() & 31);
#pragma unroll
  for (int c = 0; c < F4; ++c) {
    const int x = x0 + 128 * c;
    const bool in_phi = x < a.P, live = x < a.P + a.cf;
    fl.base[c] = in_phi ? rows_at<FB16>(a.phi, x) : (live ? rows_at<FB16>(conf, x - a.P) : a.phi);
    fl.stride[c] = in_phi || !live ? (uint32_t)a.P : (uint32_t)a.ldq;
    fl.scale[c] = !live ? 0.f : (scaled ? (in_phi ? a.sp : a.sc) : 1.f);
  }
  return fl;
}

// scaled: times the lane's scale (the query's own row; also zeroes the lanes past P + cf). Rows read unscaled meet
// such a row in a product, whose dead lanes are then zero, or are summed with weights and scaled once at the end.
template <int F4, bool FB16 = false>
__device__ __forceinline__ void feat_row(const FeatLanes<F4>& fl, uint32_t row, float4 (&f)[F4], bool scaled = true) {
#pragma unroll
  for (int c = 0; c < F4; ++c) {
    float4 v = ld4r<FB16>(fl.base[c], row * fl.stride[c]);
    if (scaled) {
      v.x *= fl.scale[c]; v.y *= fl.scale[c]; v.z *= fl.scale[c]; v.w *= fl.scale[c];
    }
    f[c] = v;
  }
}

// Runs body(n, u0) over the chunks [u0, u0 + n) of [first, NU), one every `step`: n is NF, or the smallest of
// N2 >= N3 that covers what is left, so a short tail does not load a full chunk of idle rows (n is a compile-time
// constant: the row arrays stay in registers). By default N2 = NF / 2 and N3 = NF / 4; NF = 12 takes 8 and 4.
template <int NF, int N2 = (NF % 3 == 0 ? 2 * NF / 3 : (NF >= 2 ? NF / 2 : 1)),
          int N3 = (NF % 3 == 0 ? NF / 3 : (NF >= 4 ? NF / 4 : 1)), class F>
__device__ __forceinline__ void for_chunks(int first, int NU, int step, F&& body) {
  for (int u0 = first; u0 < NU; u0 += step) {
    const int rem = NU - u0;
    if (rem > N2) body(std::integral_constant<int, NF>{}, u0);
    else if (rem > N3) body(std::integral_constant<int, N2>{}, u0);
    else body(std::integral_constant<int, N3>{}, u0);
  }
}

// the sums of the two 32-lane halves land in lane 16 (lanes 0-31) and lane 48 (lanes 32-63); the other lanes hold
// partial sums. Adds row 0 + row 1 and row 2 + row 3 of the 16-lane row sums, as readlane sums would.
__device__ __forceinline__ float half_sums_at_16_48(float v) {
  v = row_sum16(v);
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));  // row_bcast:15
}

template <int F4>
__device__ __forceinline__ float dot_f(const float4 (&q)[F4], const float4 (&k)[F4]) {
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < F4; ++c) s += dot4(q[c], k[c]);
  return s;
}

__device__ __forceinline__ float rate_of(const Cand& a, int tau) { return a.gamma[tau] / (float)a.C; }

// Per-table sums over the candidate entries, which are grouped by table (entries [off[tau], off[tau+1]) of table tau):
// each table gets G = 64 / (T rounded up to a power of two) lanes, which stride through its entries and then add up
// in a fixed butterfly. Deterministic, and no lane walks a whole table alone. Every lane of table tau's group (lanes
// tau*G .. tau*G + G - 1) returns its sum.
__device__ __forceinline__ int lanes_per_table(int T) {
  int tp = 1;
  while (tp < T) tp <<= 1;
  return kWave / tp;
}
template <class F>
__device__ __forceinline__ float table_sum(const Scratch& S, int T, int G, F val) {
  const int lane = lane_id(), tau = lane / G;
  float s = 0.f;
  if (tau < T)
    for (int m = S.off[tau] + lane % G; m < S.off[tau + 1]; m += G) s += val(m);
  for (int x = G >> 1; x > 0; x >>= 1) s += __shfl_xor(s, x, kWave);
  return s;
}

// Suffix match of `other` against the token itself: the number of leading j < K with sig[other - 1 - j] ==
// sig[self - 1 - j], both in range; NaN never matches (reference nucleo:98-108, 313-320). The reference's K = 4 keeps
// the token's own four previous signatures in registers (`mine`, uniform across the wave); K up to 16 reads both sides.
__device__ __forceinline__ void own_suffix_of(const float* __restrict__ sigb, int64_t self_pos, int K,
                                              float (&mine)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) mine[j] = (j < K && self_pos - 1 - j >= 0) ? sigb[self_pos - 1 - j] : 0.f;
}

__device__ __forceinline__ int suffix_len_of(const float* __restrict__ sigb, const float (&mine)[4], int64_t self_pos,
                                            int64_t other, int K) {
  int ell = 0;
  bool run = true;
  if (K <= 4) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t io = other - 1 - j;
      v[j] = sigb[io >= 0 ? io : 0];               // every load in flight at once
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      run = run && j < K && other - 1 - j >= 0 && self_pos - 1 - j >= 0 && v[j] == mine[j];
      ell += run ? 1 : 0;
    }
    return ell;
  }
  for (int j = 0; j < K && run; ++j) {
    const int64_t io = other - 1 - j, is = self_pos - 1 - j;
    run = io >= 0 && is >= 0 && sigb[io] == sigb[is];
    ell += run ? 1 : 0;
  }
  return ell;
}

// What a unique's score terms read from memory, by its position k: the tokens before it (its suffix, K <= 4), its clock
// and its log_alfa; loaded ahead of their use (unique_terms)
struct UniqueAt {
  int64_t k;
  float s[4];
  double bk;
  float la;
};
// unique u's (u < NU; past NU, the last unique's; with no uniques, position self_pos's, never used)
__device__ __forceinline__ UniqueAt unique_at(const Cand& a, int64_t b, const Scratch& S, int NU, int u,
                                              const float* __restrict__ sigb, int64_t self_pos) {
  UniqueAt x;
  x.k = NU > 0 ? S.upos[u < NU ? u : NU - 1] : self_pos;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t io = x.k - 1 - j;
    x.s[j] = sigb[io >= 0 ? io : 0];
  }
  x.bk = a.Bt[b * a.L + x.k];
  x.la = a.la[b * a.L + x.k];
  return x;
}
// suffix_len_of for K <= 4 on the loaded tokens (the same comparisons)
__device__ __forceinline__ int suffix_len4(const UniqueAt& x, const float (&mine)[4], int64_t self_pos, int K) {
  int ell = 0;
  bool run = true;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    run = run && j < K && x.k - 1 - j >= 0 && self_pos - 1 - j >= 0 && x.s[j] == mine[j];
    ell += run ? 1 : 0;
  }
  return ell;
}

// Packs every table's window of token (b, t) into S.key and the table segments into S.off. query_window: the
// `win & 255` sorted ranks before the token's; otherwise (the key pass) the `win >> 8` after it. The segment offsets
// are a prefix sum of the window lengths, so entry m finds its table by a binary search over T offsets and one round
// of `order` loads fills the list, table-major and oldest first. Returns the count M.
__device__ __forceinline__ int gather(const Cand& a, int64_t b, int64_t t, bool query_window, Scratch& S) {
  const int lane = lane_id();
  int s = 0, n = 0;
  if (lane < a.T) {
    const uint32_t o = (uint32_t)((b * a.L + t) * a.T) + (uint32_t)lane;   // B L T < 2^31 (check_args)
    s = a.rank[o];
    const int w = a.win[o];
    n = query_window ? (w & 255) : ((w >> 8) & 255);
  }
  int off = 0, M = 0;
  for (int tt = 0; tt < a.T; ++tt) {
    const int nt = readlane_i(n, tt);
    if (lane == tt) off = M;
    M += nt;
  }
  if (lane < a.T) {
    S.off[lane] = off;
    S.wrank[lane] = s;
  }
  if (lane == 0) S.off[a.T] = M;
  wave_lds_sync();
  for (int m0 = 0; m0 < M; m0 += kWave) {
    const int m = m0 + lane;
    if (m < M) {
      int lo = 0, hi = a.T - 1;                  // the last table whose segment starts at or before m
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (S.off[mid] <= m) lo = mid; else hi = mid - 1;
      }
      const int i = m - S.off[lo];
      // query window: ranks s - n .. s - 1; key window: s + 1 .. s + n (in range by construction; clamped so that
      // inconsistent inputs cannot read out of bounds)
      int j = query_window ? S.wrank[lo] - (S.off[lo + 1] - S.off[lo]) + i : S.wrank[lo] + 1 + i;
      j = j < 0 ? 0 : (j >= a.L ? (int)a.L - 1 : j);
      int pos = a.order[(uint32_t)((b * a.T) * a.L) + (uint32_t)lo * (uint32_t)a.L + (uint32_t)j];
      pos = pos < 0 ? 0 : (pos >= a.L ? (int)a.L - 1 : pos);          // a position whatever the sort left
      S.key[m] = (pos << 5) | lo;
    }
  }
  wave_lds_sync();
  return M;
}

// Generation: the candidates of position t are the ring contents of its bucket in every table, oldest first. The
// bucket ids come from the signs of the query's own hash outputs (written to ids_out for the ring insert).
__device__ __forceinline__ int gather_rings(const Cand& a, int64_t b, int64_t t, Scratch& S) {
  const int lane = lane_id();
  // the query's bucket id in each table from the signs of its phi row (strict > 0, nucleo:663): the whole row in one
  // round of loads (element c * 64 + lane; P = T nb <= 255), then table `lane`'s nb bits out of the ballots
  const float* ph = a.phi + (b * a.L + t) * a.P;
  float hv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {                   // unconditional loads (lanes past P read element P - 1), so all
    const int e = c * kWave + lane;               // four are in flight before the first ballot waits
    hv[c] = ph[e < a.P ? e : a.P - 1];
  }
  uint64_t pm[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) pm[c] = __ballot(c * kWave + lane < a.P && hv[c] > 0.f);
  int id = 0;
  if (lane < a.T) {
    const int e0 = lane * a.nb, w = e0 >> 6, o = e0 & 63;
    const uint64_t lo = w == 0 ? pm[0] : (w == 1 ? pm[1] : (w == 2 ? pm[2] : pm[3]));
    uint64_t bits = lo >> o;
    if (o + a.nb > 64) bits |= (w == 0 ? pm[1] : (w == 1 ? pm[2] : pm[3])) << (64 - o);   // w <= 2 here
    id = (int)(bits & ((1ull << a.nb) - 1ull));
    a.ids_out[b * a.T + lane] = id;
  }
  // one round of loads: each bucket's count and every slot of its ring, whose addresses need only the ids; the slots
  // go to LDS (the dedupe's hash array, dead until dedupe clears it) and each entry then takes its slot oldest first
  const int cnt = lane < a.T ? a.counts[(b * a.T + lane) * ((int64_t)1 << a.nb) + id] : 0;
  const int slots = a.T * a.C;
  static_assert(kHash >= kMaxSlots, "the ring slots are staged in the dedupe's hash array");
  int raw[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int sl = c * kWave + lane;
    const int tau = sl < slots ? sl / a.C : 0;
    const int idt = __shfl(id, tau, 64);
    raw[c] = sl < slots ? a.rings[((b * a.T + tau) * ((int64_t)1 << a.nb) + idt) * a.C + (sl - tau * a.C)] : -1;
  }
#pragma unroll
  for (int c = 0; c < kCh; ++c)
    if (c * kWave + lane < slots) S.hpos[c * kWave + lane] = raw[c];
  wave_lds_sync();
  int pos[kCh], tt[kCh];
  bool ok[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int sl = c * kWave + lane;
    const int tau = sl < slots ? sl / a.C : 0;
    const int i = sl - tau * a.C;
    const int ct = __shfl(cnt, tau, 64);
    const int n = ct < a.C ? ct : a.C;              // filled slots
    const int start = ct < a.C ? 0 : ct % a.C;     // the oldest entry
    const bool v = sl < slots && i < n;
    const int slot = start + i < a.C ? start + i : start + i - a.C;
    const int p = v ? S.hpos[tau * a.C + slot] : -1;
    ok[c] = v && p >= 0 && p < t;
    tt[c] = tau;
    pos[c] = ok[c] ? p : 0;
  }
  int base = 0;
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const uint64_t bal = __ballot(ok[c]);
    if (ok[c]) S.key[base + __popcll(bal & ((1ull << lane) - 1ull))] = (pos[c] << 5) | tt[c];
    base += __popcll(bal);
  }
  wave_lds_sync();
  if (lane <= a.T) {
    int lo = 0, hi = base;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((S.key[mid] & 31) < lane) lo = mid + 1; else hi = mid;
    }
    S.off[lane] = lo;
  }
  wave_lds_sync();
  return base;
}

// One slot per distinct position, in order of first appearance (table-major): S.uid[entry], S.upos[unique].
// Every entry claims its position's slot in an LDS hash table (compare-and-swap, linear probing) and keeps the
// smallest entry index there (atomic min, order-independent), so the numbering is deterministic.
// a slot in [0, kHash): the high part of (Knuth's multiplicative hash) * kHash
__device__ __forceinline__ uint32_t pos_hash(int pos, uint32_t slots) {
  return __umulhi((uint32_t)pos * 2654435761u, slots);
}

__device__ __forceinline__ int dedupe(const Cand& a, int M, Scratch& S) {
  const int lane = lane_id();
  const uint32_t hs = M <= kWave ? 2 * kWave : kHash;   // slots in use: load <= 1/2 for lists of up to 64 entries
  for (int i = lane; i < (int)hs; i += kWave) {
    S.hpos[i] = -1;
    S.hfirst[i] = 0x7fffffff;
  }
  wave_lds_sync();
  int slot[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    slot[c] = 0;
    const int m = c * kWave + lane;
    if (c * kWave < M && m < M) {
      const int pos = S.key[m] >> 5;
      uint32_t h = pos_hash(pos, hs);
      for (uint32_t probe = 0; probe < hs; ++probe) {
        const int old = atomicCAS(&S.hpos[h], -1, pos);
        if (old == -1 || old == pos) break;
        h = h + 1 == hs ? 0u : h + 1;
      }
      atomicMin(&S.hfirst[h], m);
      slot[c] = (int)h;
    }
  }
  wave_lds_sync();
  int nu = 0;
  bool prim[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int m = c * kWave + lane;
    prim[c] = false;
    if (c * kWave < M) {
      prim[c] = m < M && S.hfirst[slot[c]] == m;
      const uint64_t bal = __ballot(prim[c]);
      if (prim[c]) {
        const int u = nu + __popcll(bal & ((1ull << lane) - 1ull));
        S.uid[m] = (uint8_t)u;
        S.upos[u] = S.key[m] >> 5;
      }
      nu += __popcll(bal);
    }
  }
  wave_lds_sync();
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int m = c * kWave + lane;
    if (m < M && !prim[c]) S.uid[m] = S.uid[S.hfirst[slot[c]]];
  }
  wave_lds_sync();
  return nu;
}

// (In these helpers self_pos is the token's own position inside batch row b: the row idle lanes read.)
//
// base scores <query, key> of every unique, 2*kRows rows in flight (kRows per half-wave). query side: fixed = the
// query's scaled features and the rows are keys; key side: fixed = the key's raw features, rows = queries (scaled).
// The product is always query * key and the reduction tree is the same, so both sides produce the same bits.
template <int F4, bool FB16 = false>
__device__ __forceinline__ void unique_bases(const Cand& a, int64_t b, int64_t self_pos, int NU,
                                             bool rows_are_queries, const float4 (&fixed)[F4], Scratch& S,
                                             int first = 0, int step = 2 * kRows) {
  const int lane = lane_id(), half = lane >> 5;
  const FeatLanes<F4> fl = feat_lanes<F4, FB16>(a, rows_are_queries ? a.Qc : a.Kc, rows_are_queries);
  const uint32_t row0 = (uint32_t)(b * a.L);
  // the fixed side's dead lanes are zero when it is the query's scaled row; key rows then need no scaling
  const bool scale_rows = rows_are_queries;
  for_chunks<2 * kRows>(first, NU, step, [&](auto n, int u0) {
    constexpr int R = decltype(n)::value / 2;          // rows per half-wave
    int pos[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {                      // every position read before any row load
      const int u = u0 + 2 * r + half;
      pos[r] = S.upos[u < NU ? u : NU - 1];
    }
    float4 f[R][F4];
#pragma unroll
    for (int r = 0; r < R; ++r) feat_row<F4, FB16>(fl, row0 + (uint32_t)pos[r], f[r], scale_rows);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float h = half_sums_at_16_48(rows_are_queries ? dot_f(f[r], fixed) : dot_f(fixed, f[r]));
      const int u = u0 + 2 * r + half;
      if ((lane & 31) == 16 && u < NU) S.ua[u] = h;
    }
  });
  (void)self_pos;
  wave_lds_sync();
}

// The base scores with P + cf <= 128 (F4 == 1): each aligned group of 8 lanes (g = lane / 8, j = lane % 8) reads one
// candidate's [phi ; Kc] row, lane j holding features 32 k + 4 j .. + 3 of chunk k = 0..3. One load instruction then
// covers 128 contiguous bytes of each of 8 rows, a lane's 16 products need no cross-lane step until the group's
// 3-step DPP sum, and 16 rows cost 8 loads, 32 FMAs and 6 DPP adds per lane.
struct Feat8 {
  const float* base[4];   // per chunk: phi + f, conf + (f - P), or phi itself for dead lanes (f >= P + cf)
  bool conf[4];           // the chunk's rows have conf's stride ldq instead of P
  float scale[4];         // scale_phi, scale_c, or 0 past P + cf
};
template <bool FB16>
__device__ __forceinline__ Feat8 feat8(const Cand& a, const float* conf, bool scaled) {
  Feat8 fl;
  const int j = lane_id() & 7;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int f = 32 * k + 4 * j;
    const bool in_phi = f < a.P, live = f < a.P + a.cf;
    fl.base[k] = in_phi ? rows_at<FB16>(a.phi, f) : (live ? rows_at<FB16>(conf, f - a.P) : a.phi);
    fl.conf[k] = !in_phi && live;
    fl.scale[k] = !live ? 0.f : (scaled ? (in_phi ? a.sp : a.sc) : 1.f);
  }
  return fl;
}
template <bool FB16>
__device__ __forceinline__ void feat8_row(const Cand& a, const Feat8& fl, uint32_t row, float4 (&f)[4], bool scaled) {
  const uint32_t op = row * (uint32_t)a.P, oc = row * (uint32_t)a.ldq;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float4 v = ld4r<FB16>(fl.base[k], fl.conf[k] ? oc : op);
    if (scaled) {
      v.x *= fl.scale[k]; v.y *= fl.scale[k]; v.z *= fl.scale[k]; v.w *= fl.scale[k];
    }
    f[k] = v;
  }
}
// the sum over each aligned group of 8 lanes, in all 8 (pairs, then quads, then the half-row mirror adds the quads)
__device__ __forceinline__ float group8_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1032
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2301
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // half mirror
}
// query side of the base scores: S.ua[u] = <query's scaled [phi ; Qc], [phi_u ; Kc_u]> for the uniques of chunks of
// 16 starting at `first`, one every `step`
template <bool FB16>
__device__ __forceinline__ void unique_bases8(const Cand& a, int64_t b, int64_t tok, int NU, Scratch& S, int first,
                                              int step) {
  const int lane = lane_id(), g = lane >> 3;
  const Feat8 fq = feat8<FB16>(a, a.Qc, true);
  const Feat8 fl = feat8<FB16>(a, a.Kc, false);
  const uint32_t row0 = (uint32_t)(b * a.L);
  // fp32 rows: the query's features pre-scaled. bf16 rows: the query's stay packed, each chunk's v_dot2c products
  // then take the chunk's scale (scale_phi, scale_c, or 0 past P + cf: a chunk lies in one of the two)
  float4 q[4];
  uint2 qb[4];
  if constexpr (FB16) {
    const uint32_t op = (uint32_t)tok * (uint32_t)a.P, oc = (uint32_t)tok * (uint32_t)a.ldq;
#pragma unroll
    for (int k = 0; k < 4; ++k) qb[k] = ld_bf16x4(fq.base[k], fq.conf[k] ? oc : op);
  } else {
    feat8_row<FB16>(a, fq, (uint32_t)tok, q, true);
  }
  for_chunks<16>(first, NU, step, [&](auto n, int u0) {
    constexpr int RG = decltype(n)::value >= 8 ? decltype(n)::value / 8 : 1;   // row groups of 8 in flight
    int pos[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {                     // every position read before any row load
      const int u = u0 + 8 * r + g;
      pos[r] = S.upos[u < NU ? u : NU - 1];
    }
    float p[RG];
    if constexpr (FB16) {
      uint2 f[RG][4];
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const uint32_t row = row0 + (uint32_t)pos[r];
        const uint32_t op = row * (uint32_t)a.P, oc = row * (uint32_t)a.ldq;
#pragma unroll
        for (int k = 0; k < 4; ++k) f[r][k] = ld_bf16x4(fl.base[k], fl.conf[k] ? oc : op);
      }
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        p[r] = fq.scale[0] * dot_bf16x4(qb[0], f[r][0], 0.f);
#pragma unroll
        for (int k = 1; k < 4; ++k) p[r] += fq.scale[k] * dot_bf16x4(qb[k], f[r][k], 0.f);
      }
    } else {
      float4 f[RG][4];
#pragma unroll
      for (int r = 0; r < RG; ++r) feat8_row<FB16>(a, fl, row0 + (uint32_t)pos[r], f[r], false);
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        p[r] = dot4(q[0], f[r][0]);
#pragma unroll
        for (int k = 1; k < 4; ++k) p[r] += dot4(q[k], f[r][k]);
      }
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const float pr = group8_sum(p[r]);
      const int u = u0 + 8 * r + g;
      if ((lane & 7) == 0 && u < NU) S.ua[u] = pr;
    }
  });
  wave_lds_sync();
}

// sum_u w_u * row_u over the uniques' features (kRows rows per half-wave in flight), both halves combined.
template <int F4, bool FB16 = false>
__device__ __forceinline__ void unique_feature_sum(const Cand& a, int64_t b, int64_t self_pos, int NU,
                                                   bool rows_are_queries, const float* wts, Scratch& S,
                                                   float4 (&g)[F4]) {
  const int half = lane_id() >> 5;
  const FeatLanes<F4> fl = feat_lanes<F4, FB16>(a, rows_are_queries ? a.Qc : a.Kc, rows_are_queries);
  const uint32_t row0 = (uint32_t)(b * a.L);
#pragma unroll
  for (int c = 0; c < F4; ++c) g[c] = zero4();
  for_chunks<2 * kRows>(0, NU, 2 * kRows, [&](auto n, int u0) {
    constexpr int R = decltype(n)::value / 2;          // rows per half-wave
    int pos[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {                      // every position read before any row load
      const int u = u0 + 2 * r + half;
      pos[r] = S.upos[u < NU ? u : NU - 1];
    }
    float4 f[R][F4];
#pragma unroll
    for (int r = 0; r < R; ++r) feat_row<F4, FB16>(fl, row0 + (uint32_t)pos[r], f[r], false);
#pragma unroll
    for (int r = 0; r < R; ++r) {                      // the weights, read while the rows are in flight
      const int u = u0 + 2 * r + half;
      float w = wts[u < NU ? u : NU - 1];
      w = u < NU ? w : 0.f;
#pragma unroll
      for (int c = 0; c < F4; ++c) fma4(g[c], w, f[r][c]);
    }
  });
#pragma unroll
  for (int c = 0; c < F4; ++c) {   // both halves combined, then the lane's scale (zero past P + cf) once
    g[c].x = (g[c].x + __shfl_xor(g[c].x, 32, 64)) * fl.scale[c];
    g[c].y = (g[c].y + __shfl_xor(g[c].y, 32, 64)) * fl.scale[c];
    g[c].z = (g[c].z + __shfl_xor(g[c].z, 32, 64)) * fl.scale[c];
    g[c].w = (g[c].w + __shfl_xor(g[c].w, 32, 64)) * fl.scale[c];
  }
  (void)self_pos;
}

// Widths past 256 * DCH (d > 1024) run the value phases over column slabs of 256 * DCH: columns c0 .. c0 + 256 DCH - 1
// of every row in one pass, the lanes past d reading column d - 4 (a real column; their results are not used).
__device__ __forceinline__ int slab_col(const Cand& a, int c0, int ch, int lane) {
  const int dd = c0 + ch * 256 + lane * 4;
  return dd < a.d ? dd : a.d - 4;
}

// <fixed, row_u> over the d columns for every unique (rows of batch row `rows`), R rows in flight, written to
// out[u] (added to it when `add`: the slabs after the first); the key side (w_u != nullptr) also accumulates
// dV += w_u row_u from the same loads. fixed holds columns c0 .. c0 + 256 DCH - 1 (zero past d).
// The wave totals of N = 2, 4 or 8 per-lane values at once, by a transposing butterfly: at distances 32 (N >= 2), 16
// (N >= 4) and 8 (N = 8) each lane keeps half of its values and adds its partner's copies of them, so one value is
// left per lane, value (lane >> (6 - log2 N)) & (N - 1); the lanes that hold it (aligned groups of 64 / N) then add it
// up with DPP steps. Returns that total; wave_sums_lead(N) says which lane writes value i: about 30 VALU and 6
// LDS-pipe exchanges for 8 totals, against 8 separate wave sums.
template <int N>
__device__ __forceinline__ float wave_sums(const float (&v)[N]) {
  static_assert(N == 2 || N == 4 || N == 8, "2, 4 or 8 values");
  const int lane = lane_id();
  const bool h32 = lane & 32;
  float a[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i)
    a[i] = (h32 ? v[N / 2 + i] : v[i]) + __shfl_xor(h32 ? v[i] : v[N / 2 + i], 32, kWave);
  if constexpr (N == 2) {                     // halves of 32: the row sums, then row 1 (3) adds row 0 (2)
    const float x = row_sum16(a[0]);
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xA, 0xF, false));
  } else {
    const bool h16 = lane & 16;
    float c[N / 4];
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
      c[i] = (h16 ? a[N / 4 + i] : a[i]) + __shfl_xor(h16 ? a[i] : a[N / 4 + i], 16, kWave);
    if constexpr (N == 4) {
      return row_sum16(c[0]);
    } else {
      const bool h8 = lane & 8;
      const float send = h8 ? c[0] : c[1];
      const float x = (h8 ? c[1] : c[0]) +
                      __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x128, 0xF, 0xF, false));
      return group8_sum(x);
    }
  }
}
// the value wave_sums<N> leaves in this lane, and whether this lane is the one that writes it
template <int N>
__device__ __forceinline__ int wave_sums_index() { return (lane_id() >> (N == 8 ? 3 : (N == 4 ? 4 : 5))) & (N - 1); }
template <int N>
__device__ __forceinline__ bool wave_sums_lead() {
  const int lane = lane_id();
  return N == 8 ? (lane & 7) == 0 : (N == 4 ? (lane & 15) == 0 : (lane & 31) == 16);
}

// out[u] = <fixed row, row_u> over columns c0 .. c0 + 256 DCH - 1 for every unique (rows of batch row `rows`), NF rows
// in flight and their dot products reduced together (wave_sums); added to out[u] when `add` (the slabs after the
// first). `fixed` is the fixed row's element 0 (dO of the query); past d both sides read column d - 4 and the fixed
// side is zeroed. bf16 rows (B16) stay packed: v_dot2c_f32_bf16 takes both sides as they are stored.
template <int DCH, bool B16 = false>
__device__ __forceinline__ void unique_row_dots(const Cand& a, const float* rows, int64_t ld, int NU,
                                                const float* fixed, Scratch& S, float* out, int c0 = 0,
                                                bool add = false) {
  const int lane = lane_id();
  constexpr int NF = DCH >= 3 ? 2 : (DCH == 2 ? 4 : 8);
  int col[DCH];
  using Q = typename std::conditional<B16, uint2, float4>::type;
  Q fq[DCH];
#pragma unroll
  for (int ch = 0; ch < DCH; ++ch) {
    col[ch] = slab_col(a, c0, ch, lane);
    const bool live = c0 + ch * 256 + lane * 4 < a.d;
    if constexpr (B16) fq[ch] = live ? ld_bf16x4(fixed, (uint32_t)col[ch]) : make_uint2(0u, 0u);
    else fq[ch] = live ? ld4(fixed + col[ch]) : zero4();
  }
  for_chunks<NF>(0, NU, NF, [&](auto n, int u0) {
    constexpr int R = decltype(n)::value;
    int p[R];
#pragma unroll
    for (int r = 0; r < R; ++r)                        // wave-uniform rows: their offsets are scalar arithmetic
      p[r] = __builtin_amdgcn_readfirstlane(S.upos[u0 + r < NU ? u0 + r : NU - 1]);
    Q o[R][DCH];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float* row = rows_at<B16>(rows, (int64_t)(uint32_t)p[r] * ld);
#pragma unroll
      for (int ch = 0; ch < DCH; ++ch) {
        if constexpr (B16) o[r][ch] = ld_bf16x4(row, (uint32_t)col[ch]);
        else o[r][ch] = ld4(row + col[ch]);
      }
    }
    float q[NF];
#pragma unroll
    for (int r = 0; r < NF; ++r) {
      q[r] = 0.f;
      if (r < R) {
#pragma unroll
        for (int ch = 0; ch < DCH; ++ch) {
          if constexpr (B16) q[r] = dot_bf16x4(o[r][ch], fq[ch], q[r]);
          else q[r] += dot4(o[r][ch], fq[ch]);
        }
      }
    }
    const float tot = wave_sums<NF>(q);
    const int r = wave_sums_index<NF>(), u = u0 + r;
    if (wave_sums_lead<NF>() && r < R && u < NU) out[u] = add ? out[u] + tot : tot;
  });
  wave_lds_sync();
}

// Per unique, the sums over tables of NV per-entry values, in table order: out[v][u] = the sum, tables ascending, of
// val[v][c] over the entries c * 64 + lane of unique u (tau[c] < 0: no entry; a unique appears at most once in a
// table). Each pass zeroes a cell per (unique, value, table) for the uniques [u0, u0 + per) in `slots` (nslot floats of
// LDS that are dead during the call, 16-byte aligned), every entry writes its cell, then lane u adds its cells in
// table order (the absent tables' cells add exact zeros, so the sums equal those of a table-by-table loop).
template <int NV>
__device__ __forceinline__ void unique_table_sums(int T, int NU, const int (&tau)[kCh], const int (&un)[kCh],
                                                  const float (&val)[NV][kCh], float* slots, int nslot,
                                                  float* const (&out)[NV]) {
  const int lane = lane_id();
  int tp = 4;                                   // cells per (unique, value): T rounded up to a power of 2, >= 4
  while (tp < T) tp <<= 1;
  const int per = nslot / (tp * NV);
  wave_lds_sync();                              // the slots' earlier readers are done
  for (int u0 = 0; u0 < NU; u0 += per) {
    for (int i = 4 * lane; i < per * tp * NV; i += 4 * kWave) *reinterpret_cast<float4*>(slots + i) = zero4();
    wave_lds_sync();
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const int u = un[c] - u0;
      if (tau[c] >= 0 && u >= 0 && u < per) {
#pragma unroll
        for (int v = 0; v < NV; ++v) slots[(u * NV + v) * tp + tau[c]] = val[v][c];
      }
    }
    wave_lds_sync();
    for (int u = u0 + lane; u < NU && u < u0 + per; u += kWave) {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const float* cell = slots + ((u - u0) * NV + v) * tp;
        float acc = 0.f;
        for (int t4 = 0; t4 < tp; t4 += 4) {
          const float4 q = *reinterpret_cast<const float4*>(cell + t4);
          acc += q.x; acc += q.y; acc += q.z; acc += q.w;
        }
        out[v][u] = acc;
      }
    }
    wave_lds_sync();
  }
}

// Entries of the candidate list held one per lane (entry c*64 + lane in chunk c).
struct Entries {
  int u[kCh];        // unique of the entry
  int tau[kCh];      // table (-1 when the slot is empty)
  float sc[kCh];     // score
};

// The entries' scores: S.ua[u] + rate * S.ub[u] (the clock difference); with clock32, in the reference's fp32 order
// and roundings ((base + w_suf) + (log_alfa_k + rate B_k)) - rate B_q, from S.ua = base + w_suf, S.uc = log_alfa_k and
// S.ub = B_k (nucleo:330-332: no fused multiply-add, each product and sum rounded on its own).
__device__ __forceinline__ void load_entries(const Cand& a, int M, const Scratch& S, Entries& E) {
  const int lane = lane_id();
  const float rate_l = lane < a.T ? rate_of(a, lane) : 0.f;   // one division per table, shuffled to the entries
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int m = c * kWave + lane;
    const bool in = m < M;
    const int e = in ? S.key[m] : 0;
    E.tau[c] = in ? (e & 31) : -1;
    const int u = in ? S.uid[m] : 0;
    E.u[c] = u;
    const float r = __shfl(rate_l, e & 31, kWave);          // every lane takes part (no divergent shuffle)
    E.sc[c] = !in ? -INFINITY
                  : (a.clock32 ? __fsub_rn(__fadd_rn(S.ua[u], __fadd_rn(S.uc[u], __fmul_rn(r, S.ub[u]))),
                                           __fmul_rn(r, S.bq32))
                               : S.ua[u] + r * S.ub[u]);
  }
}

// A query's candidate list as the forward leaves it for the backward's query pass, at lists + token * rec (bytes):
//   header  (T + 2) u16: the table offsets off[0..T] (entries of table tau are [off[tau], off[tau + 1])), then NU
//   e16     per entry m < M = off[T]: its unique | table << 8
//   upos    per unique u < NU: the candidate's position (int32)
//   ub      per unique: fp32(Bt_k - Bt_q)
//   uell    per unique: the suffix-match length (u8)
// Every region is sized for T * C (the most entries and uniques a query can have); 16-byte aligned. (The entries' att
// stays in the entries array only: the query pass reads it there, next to the ds it writes, which keeps those lines
// in L2 for the key pass; a copy in the record made the key pass 6 us slower at cfg2.)
struct RecLayout { int64_t e16, upos, ub, uell, size; };
__host__ __device__ inline RecLayout rec_layout(int T, int C) {
  const int64_t tc = (int64_t)T * C;
  RecLayout r;
  r.e16 = 128;                                    // (T + 2) u16 <= 68 bytes
  r.upos = (r.e16 + 2 * tc + 15) / 16 * 16;
  r.ub = r.upos + 4 * tc;
  r.uell = r.ub + 4 * tc;
  r.size = (r.uell + tc + 15) / 16 * 16;
  return r;
}

// The query pass's view of a record: S.off, S.key (the table of each entry; the position part is not needed there),
// S.uid, S.upos, S.ub and S.uell. The first 64 entries and uniques are loaded with the header in one
// round (most queries have no more); loads past M or NU stay inside the record and are ignored.
__device__ __forceinline__ void load_record(const Cand& a, const uint8_t* rec, Scratch& S, int& M, int& NU) {
  const int lane = lane_id();
  const RecLayout R = rec_layout(a.T, a.C);
  const int tc = a.T * a.C;
  const uint16_t* hdr = reinterpret_cast<const uint16_t*>(rec);
  const uint16_t* e16 = reinterpret_cast<const uint16_t*>(rec + R.e16);
  const int32_t* upos = reinterpret_cast<const int32_t*>(rec + R.upos);
  const float* ub = reinterpret_cast<const float*>(rec + R.ub);
  const uint8_t* uell = rec + R.uell;
  const int i0 = lane < tc ? lane : 0;
  const int h = lane <= a.T + 1 ? (int)hdr[lane] : 0;
  const int e0 = e16[i0];
  const int p0 = upos[i0];
  const float b0 = ub[i0];
  const int l0 = uell[i0];
  M = readlane_i(h, a.T);
  NU = readlane_i(h, a.T + 1);
  if (lane <= a.T) S.off[lane] = h;
  if (lane < M) {
    S.key[lane] = e0 >> 8;
    S.uid[lane] = (uint8_t)(e0 & 255);
  }
  for (int m = kWave + lane; m < M; m += kWave) {
    const int e = e16[m];
    S.key[m] = e >> 8;
    S.uid[m] = (uint8_t)(e & 255);
  }
  if (lane < NU) {
    S.upos[lane] = p0;
    S.ub[lane] = b0;
    S.uell[lane] = (uint8_t)l0;
  }
  for (int u = kWave + lane; u < NU; u += kWave) {
    S.upos[u] = upos[u];
    S.ub[u] = ub[u];
    S.uell[u] = uell[u];
  }
  wave_lds_sync();
}

// ---------------------------------------------------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------------------------------------------------
// value rows in flight per wave in the copy-gather (the loads of one chunk)
template <int DCH>
constexpr int gather_rows_in_flight() { return DCH >= 4 ? 4 : (DCH >= 2 ? 8 : 12); }

// The copy-gather's rows: acc += sum over uniques u of (sum over tables of att) V_u, for u in chunks of UNR
// consecutive uniques starting at `first`, one chunk every `step` (UNR rows in flight per chunk).
template <int DCH, bool B16 = false>
__device__ __forceinline__ void gather_values(const Cand& a, int64_t b, const Scratch& S, int NU, int first, int step,
                                              float4 (&acc)[DCH], int c0 = 0) {
  constexpr int UNR = gather_rows_in_flight<DCH>();
  const int lane = lane_id();
  const float* Vb = rows_at<B16>(a.V, (b * a.L + a.vshift) * a.ldv);
  int col[DCH];
#pragma unroll
  for (int ch = 0; ch < DCH; ++ch) col[ch] = slab_col(a, c0, ch, lane);
  for_chunks<UNR>(first, NU, step, [&](auto n, int u0) {
    constexpr int R = decltype(n)::value;
    int p[R];
    float w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {                      // wave-uniform rows and weights: scalar offsets
      const int u = u0 + r < NU ? u0 + r : NU - 1;
      p[r] = __builtin_amdgcn_readfirstlane(S.upos[u]);
      w[r] = u0 + r < NU ? S.uc[u] : 0.f;            // the same in every lane (an LDS broadcast)
    }
    float4 v[R][DCH];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float* row = rows_at<B16>(Vb, (int64_t)(uint32_t)p[r] * a.ldv);
#pragma unroll
      for (int ch = 0; ch < DCH; ++ch) v[r][ch] = ld4r<B16>(row, (uint32_t)col[ch]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int ch = 0; ch < DCH; ++ch) fma4(acc[ch], w[r], v[r][ch]);
  });
}

// A query token's candidate list (gather and dedupe; the record's header and entries when it is kept): returns the
// entry count M, and the unique count NU in *nu.
template <bool RING>
__device__ __forceinline__ int token_list(const Cand& a, int64_t b, int64_t t, Scratch& S, uint8_t* rec, int* nu) {
  const int lane = lane_id();
  const int M = RING ? gather_rings(a, b, t, S) : gather(a, b, t, true, S);
  const int NU = dedupe(a, M, S);
  if (rec) {
    const RecLayout R = rec_layout(a.T, a.C);
    uint16_t* hdr = reinterpret_cast<uint16_t*>(rec);
    uint16_t* e16 = reinterpret_cast<uint16_t*>(rec + R.e16);
    if (lane <= a.T) hdr[lane] = (uint16_t)S.off[lane];
    if (lane == a.T + 1) hdr[lane] = (uint16_t)NU;
    for (int m = lane; m < M; m += kWave) e16[m] = (uint16_t)(((S.key[m] & 31) << 8) | S.uid[m]);
  }
  *nu = NU;
  return M;
}

// The uniques' score terms: S.ua = base + w_suf[ell] + log_alfa_k, S.ub = fp32(Bt_k - Bt_q), S.uc = 0 (and the
// record's per-unique fields). NW = 1: the whole wave does every unique. NW > 1: wave `wave` of NW does the chunks of
// 2 kRows uniques wave, wave + NW, ... (its bases and then their other terms, so no other wave's results are read).
// STEP_CLOCK: Bt_q is formed from Bt[t - 1] and the repetition step's beta (a.rep), which writes Bt[t] concurrently.
template <int F4, int NW, bool FB16 = false, bool STEP_CLOCK = false>
__device__ __forceinline__ void unique_terms(const Cand& a, int64_t b, int64_t t, int NU, Scratch& S, uint8_t* rec,
                                             int wave) {
  const int lane = lane_id();
  const int64_t tok = b * a.L + t;
  const RecLayout R = rec_layout(a.T, a.C);
  // Lanes take uniques u0 + lane (NW == 1: all 64 lanes; NW > 1: the first 2 kRows lanes of each wave's chunks); the
  // loop below is wave-uniform, so every lane takes part in the shuffle. With NW > 1 (the generation step, where each
  // wave has chunks to spare registers for), what the terms read that depends only on the uniques' positions is loaded
  // before the base scores' rows, so that both are in flight together: this lane's unique in the wave's first NPRE
  // chunks. (With NW = 1 those registers would spill: the whole-text kernels run at their register limit.)
  constexpr int NPRE = NW == 1 ? 0 : 2;
  constexpr int PRE = NPRE > 0 ? NPRE : 1;
  const int per = NW == 1 ? kWave : 2 * kRows;
  const int ustart = NW == 1 ? 0 : wave * 2 * kRows;
  const float* sigb = a.sig + b * a.L;
  float mine[4];
  double bq;
  float wsuf_l;                                             // w_suf[x] in lane x (K <= 16), read by shuffles
  auto own_terms = [&]() {                                  // the query's own suffix and clock
    own_suffix_of(sigb, t, a.K, mine);
    bq = STEP_CLOCK ? clock_at(a.Bt + b * a.L, t, a.rep.beta_t[b], a.rep.reloj32) : a.Bt[tok];
    wsuf_l = lane <= a.K ? a.w_suf[lane] : 0.f;
  };
  UniqueAt pre[PRE];
  if constexpr (NPRE > 0) {
    own_terms();
#pragma unroll
    for (int i = 0; i < NPRE; ++i) pre[i] = unique_at(a, b, S, NU, ustart + i * NW * per + lane, sigb, t);
  }
  if constexpr (F4 == 1) {
    unique_bases8<FB16>(a, b, tok, NU, S, wave * 2 * kRows, NW * 2 * kRows);
  } else {
    float4 qf[F4];
    feat_row<F4, FB16>(feat_lanes<F4, FB16>(a, a.Qc, true), (uint32_t)tok, qf);
    unique_bases<F4, FB16>(a, b, t, NU, false, qf, S, wave * 2 * kRows, NW * 2 * kRows);
  }
  if constexpr (NPRE == 0) own_terms();
  if (a.clock32 && lane == 0 && wave == 0) S.bq32 = (float)bq;
  int i = 0;
  for (int u0 = ustart; u0 < NU; u0 += NW * per, ++i) {
    const int u = u0 + lane;
    const bool in = lane < per && u < NU;
    int64_t k;
    int ell;
    double bk;
    float la;
    if constexpr (NPRE > 0) {
      UniqueAt x;
      if (i < NPRE) {
#pragma unroll
        for (int c = 0; c < NPRE; ++c)                  // a register copy, no indexing by i
          if (c == i) x = pre[c];
      } else {
        x = unique_at(a, b, S, NU, u, sigb, t);
      }
      k = x.k;
      ell = a.K <= 4 ? suffix_len4(x, mine, t, a.K) : suffix_len_of(sigb, mine, t, k, a.K);
      bk = x.bk;
      la = x.la;
    } else {
      k = S.upos[in ? u : NU - 1];
      ell = suffix_len_of(sigb, mine, t, k, a.K);
      bk = a.Bt[b * a.L + k];
      la = a.la[b * a.L + k];
    }
    const float db = (float)(bk - bq);     // with the fp32 clock, the fp32 difference of the two values
    const float ws = __shfl(wsuf_l, ell, kWave);
    if (in) {
      if (a.clock32) {                     // the clock term is formed per entry (load_entries)
        S.ua[u] = S.ua[u] + ws;
        S.ub[u] = (float)bk;
        S.uc[u] = la;
      } else {
        S.ua[u] = (S.ua[u] + ws) + la;
        S.ub[u] = db;
        S.uc[u] = 0.f;
      }
      if (rec) {
        reinterpret_cast<int32_t*>(rec + R.upos)[u] = (int32_t)k;
        reinterpret_cast<float*>(rec + R.ub)[u] = db;
        rec[R.uell + u] = (uint8_t)ell;
      }
    }
  }
  wave_lds_sync();
}

template <int DCH, bool VALUES, bool B16 = false>
__device__ __forceinline__ void token_weights(const Cand& a, int64_t b, int M, int NU, Scratch& S, float* salida_row,
                                              float* signals_row, float* ent_rows, bool count_leak = true);

// One query token's candidate attention: salida row (d), the 4 gate signals and, when `ent_rows` is given, every
// entry's weight at ent_rows[2 (tau * C + distance - 1)]. RING: candidates from the generation rings instead of the
// sorted windows.
template <int F4, int DCH, bool RING, int RB = 0>
__device__ __forceinline__ void forward_token(const Cand& a, int64_t b, int64_t t, Scratch& S, float* salida_row,
                                              float* signals_row, float* ent_rows) {
  const int64_t tok = b * a.L + t;
  uint8_t* rec = (!RING && a.lists) ? a.lists + tok * a.rec : nullptr;
  int NU;
  const int M = token_list<RING>(a, b, t, S, rec, &NU);
  unique_terms<F4, 1, RB == 2>(a, b, t, NU, S, rec, 0);
  token_weights<DCH, true, RB >= 1>(a, b, M, NU, S, salida_row, signals_row, ent_rows);
}

// The rest of a query's attention once its list and unique terms are in S: the exact masked softmax, the entries'
// weights (into ent_rows when given), the 4 gate signals and, with VALUES, the copy-gather into salida_row (without
// it, S.uc holds each unique's summed weight for the caller).
template <int DCH, bool VALUES, bool B16>
__device__ __forceinline__ void token_weights(const Cand& a, int64_t b, int M, int NU, Scratch& S, float* salida_row,
                                              float* signals_row, float* ent_rows, bool count_leak) {
  const int lane = lane_id();

  // Exact masked softmax of every table at once: the per-table max through an LDS atomic max on order-preserving
  // integer keys (order-independent), one exp per entry, the per-table sums by lane groups (table_sum).
  Entries E;
  load_entries(a, M, S, E);
  uint32_t* tmax = reinterpret_cast<uint32_t*>(S.tsum);
  if (lane < a.T) tmax[lane] = 0u;                       // below every key
  wave_lds_sync();
#pragma unroll
  for (int c = 0; c < kCh; ++c)
    if (c * kWave < M && E.tau[c] >= 0) atomicMax(&tmax[E.tau[c]], order_key(E.sc[c]));
  wave_lds_sync();
  float e[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    e[c] = 0.f;
    if (c * kWave < M && E.tau[c] >= 0) {
      e[c] = __expf(E.sc[c] - from_order_key(tmax[E.tau[c]]));
      S.ua[c * kWave + lane] = e[c];                     // per-entry now: the base scores are in E.sc
    }
  }
  wave_lds_sync();
  // one lead lane per table (lane tau * G) carries the table's softmax denominator, max and peak
  const int G = lanes_per_table(a.T), tg = lane / G;
  const bool lead = lane % G == 0 && tg < a.T;
  const float den = table_sum(S, a.T, G, [&](int m) { return S.ua[m]; });
  bool has = false;
  float mx = -INFINITY, inv = 0.f;
  if (lead) {
    if (S.off[tg] < S.off[tg + 1]) {
      has = true;
      mx = from_order_key(tmax[tg]);
      inv = 1.f / den;
      // the reference's -1e9 fill (without the exact mask) gives its invalid keys weight exp(-1e9 - mx), which is
      // nonzero in fp32 once mx is within ~104 of -1e9 (the fp32 spacing there is 64)
      if (count_leak && a.leak && mx <= kFill + kLeakReach) atomicAdd(a.leak, 1);
    }
    S.tinv[tg] = inv;
  }
  wave_lds_sync();
  float w[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    w[c] = 0.f;
    const int m = c * kWave + lane;
    if (c * kWave < M && E.tau[c] >= 0) {
      w[c] = e[c] * S.tinv[E.tau[c]];
      if (ent_rows) ent_rows[2 * (E.tau[c] * a.C + (S.off[E.tau[c] + 1] - 1 - m))] = w[c];   // entries ascend
    }
  }
  {                                                      // per unique, the weights summed over tables (S.uc)
    float wv[1][kCh];
#pragma unroll
    for (int c = 0; c < kCh; ++c) wv[0][c] = w[c];
    float* const out[1] = {S.uc};
    unique_table_sums<1>(a.T, NU, E.tau, E.u, wv, S.ua, 2 * kMaxSlots, out);   // ua and ub are dead here
  }
  const float pt = (float)__popcll(__ballot(has));       // has is set in lead lanes only
  const float best = wave_max_u(mx);
  const float pico = wave_sum_u(inv);                    // the largest weight of a table is exp(0) / den
  const float pctx = (float)__popcll(__ballot(has && tg >= a.T - a.Tc));

  if (lane == 0) {
    signals_row[0] = pt;
    signals_row[1] = pt > 0.f ? fmaxf(best, -1e9f) : -1e9f;
    signals_row[2] = pico;
    signals_row[3] = pctx;
  }
  if constexpr (VALUES) {
    // copy-gather over the distinct candidates: sum_u (sum_tau att) V_u, a slab of 256 DCH columns at a time
    for (int c0 = 0; c0 < a.d; c0 += 256 * DCH) {
      float4 acc[DCH];
#pragma unroll
      for (int ch = 0; ch < DCH; ++ch) acc[ch] = zero4();
      gather_values<DCH, B16>(a, b, S, NU, 0, gather_rows_in_flight<DCH>(), acc, c0);
#pragma unroll
      for (int ch = 0; ch < DCH; ++ch) {
        const int dd = c0 + ch * 256 + lane * 4;
        if (dd < a.d) st4r<B16>(salida_row, dd, acc[ch]);
      }
    }
  }
}

// RB: how V (and the backward's dO) and the features [phi ; Qc ; Kc] are stored: 0 fp32; 1 V and dO bf16; 2 all bf16
template <int F4, int DCH, int RB>
__global__ __launch_bounds__(kWave * kWavesPerBlock, (F4 == 1 && DCH == 1) ? (RB == 0 ? 7 : 6) : 1)
void k_cand_fwd(Cand a) {   // 6-7 waves per SIMD when narrow
  __shared__ Scratch scratch[kWavesPerBlock];
  Scratch& S = scratch[threadIdx.x >> 6];
  const TokAt at = sorted_token_of_wave(a);
  if (at.tok < 0) return;
  const int64_t tok = at.tok;
  float* salida_row = const_cast<float*>(rows_at<RB >= 1>(a.salida, tok * a.d));   // bf16 with the value rows
  forward_token<F4, DCH, false, RB>(a, at.b, at.t, S, salida_row, a.signals + tok * 4, a.ent + tok * a.T * a.C * 2);
}

// Generation step: one workgroup of kDecodeWaves waves per batch row; the query is position tq = a.tq (or *a.tq_dev)
// of the caches (a.L = their capacity; a position outside them writes nothing). Wave 0 gathers the ring candidates
// and dedupes them; every wave forms the score terms of its share of the distinct candidates; wave 0 normalizes;
// then every wave sums the value rows of its share (chunks of consecutive uniques, one chunk in kDecodeWaves per
// wave), and wave 0 adds the waves' sums in wave order.
// With a.insert, tq then enters its bucket's ring in every table at slot count % C, overwriting the oldest (reference
// nucleo:1610-1618): only wave 0 touches batch row b's rings, and its ring reads were consumed before.
// REP: the workgroups past the B batch rows run the repetition step (a.rep), one thread per (row, n-gram length). It
// writes Bt[tq], the Hawkes tables, the streak and its own outputs, none of which the attention reads (the candidates'
// positions are below tq, and the query's clock is formed as the step forms it), and reads nothing the attention
// writes.
// Column split (gridDim.y > 1, with a.done): workgroup y of a row gathers the value columns [256 DCH y, 256 DCH (y +
// 1)) after forming the list, scores and weights as every workgroup of the row does (the same bits; only y = 0 counts
// the leak): the value rows one CU pulls are what bound the gather. The rings change only once every workgroup of the
// row has read them: each adds 1 to a.done[b] once its ring reads are consumed (after the workgroup's first barrier),
// and the one that reads gridDim.y - 1 inserts tq and sets the count back to 0. Nothing waits on the count.
constexpr int kDecodeWaves = 8;

template <int F4, int DCH, bool REP>
__global__ __launch_bounds__(kWave * kDecodeWaves) void k_decode_attend(Cand a) {
  __shared__ Scratch S;
  __shared__ float4 part[kDecodeWaves][DCH][kWave];
  __shared__ int nu_shared;
  if (REP && blockIdx.x >= a.B) {
    if (blockIdx.y != 0) return;
    const int64_t e = (int64_t)(blockIdx.x - a.B) * blockDim.x + threadIdx.x;
    const int64_t t = step_pos(a.rep);
    if (e < a.rep.B * a.rep.n && t >= 0 && t < a.rep.stride) repetition_row(a.rep, a.rep_tab, e, t);
    return;
  }
  const int64_t b = blockIdx.x;
  const int64_t tq = a.tq_dev ? *a.tq_dev : a.tq;
  if (b >= a.B || tq < 0 || tq >= a.L) return;            // the same for every wave of the workgroup
  const int wave = threadIdx.x >> 6, lane = lane_id();
  __shared__ int m_shared;
  if (wave == 0) {
    int nu;
    const int m = token_list<true>(a, b, tq, S, nullptr, &nu);
    if (lane == 0) {
      nu_shared = nu;
      m_shared = m;
    }
  }
  __syncthreads();
  const int ny = gridDim.y;
  __shared__ int last_shared;
  if (ny > 1 && threadIdx.x == 0) last_shared = atomicAdd(&a.done[b], 1) == ny - 1;
  const int NU = nu_shared;
  unique_terms<F4, kDecodeWaves, false, REP>(a, b, tq, NU, S, nullptr, wave);
  __syncthreads();
  if (wave == 0) token_weights<DCH, false>(a, b, m_shared, NU, S, nullptr, a.signals + b * 4, nullptr, blockIdx.y == 0);
  __syncthreads();
  constexpr int UNR = gather_rows_in_flight<DCH>();
  for (int c0 = 256 * DCH * blockIdx.y; c0 < a.d; c0 += 256 * DCH * ny) {   // one slab of 256 DCH columns at a time
    float4 acc[DCH];
#pragma unroll
    for (int ch = 0; ch < DCH; ++ch) acc[ch] = zero4();
    gather_values<DCH>(a, b, S, NU, wave * UNR, kDecodeWaves * UNR, acc, c0);
#pragma unroll
    for (int ch = 0; ch < DCH; ++ch) part[wave][ch][lane] = acc[ch];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int ch = 0; ch < DCH; ++ch) {
        float4 s = part[0][ch][lane];
        for (int w = 1; w < kDecodeWaves; ++w) {
          const float4 q = part[w][ch][lane];
          s.x += q.x; s.y += q.y; s.z += q.z; s.w += q.w;
        }
        const int dd = c0 + ch * 256 + lane * 4;
        if (dd < a.d) *reinterpret_cast<float4*>(a.salida + b * a.d + dd) = s;
      }
    }
    __syncthreads();                                       // part is rewritten by the next slab
  }
  if (wave != 0) return;
  const bool last = ny == 1 || last_shared;
  if (ny > 1 && last && lane == 0) atomicExch(&a.done[b], 0);   // at the adds' coherence point
  if (a.insert && last && lane < a.T) {
    const int id = a.ids_out[b * a.T + lane];
    const int64_t bucket = (b * a.T + lane) * ((int64_t)1 << a.nb) + id;
    const int c = a.counts[bucket];
    a.rings[bucket * a.C + c % a.C] = (int32_t)tq;
    a.counts[bucket] = c + 1;
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// backward, query pass: needs no scores. att comes from the forward; per distinct key, dp = <dO_q, V_k>, the clock
// difference and the suffix length; per table D = sum att dp, then ds = att (dp - D) per entry, kept for the key pass.
// ---------------------------------------------------------------------------------------------------------------------
template <int F4, int DCH, int RB>
__global__ __launch_bounds__(kWave * kWavesPerBlock, (F4 == 1 && DCH == 1) ? 7 : 1) void k_cand_bwd_q(Cand a) {
  constexpr bool B16 = RB >= 1, FB16 = RB == 2;
  __shared__ Scratch scratch[kWavesPerBlock];
  Scratch& S = scratch[threadIdx.x >> 6];
  const TokAt at = sorted_token_of_wave(a);
  if (at.tok < 0) return;
  const int lane = lane_id(), half = lane >> 5;
  const int64_t tok = at.tok, b = at.b, t = at.t;

  int M, NU;
  if (a.lists) {             // the forward's list: no gather, dedupe or per-candidate clock and suffix loads
    load_record(a, a.lists + tok * a.rec, S, M, NU);
  } else {
    M = gather(a, b, t, true, S);
    NU = dedupe(a, M, S);
    const float* sigb = a.sig + b * a.L;
    float mine[4];
    own_suffix_of(sigb, t, a.K, mine);
    const double bq = a.Bt[tok];
    for (int u = lane; u < NU; u += kWave) {
      const int64_t k = S.upos[u];
      S.uell[u] = (uint8_t)suffix_len_of(sigb, mine, t, k, a.K);
      S.ub[u] = (float)(a.Bt[b * a.L + k] - bq);
    }
  }
  // every entry's att from the forward, loaded now so that it arrives with the value rows below
  float* erow = a.ent + tok * a.T * a.C * 2;
  float att[kCh], dp[kCh];
  int tau[kCh], un[kCh], slot[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int m = c * kWave + lane;
    const bool in = m < M;
    const int e = in ? S.key[m] : 0;
    tau[c] = in ? (e & 31) : -1;
    un[c] = in ? S.uid[m] : 0;
    slot[c] = in ? (e & 31) * a.C + (S.off[(e & 31) + 1] - 1 - m) : 0;
    att[c] = in ? erow[2 * slot[c]] : 0.f;
  }
  // dp_u = <dO_q, V_u>, summed over the slabs of 256 DCH columns (ends with a wave sync)
  for (int c0 = 0; c0 < a.d; c0 += 256 * DCH) {
    unique_row_dots<DCH, B16>(a, rows_at<B16>(a.V, (b * a.L + a.vshift) * a.ldv), a.ldv, NU,
                              rows_at<B16>(a.dsal, tok * a.d), S, S.uc, c0, c0 > 0);
  }

  // per entry: att * dp (S.ua is a per-entry buffer here)
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int m = c * kWave + lane;
    const bool in = tau[c] >= 0;
    dp[c] = in ? S.uc[un[c]] : 0.f;
    if (in) S.ua[m] = att[c] * dp[c];
  }
  wave_lds_sync();
  const int G = lanes_per_table(a.T), tg = lane / G;
  const bool lead = lane % G == 0 && tg < a.T;
  {                                                     // D per table
    const float D = table_sum(S, a.T, G, [&](int m) { return S.ua[m]; });
    if (lead) S.tsum[tg] = D;
  }
  wave_lds_sync();
  float ds[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int m = c * kWave + lane;
    const bool in = tau[c] >= 0;
    ds[c] = in ? att[c] * (dp[c] - S.tsum[tau[c]]) : 0.f;
    if (in) {
      erow[2 * slot[c] + 1] = ds[c];
      S.ua[m] = ds[c];
    }
  }
  wave_lds_sync();
  float* part = a.partials + tok * (a.T + a.K + 1);
  float dbq_t = 0.f;
  {                                                     // per table: sum ds (clock) and sum ds * dt (d gamma)
    const float sds = table_sum(S, a.T, G, [&](int m) { return S.ua[m]; });
    const float sdt = table_sum(S, a.T, G, [&](int m) { return S.ua[m] * S.ub[S.uid[m]]; });
    if (lead) {
      part[tg] = sdt / (float)a.C;                     // d gamma_tau: the rate is gamma / C
      dbq_t = -rate_of(a, tg) * sds;
    }
  }
  {                                                     // per unique: ds summed over tables (S.uc)
    float dv[1][kCh];
#pragma unroll
    for (int c = 0; c < kCh; ++c) dv[0][c] = ds[c];
    float* const out[1] = {S.uc};
    unique_table_sums<1>(a.T, NU, tau, un, dv, S.ua, 2 * kMaxSlots, out);   // ua and ub are dead here
  }

  // d phi_q, d Qc_q = sum_u (sum_tau ds) [phi_u ; Kc_u]
  float4 gq[F4];
  unique_feature_sum<F4, FB16>(a, b, t, NU, false, S.uc, S, gq);
  if (half == 0) {   // P and cf are multiples of 4: a lane's 4 features lie in one of the two rows
#pragma unroll
    for (int c = 0; c < F4; ++c) {
      const int f0 = 4 * lane + 128 * c;
      if (f0 < a.P)
        *reinterpret_cast<float4*>(a.dphi + tok * a.P + f0) =
            make_float4(gq[c].x * a.sp, gq[c].y * a.sp, gq[c].z * a.sp, gq[c].w * a.sp);
      else if (f0 < a.P + a.cf)
        *reinterpret_cast<float4*>(a.dQc + tok * a.ldq + (f0 - a.P)) =
            make_float4(gq[c].x * a.sc, gq[c].y * a.sc, gq[c].z * a.sc, gq[c].w * a.sc);
    }
  }
  {   // d w_suf[x] = the ds of the entries whose suffix match is x = sum over the uniques u with ell_u = x of their
      // summed ds (S.uc): lane group x strides over the uniques, then adds up in a fixed butterfly
    const int Gx = lanes_per_table(a.K + 1), x = lane / Gx;
    float v = 0.f;
    if (x <= a.K)
      for (int u = lane % Gx; u < NU; u += Gx) v += S.uell[u] == x ? S.uc[u] : 0.f;
    for (int m = Gx >> 1; m > 0; m >>= 1) v += __shfl_xor(v, m, kWave);
    if (lane % Gx == 0 && x <= a.K) part[a.T + x] = v;
  }
  float dbq = 0.f;
  for (int tt = 0; tt < a.T; ++tt) dbq += readlane_f(dbq_t, tt * G);
  if (lane == 0) a.dBt[tok] = (double)dbq;
}

// sum_u w_u row_u over the uniques' d-wide rows (rows of batch row b), UNR rows in flight
template <int DCH, bool B16 = false>
__device__ __forceinline__ void unique_row_sum(const Cand& a, const float* rows, int64_t self_pos, int NU,
                                               const float* w_u, const Scratch& S, float4 (&acc)[DCH], int c0 = 0) {
  const int lane = lane_id();
  constexpr int UNR = DCH >= 4 ? 4 : (DCH >= 2 ? 8 : 8);   // fits the key pass's register budget (6 waves at DCH 1)
  int col[DCH];
#pragma unroll
  for (int ch = 0; ch < DCH; ++ch) {
    acc[ch] = zero4();
    col[ch] = slab_col(a, c0, ch, lane);
  }
  for_chunks<UNR>(0, NU, UNR, [&](auto n, int u0) {
    constexpr int R = decltype(n)::value;
    int p[R];
    float w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {                      // wave-uniform rows and weights: scalar offsets
      const int u = u0 + r < NU ? u0 + r : NU - 1;
      p[r] = __builtin_amdgcn_readfirstlane(S.upos[u]);
      w[r] = u0 + r < NU ? w_u[u] : 0.f;             // the same in every lane (an LDS broadcast)
    }
    float4 v[R][DCH];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float* row = rows_at<B16>(rows, (int64_t)(uint32_t)p[r] * a.d);
#pragma unroll
      for (int ch = 0; ch < DCH; ++ch) v[r][ch] = ld4r<B16>(row, (uint32_t)col[ch]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int ch = 0; ch < DCH; ++ch) fma4(acc[ch], w[r], v[r][ch]);
  });
  (void)self_pos;
}

// ---------------------------------------------------------------------------------------------------------------------
// backward, key pass: no scores either. Every entry's att (forward) and ds (query pass) are read at the query's
// slot for this key; per distinct query the table sums weight dO (-> dV) and [phi_q ; Qc_q] (-> d phi_k, d Kc_k).
// ---------------------------------------------------------------------------------------------------------------------
template <int F4, int DCH, int RB>
__global__ __launch_bounds__(kWave * kWavesPerBlock, (F4 == 1 && DCH == 1) ? 6 : ((F4 == 1 && DCH == 2) ? 5 : 1))
void k_cand_bwd_k(Cand a) {
  constexpr bool B16 = RB >= 1, FB16 = RB == 2;
  __shared__ Scratch scratch[kWavesPerBlock];
  Scratch& S = scratch[threadIdx.x >> 6];
  const TokAt at = sorted_token_of_wave(a);
  if (at.tok < 0) return;
  const int lane = lane_id(), half = lane >> 5;
  const int64_t tok = at.tok, b = at.b, k = at.t;
  // the query pass's d phi and dBt of this token, loaded now so their latency hides behind the gathers
  float4 dphi_q[F4];
#pragma unroll
  for (int c = 0; c < F4; ++c) {
    const int f0 = 4 * lane + 128 * c;
    dphi_q[c] = half == 0 && f0 < a.P ? ld4(a.dphi + tok * a.P + f0) : zero4();
  }
  const double dbt_q = a.dBt[tok];   // wave-uniform

  const int M = gather(a, b, k, false, S);
  const int NU = dedupe(a, M, S);
  float att[kCh], ds[kCh];
  int tau[kCh], un[kCh];
  float dla = 0.f, dbk = 0.f;
  const float rate_l = lane < a.T ? rate_of(a, lane) : 0.f;   // one division per table, shuffled to the entries
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int m = c * kWave + lane;
    const bool in = m < M;
    const int e = in ? S.key[m] : 0;
    tau[c] = in ? (e & 31) : -1;
    un[c] = in ? S.uid[m] : 0;
    att[c] = 0.f;
    ds[c] = 0.f;
    const float rate = __shfl(rate_l, e & 31, kWave);        // every lane takes part (no divergent shuffle)
    if (in) {   // the key sits at distance m - lo + 1 before query (e >> 5) in table tau
      const uint32_t o = ((uint32_t)(b * a.L + (e >> 5)) * (uint32_t)a.T + (uint32_t)(e & 31)) * (uint32_t)a.C +
                         (uint32_t)(m - S.off[e & 31]);
      const float2 w2 = *reinterpret_cast<const float2*>(a.ent + 2 * (uint64_t)o);
      att[c] = w2.x;
      ds[c] = w2.y;
      dla += ds[c];
      dbk += rate * ds[c];
    }
  }
  // per unique, summed over tables: att (S.uc, the dV weights) and ds (the feature weights, in the key array, which
  // is dead once the entries are in registers)
  float* const dsum = reinterpret_cast<float*>(S.key);
  {
    float v[2][kCh];
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      v[0][c] = att[c];
      v[1][c] = ds[c];
    }
    float* const out[2] = {S.uc, dsum};
    unique_table_sums<2>(a.T, NU, tau, un, v, S.ua, 2 * kMaxSlots, out);   // ua and ub are dead here
  }
  // park the prefetched d phi in LDS (ua is free again) to keep registers for the gathers
#pragma unroll
  for (int c = 0; c < F4; ++c) {
    const int f0 = 4 * lane + 128 * c;
    if (half == 0 && f0 < a.P) *reinterpret_cast<float4*>(S.ua + f0) = dphi_q[c];
  }

  // with vshift, V[k] is the projection of k + 1: its gradient goes to row k + 1, and the last position (which no
  // query sees, so dv is 0) clears row 0, the projection no V reads
  const int64_t dv_row = a.vshift ? b * a.L + (k + 1 < a.L ? k + 1 : 0) : tok;
  // dV_k = sum_u (sum_tau att) dO_u, a slab of 256 DCH columns at a time
  for (int c0 = 0; c0 < a.d; c0 += 256 * DCH) {
    float4 dv[DCH];
    unique_row_sum<DCH, B16>(a, rows_at<B16>(a.dsal, b * a.L * a.d), k, NU, S.uc, S, dv, c0);
#pragma unroll
    for (int ch = 0; ch < DCH; ++ch) {
      const int dd = c0 + ch * 256 + lane * 4;
      if (dd < a.d) st4r<B16>(a.dV, dv_row * a.ldv + dd, dv[ch]);
    }
  }
  // d phi_k, d Kc_k = sum_u (sum_tau ds) [phi_q * scale_phi ; Qc_q * scale_c]
  float4 gk[F4];
  unique_feature_sum<F4, FB16>(a, b, k, NU, true, dsum, S, gk);
  if (half == 0) {   // P and cf are multiples of 4: a lane's 4 features lie in one of the two rows
#pragma unroll
    for (int c = 0; c < F4; ++c) {
      const int f0 = 4 * lane + 128 * c;
      if (f0 < a.P)
        *reinterpret_cast<float4*>(a.dphi + tok * a.P + f0) =
            make_float4(S.ua[f0] + gk[c].x, S.ua[f0 + 1] + gk[c].y, S.ua[f0 + 2] + gk[c].z, S.ua[f0 + 3] + gk[c].w);
      else if (f0 < a.P + a.cf)
        *reinterpret_cast<float4*>(a.dKc + tok * a.ldq + (f0 - a.P)) = gk[c];
    }
  }
  const float sla = wave_sum_u(dla);
  const float sbk = wave_sum_u(dbk);
  if (lane == 0) {
    a.dla[tok] = sla;
    a.dBt[tok] = dbt_q + (double)sbk;
  }
}

// the candidate lists the kernels walk, materialized: (B, L, T, C) text positions (-1 = empty slot; the valid
// candidates fill the last slots, oldest first) and the suffix-match length of each against its query
__global__ __launch_bounds__(kWave * kWavesPerBlock) void k_cand_lists(Cand a, int32_t* __restrict__ pos,
                                                                       int32_t* __restrict__ ell) {
  __shared__ Scratch scratch[kWavesPerBlock];
  Scratch& S = scratch[threadIdx.x >> 6];
  const int64_t tok = token_of_wave(a);
  if (tok >= a.B * a.L) return;
  const int lane = lane_id();
  const int64_t b = tok / a.L, t = tok % a.L;
  gather(a, b, t, true, S);
  const float* sigb = a.sig + b * a.L;
  float mine[4];
  own_suffix_of(sigb, t, a.K, mine);
  for (int tau = 0; tau < a.T; ++tau) {
    const int lo = S.off[tau], n = S.off[tau + 1] - lo;
    if (lane < a.C) {
      const int64_t o = (tok * a.T + tau) * a.C + lane;
      const int i = lane - (a.C - n);
      const int64_t k = i >= 0 ? (S.key[lo + i] >> 5) : -1;
      pos[o] = (int32_t)k;
      ell[o] = i >= 0 ? suffix_len_of(sigb, mine, t, k, a.K) : -1;
    }
  }
}

// The wave's token, as wave-uniform scalars (so that no per-lane division or 64-bit index math follows from it).
__device__ __forceinline__ TokAt sorted_token_of_wave(const Cand& a) {
  const int64_t i = token_of_wave(a);
  if (i >= a.B * a.L) return {0, 0, -1};
  const int64_t b = row_of(a, i), r = i - b * a.L;
  if (!ASRN_SORTED_MAP) return {b, r, i};
  const int tab = ASRN_SORTED_TABLE < 0 ? a.T - 1 : (ASRN_SORTED_TABLE < a.T ? ASRN_SORTED_TABLE : 0);
  // a permutation of the row's positions (the bucket sort's), clamped so that inconsistent inputs stay in bounds
  int p = __builtin_amdgcn_readfirstlane(a.order[(uint32_t)((b * a.T + tab) * a.L + r)]);
  p = p < 0 ? 0 : (p >= a.L ? (int)a.L - 1 : p);
  return {b, p, b * a.L + p};
}

static int check_args(const Cand& a, const char* what) {
  ASRN_REQUIRE(a.B >= 0 && a.L >= 0, "%s: bad sizes", what);
  ASRN_REQUIRE(a.L < (int64_t(1) << 26), "%s: L=%lld too long (positions are packed in 26 bits)", what,
               (long long)a.L);
  ASRN_REQUIRE(a.d >= 4 && a.d % 4 == 0, "%s: d=%d must be a multiple of 4, at least 4", what, a.d);
  ASRN_REQUIRE(a.C >= 1 && a.C <= 64, "%s: chunk C=%d must be in [1, 64]", what, a.C);
  ASRN_REQUIRE(a.T >= 1 && a.T <= 32 && a.T * a.C <= kMaxSlots && a.Tc >= 0 && a.Tc <= a.T,
               "%s: T=%d, C=%d, Tc=%d: needs T <= 32 and T*C <= %d", what, a.T, a.C, a.Tc, kMaxSlots);
  ASRN_REQUIRE(a.P >= 1 && a.cf >= 1 && a.P + a.cf <= 256, "%s: P + cf = %d must be <= 256", what, a.P + a.cf);
  ASRN_REQUIRE(a.P % 4 == 0 && a.cf % 4 == 0, "%s: P=%d and cf=%d must be multiples of 4 (feature rows are read as "
               "float4; pad the columns with zeros)", what, a.P, a.cf);
  {
    const int64_t widest = a.d > a.P ? (a.d > a.cf ? a.d : a.cf) : (a.P > a.cf ? a.P : a.cf);
    ASRN_REQUIRE(a.B * a.L * widest < (int64_t(1) << 31), "%s: B*L*max(d, P) = %lld elements must stay below 2^31 "
                 "(32-bit row offsets)", what, (long long)(a.B * a.L * widest));
  }
  ASRN_REQUIRE(a.K >= 0 && a.K <= 16, "%s: suffix K=%d must be in [0, 16]", what, a.K);
  ASRN_REQUIRE(a.B * a.L * a.T < (int64_t(1) << 31) && a.B * a.L * a.T * a.C * 2 < (int64_t(1) << 31),
               "%s: B*L*T*C*2 = %lld must stay below 2^31 (32-bit index and entry offsets)", what,
               (long long)(a.B * a.L * a.T * a.C * 2));
  ASRN_REQUIRE(a.ldv >= a.d && a.ldv % 4 == 0 && ((uintptr_t)a.V & 15) == 0 && (a.vshift == 0 || a.vshift == 1),
               "%s: V rows need a stride ldv >= d, a multiple of 4, a 16-byte aligned V and v_shift 0 or 1", what);
  ASRN_REQUIRE(a.L * a.ldv < (int64_t(1) << 31), "%s: L*ldv must stay below 2^31 (32-bit row offsets)", what);
  ASRN_REQUIRE(a.ldq >= a.cf && a.ldq % 4 == 0 && ((uintptr_t)a.Qc & 15) == 0 && ((uintptr_t)a.Kc & 15) == 0 &&
                   a.B * a.L * a.ldq < (int64_t(1) << 31),
               "%s: Qc/Kc rows need a stride ldq >= cf, a multiple of 4, 16-byte aligned rows, B*L*ldq < 2^31", what);
  return 0;
}

static Cand make(const float* phi, const float* V, const float* Qc, const float* Kc, const float* sig,
                 const double* Bt, const float* la, const float* w_suf, const float* gamma, const int32_t* order,
                 const int32_t* win, const int32_t* rank, int64_t B, int64_t L, int d, int P, int cf, int K, int T,
                 int Tc, int C, float sp, float sc) {
  Cand a = {};
  a.phi = phi; a.V = V; a.Qc = Qc; a.Kc = Kc; a.sig = sig; a.Bt = Bt; a.la = la; a.w_suf = w_suf;
  a.gamma = gamma; a.order = order; a.win = win; a.rank = rank;
  a.ldv = d; a.vshift = 0; a.ldq = cf;
  a.B = B; a.L = L; a.d = d; a.P = P; a.cf = cf; a.K = K; a.T = T; a.Tc = Tc; a.C = C;
  a.Linv = L > 1 ? ~(uint64_t)0 / (uint64_t)L + 1 : 0;
  a.sp = sp; a.sc = sc;
  return a;
}

// launch a kernel template for the (float4 feature chunks per lane, d chunks) bucket of the arguments
template <template <int, int, int> class Launcher, int RB>
static int dispatch_rows(const Cand& a, hipStream_t st) {
  const int dch = (a.d + 255) / 256;
  if (a.P + a.cf <= 128) {
    switch (dch) {
      case 1: return Launcher<1, 1, RB>::run(a, st);
      case 2: return Launcher<1, 2, RB>::run(a, st);
      case 3: return Launcher<1, 3, RB>::run(a, st);
      default: return Launcher<1, 4, RB>::run(a, st);
    }
  }
  switch (dch) {
    case 1: return Launcher<2, 1, RB>::run(a, st);
    case 2: return Launcher<2, 2, RB>::run(a, st);
    case 3: return Launcher<2, 3, RB>::run(a, st);
    default: return Launcher<2, 4, RB>::run(a, st);
  }
}
// The row-wise XCD mapping (Cand::slice) for the whole-text kernels: when every batch row's gathered rows together
// exceed half of the 256 MB last-level cache and a row splits into 8 equal slices. The environment variable
// ASRN_ROWWISE=0 or 1 forces it off or on (read at each call; the results are the same bits either way, since every
// wave computes its own token).
static void set_mapping(Cand& a, int rows_bf16) {
  const int64_t fb = rows_bf16 == 2 ? 2 : 4, vb = rows_bf16 >= 1 ? 2 : 4;
  const int64_t bytes = a.B * a.L * ((a.P + a.cf) * fb + a.d * vb);
  bool on = a.B > 1 && bytes > (int64_t(128) << 20);
  if (const char* f = getenv("ASRN_ROWWISE")) {
    if (f[0] == '0' && f[1] == 0) on = false;
    if (f[0] == '1' && f[1] == 0) on = true;
  }
  a.slice = (on && a.L % kXcds == 0 && kWavesPerBlock == 1) ? a.L / kXcds : 0;
}

// rows_bf16: 0 fp32 rows; 1 V (and the backward's dO) bf16; 2 V, dO and the features bf16
template <template <int, int, int> class Launcher>
static int dispatch(const Cand& a, hipStream_t st, int rows_bf16 = 0) {
  if (rows_bf16 == 2) return dispatch_rows<Launcher, 2>(a, st);
  return rows_bf16 == 1 ? dispatch_rows<Launcher, 1>(a, st) : dispatch_rows<Launcher, 0>(a, st);
}

static dim3 grid_of(const Cand& a) { return dim3((unsigned)((a.B * a.L + kWavesPerBlock - 1) / kWavesPerBlock)); }

template <int F4, int DCH, int RB>
struct LaunchFwd {
  static int run(const Cand& a, hipStream_t st) {
    hipLaunchKernelGGL((k_cand_fwd<F4, DCH, RB>), grid_of(a), dim3(kWave * kWavesPerBlock), 0, st, a);
    return check_launch("asrn_candidates_fwd");
  }
};

template <int F4, int DCH, int RB>
struct LaunchDecode {                              // the generation caches are fp32 (RB > 0 is never dispatched)
  static int run(const Cand& a, hipStream_t st) {
    if constexpr (RB != 0) {
      return fail("asrn_decode_attend: fp32 caches only");
    } else {
      // the columns split over DCH workgroups of 256 when a count buffer is given and the rows leave CUs idle
      const bool split = DCH > 1 && a.done && a.B * DCH <= 256;
      const unsigned ny = split ? DCH : 1;
      const int64_t threads = kWave * kDecodeWaves;
      if (a.rep.beta_t) {                          // with the repetition step's workgroups after the B rows
        const int64_t extra = (a.rep.B * a.rep.n + threads - 1) / threads;
        const dim3 grid((unsigned)(a.B + extra), ny);
        if (split) hipLaunchKernelGGL((k_decode_attend<F4, 1, true>), grid, dim3(threads), 0, st, a);
        else hipLaunchKernelGGL((k_decode_attend<F4, DCH, true>), grid, dim3(threads), 0, st, a);
        return check_launch("asrn_decode_attend_repeat");
      }
      const dim3 grid((unsigned)a.B, ny);
      if (split) hipLaunchKernelGGL((k_decode_attend<F4, 1, false>), grid, dim3(threads), 0, st, a);
      else hipLaunchKernelGGL((k_decode_attend<F4, DCH, false>), grid, dim3(threads), 0, st, a);
      return check_launch("asrn_decode_attend");
    }
  }
};

template <int F4, int DCH, int RB>
struct LaunchBwd {
  static int run(const Cand& a, hipStream_t st) {
    hipLaunchKernelGGL((k_cand_bwd_q<F4, DCH, RB>), grid_of(a), dim3(kWave * kWavesPerBlock), 0, st, a);
    if (check_launch("asrn_candidates_bwd/query")) return 1;
    hipLaunchKernelGGL((k_cand_bwd_k<F4, DCH, RB>), grid_of(a), dim3(kWave * kWavesPerBlock), 0, st, a);
    return check_launch("asrn_candidates_bwd/key");
  }
};

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_candidates_fwd(const float* phi, const float* V, const float* Qc, const float* Kc,
                                   const float* sig, const double* Bt, const float* log_alfa, const float* w_suf,
                                   const float* gamma, const int32_t* order, const int32_t* win, const int32_t* rank,
                                   int64_t B, int64_t L, int32_t d, int32_t P, int32_t cf, int32_t K, int32_t T,
                                   int32_t Tc, int32_t C, float scale_phi, float scale_c, int64_t ldv,
                                   int32_t v_shift, int64_t ldq, int32_t rows_bf16, float* salida, float* signals,
                                   float* entries, uint8_t* lists, int32_t clock_mode, int32_t* leak, void* stream) {
  Cand a = make(phi, V, Qc, Kc, sig, Bt, log_alfa, w_suf, gamma, order, win, rank, B, L, d, P, cf, K, T, Tc, C,
                scale_phi, scale_c);
  a.ldv = ldv;
  a.vshift = v_shift;
  a.ldq = ldq;
  ASRN_REQUIRE(clock_mode == 0 || clock_mode == 1, "asrn_candidates_fwd: clock_mode=%d must be 0 (the fp64 clock's "
               "difference) or 1 (the core layer's fp32 clock term)", clock_mode);
  a.clock32 = clock_mode;
  a.leak = leak;
  if (check_args(a, "asrn_candidates_fwd")) return 1;
  if (B == 0 || L == 0) return 0;
  a.salida = salida; a.signals = signals; a.ent = entries;
  a.lists = lists; a.rec = rec_layout(T, C).size;
  ASRN_REQUIRE(((uintptr_t)lists & 15) == 0, "asrn_candidates_fwd: lists must be 16-byte aligned");
  ASRN_REQUIRE(rows_bf16 >= 0 && rows_bf16 <= 2, "asrn_candidates_fwd: rows_bf16 must be 0, 1 or 2");
  set_mapping(a, rows_bf16);
  return dispatch<LaunchFwd>(a, (hipStream_t)stream, rows_bf16);
}

extern "C" int asrn_candidates_bwd(const float* phi, const float* V, const float* Qc, const float* Kc,
                                   const float* sig, const double* Bt, const float* log_alfa, const float* w_suf,
                                   const float* gamma, const int32_t* order, const int32_t* win, const int32_t* rank,
                                   int64_t B, int64_t L, int32_t d, int32_t P, int32_t cf, int32_t K, int32_t T,
                                   int32_t Tc, int32_t C, float scale_phi, float scale_c, int64_t ldv,
                                   int32_t v_shift, int64_t ldq, int32_t rows_bf16, const float* dsalida,
                                   float* entries, const uint8_t* lists, float* dphi,
                                   float* dV, float* dQc, float* dKc, double* dBt, float* dlog_alfa, float* partials,
                                   void* stream) {
  Cand a = make(phi, V, Qc, Kc, sig, Bt, log_alfa, w_suf, gamma, order, win, rank, B, L, d, P, cf, K, T, Tc, C,
                scale_phi, scale_c);
  a.ldv = ldv;
  a.vshift = v_shift;
  a.ldq = ldq;
  if (check_args(a, "asrn_candidates_bwd")) return 1;
  ASRN_REQUIRE(((uintptr_t)dV & 15) == 0 && ((uintptr_t)dQc & 15) == 0 && ((uintptr_t)dKc & 15) == 0,
               "asrn_candidates_bwd: dV, dQc and dKc must be 16-byte aligned (rows of stride ldv, ldq)");
  if (B == 0 || L == 0) return 0;
  a.lists = const_cast<uint8_t*>(lists); a.rec = rec_layout(T, C).size;
  ASRN_REQUIRE(((uintptr_t)lists & 15) == 0, "asrn_candidates_bwd: lists must be 16-byte aligned");
  a.dsal = dsalida; a.ent = entries; a.dphi = dphi; a.dV = dV; a.dQc = dQc; a.dKc = dKc; a.dBt = dBt;
  a.dla = dlog_alfa; a.partials = partials;
  ASRN_REQUIRE(rows_bf16 >= 0 && rows_bf16 <= 2, "asrn_candidates_bwd: rows_bf16 must be 0, 1 or 2");
  ASRN_REQUIRE(((uintptr_t)dsalida & 15) == 0, "asrn_candidates_bwd: dsalida must be 16-byte aligned");
  set_mapping(a, rows_bf16);
  return dispatch<LaunchBwd>(a, (hipStream_t)stream, rows_bf16);
}

extern "C" int64_t asrn_candidates_record_bytes(int32_t T, int32_t C) {
  if (T < 1 || C < 1) return -1;
  return rec_layout(T, C).size;
}

extern "C" int asrn_candidate_lists(const float* sig, const int32_t* order, const int32_t* win, const int32_t* rank,
                                    int64_t B, int64_t L, int32_t T, int32_t C, int32_t K, int32_t* pos, int32_t* ell,
                                    void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && L < (int64_t(1) << 26) && T >= 1 && T <= 32 && C >= 1 && C <= 64 &&
                   T * C <= kMaxSlots && K >= 0 && K <= 16,
               "asrn_candidate_lists: bad sizes B=%lld L=%lld T=%d C=%d K=%d", (long long)B, (long long)L, T, C, K);
  if (B == 0 || L == 0) return 0;
  Cand a = {};
  a.sig = sig; a.order = order; a.win = win; a.rank = rank;
  a.B = B; a.L = L; a.T = T; a.C = C; a.K = K;
  hipLaunchKernelGGL(k_cand_lists, grid_of(a), dim3(kWave * kWavesPerBlock), 0, (hipStream_t)stream, a, pos, ell);
  return check_launch("asrn_candidate_lists");
}

// a14: the generation step's candidate attention over the per-bucket rings (see k_decode_attend)
static int decode_setup(Cand& a, const float* phi, const float* V, const float* Qc, const float* Kc, const float* sig,
                        const double* Bt, const float* log_alfa, const float* w_suf, const float* gamma,
                        int32_t* rings, int32_t* counts, int64_t B, int64_t cap, int64_t t, const int64_t* t_dev,
                        int32_t d, int32_t nb, int32_t cf, int32_t K, int32_t T, int32_t Tc, int32_t C,
                        float scale_phi, float scale_c, int32_t insert, float* salida, float* signals, int32_t* ids,
                        int32_t* leak, int32_t* done, const char* what) {
  a = make(phi, V, Qc, Kc, sig, Bt, log_alfa, w_suf, gamma, nullptr, nullptr, nullptr, B, cap, d, T * nb, cf, K, T,
           Tc, C, scale_phi, scale_c);
  if (check_args(a, what)) return 1;
  ASRN_REQUIRE(nb >= 1 && nb <= 14, "%s: nb=%d must be in [1, 14]", what, nb);
  ASRN_REQUIRE(t >= 0 && t < cap, "%s: position t=%lld outside the caches (capacity %lld)", what, (long long)t,
               (long long)cap);
  a.rings = rings; a.counts = counts; a.ids_out = ids; a.nb = nb; a.tq = t; a.tq_dev = t_dev;
  a.insert = insert ? 1 : 0;
  a.salida = salida; a.signals = signals;
  a.leak = leak;
  a.done = done;
  return 0;
}

extern "C" int asrn_decode_attend(const float* phi, const float* V, const float* Qc, const float* Kc,
                                  const float* sig, const double* Bt, const float* log_alfa, const float* w_suf,
                                  const float* gamma, int32_t* rings, int32_t* counts, int64_t B, int64_t cap,
                                  int64_t t, const int64_t* t_dev, int32_t d, int32_t nb, int32_t cf, int32_t K,
                                  int32_t T, int32_t Tc,
                                  int32_t C, float scale_phi, float scale_c, int32_t insert, float* salida,
                                  float* signals, int32_t* ids, int32_t* leak, int32_t* done, void* stream) {
  Cand a;
  if (decode_setup(a, phi, V, Qc, Kc, sig, Bt, log_alfa, w_suf, gamma, rings, counts, B, cap, t, t_dev, d, nb, cf, K,
                   T, Tc, C, scale_phi, scale_c, insert, salida, signals, ids, leak, done, "asrn_decode_attend"))
    return 1;
  if (B == 0) return 0;
  return dispatch<LaunchDecode>(a, (hipStream_t)stream);
}

extern "C" int asrn_decode_attend_repeat(const float* phi, const float* V, const float* Qc, const float* Kc,
                                         const float* sig, double* Bt, const float* log_alfa, const float* w_suf,
                                         const float* gamma, int32_t* rings, int32_t* counts, int64_t B, int64_t cap,
                                         int64_t t, const int64_t* t_dev, int32_t d, int32_t nb, int32_t cf,
                                         int32_t K, int32_t T, int32_t Tc, int32_t C, float scale_phi, float scale_c,
                                         int32_t insert, float* salida, float* signals, int32_t* ids, int32_t* leak,
                                         const double* beta_t, const double* coef, const float* kappa,
                                         const float* kappa_r, int32_t n, int64_t tab_cap, uint64_t* tab_keys,
                                         double* tab_Bu, float* tab_A, float* racha, float* vistos, float* hawkes,
                                         int32_t reloj32, int32_t* done, void* stream) {
  Cand a;
  if (decode_setup(a, phi, V, Qc, Kc, sig, Bt, log_alfa, w_suf, gamma, rings, counts, B, cap, t, t_dev, d, nb, cf, K,
                   T, Tc, C, scale_phi, scale_c, insert, salida, signals, ids, leak, done, "asrn_decode_attend_repeat"))
    return 1;
  ASRN_REQUIRE(n >= 1 && n <= 16, "asrn_decode_attend_repeat: n=%d must be in [1, 16]", n);
  ASRN_REQUIRE(tab_cap > 0 && (tab_cap & (tab_cap - 1)) == 0 && tab_cap >= 2 * (t + 1),
               "asrn_decode_attend_repeat: table capacity %lld must be a power of two >= 2 (t + 1) = %lld: grow it "
               "first", (long long)tab_cap, (long long)(2 * (t + 1)));
  ASRN_REQUIRE(beta_t && coef && kappa && kappa_r && tab_keys && tab_Bu && tab_A && racha && vistos && hawkes,
               "asrn_decode_attend_repeat: null pointer");
  if (B == 0) return 0;
  a.rep = {sig, Bt, log_alfa, beta_t, coef, kappa, kappa_r, B, cap, t, n, racha, vistos, hawkes, t_dev,
           reloj32 ? 1 : 0};
  a.rep_tab = {tab_keys, tab_Bu, tab_A, tab_cap};
  return dispatch<LaunchDecode>(a, (hipStream_t)stream);
}
