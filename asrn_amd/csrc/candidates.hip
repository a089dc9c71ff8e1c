// a3 - a8: candidate attention over the recent bucket mates, forward and backward.
//
// One wavefront per token. For table tau the query at sorted rank s sees the sorted ranks [s - C, s) of its own
// bucket: the valid lanes of a C-lane window are always a suffix of it (sorted ids are non-decreasing), so the wave
// only walks the valid candidates. Scores use coalesced feature loads: a 32-lane half-wave reads one candidate's
// [phi ; Kc] row (consecutive lanes, consecutive floats) and reduces the products with the query's pre-scaled
// [phi * scale_phi ; Qc * scale_c] row held in registers, so two candidates are scored per step. The copy-gather
// reads each candidate's V row with all 64 lanes (float4 per lane) and accumulates the 8 tables in registers:
// the table sum never leaves the kernel.
//
// The backward has one owner per output row and no atomics. The query pass recomputes the scores, gets
// dp = <dO_q, V_k> per candidate, ds = att (dp - D) with D = sum att dp, and writes the query-side gradients, D per
// (query, table) and per-query partials of d gamma and d w_suf. The key pass walks, for each key, the next <= C
// same-bucket sorted ranks (exactly the queries whose window holds the key), rebuilds att from the forward's saved
// (max, denominator), reloads dO_q once for both dp and dV, and adds the key-side gradients.
#include "common.h"

namespace asrn {

constexpr int kMaxFPL = 8;   // features per half-wave lane: P + cf <= 256
constexpr int kMaxDCH = 4;   // float4 chunks of 256 columns per lane: d <= 1024
constexpr int kWavesPerBlock = 4;

struct Cand {
  const float* phi; const float* V; const float* Qc; const float* Kc; const float* sig;
  const double* Bt; const float* la; const float* w_suf; const float* gamma;
  const int32_t* order; const int32_t* ids_s; const int32_t* rank;
  int64_t B, L;
  int d, P, cf, K, T, Tc, C, fpl, dch;
  float sp, sc;
  // forward outputs
  float* salida; float* signals; float* stats;
  // backward
  const float* dsal; const float* stats_in; float* dphi; float* dV; float* dQc; float* dKc; double* dBt;
  float* dla; float* qstats; float* partials;
};

// feature f of a row: phi for f < P, then the confirmation vector (Qc for queries, Kc for keys)
__device__ __forceinline__ float feat(const Cand& a, const float* conf, int64_t row, int f) {
  if (f < a.P) return a.phi[row * a.P + f];
  if (f < a.P + a.cf) return conf[row * a.cf + (f - a.P)];
  return 0.f;
}

// query features pre-scaled, lane layout f = (lane & 31) + 32 u
__device__ __forceinline__ void query_feats(const Cand& a, int64_t row, float (&qf)[kMaxFPL]) {
  const int hl = lane_id() & 31;
#pragma unroll
  for (int u = 0; u < kMaxFPL; ++u) {
    const int f = hl + 32 * u;
    float v = 0.f;
    if (u < a.fpl) {
      v = feat(a, a.Qc, row, f);
      v *= f < a.P ? a.sp : a.sc;
    }
    qf[u] = v;
  }
}

__device__ __forceinline__ void key_feats(const Cand& a, int64_t row, float (&kf)[kMaxFPL]) {
  const int hl = lane_id() & 31;
#pragma unroll
  for (int u = 0; u < kMaxFPL; ++u) kf[u] = u < a.fpl ? feat(a, a.Kc, row, hl + 32 * u) : 0.f;
}

__device__ __forceinline__ float dot_feats(const float (&x)[kMaxFPL], const float (&y)[kMaxFPL], int fpl) {
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxFPL; ++u)
    if (u < fpl) s += x[u] * y[u];
  return s;
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// per-table candidate window of query (b, t): lane i < C holds candidate i of [s - C, s) if valid
struct Window {
  int64_t rowr;   // b*T + tau
  int s;
  bool valid;
  int32_t k;      // text position of this lane's candidate (0 when invalid)
  int nvalid, first;
};

__device__ __forceinline__ Window query_window(const Cand& a, int64_t b, int64_t t, int tau) {
  Window w;
  const int lane = lane_id();
  w.rowr = b * a.T + tau;
  w.s = a.rank[(b * a.L + t) * a.T + tau];
  const int32_t* ids = a.ids_s + w.rowr * a.L;
  const int my = ids[w.s];
  const int j = w.s - a.C + lane;
  w.valid = lane < a.C && j >= 0 && ids[j] == my;
  w.k = w.valid ? a.order[w.rowr * a.L + j] : 0;
  w.nvalid = __popcll(__ballot(w.valid));
  w.first = a.C - w.nvalid;
  return w;
}

// score extras of lane candidate k against query q (text positions of batch row b):
//   ((base + w_suf[ell]) + log_alfa_k) + rate * fp32(Bt_k - Bt_q)     (reference estable:249-258)
__device__ __forceinline__ float score_of(const Cand& a, int64_t b, int64_t q, int64_t k, float base, float rate,
                                          float* dt_out, int* ell_out) {
  const float* sigb = a.sig + b * a.L;
  const int ell = suffix_match(sigb, q, k, a.K);
  const float dt = (float)(a.Bt[b * a.L + k] - a.Bt[b * a.L + q]);
  if (dt_out) *dt_out = dt;
  if (ell_out) *ell_out = ell;
  return ((base + a.w_suf[ell]) + a.la[b * a.L + k]) + rate * dt;
}

// base scores <q, k_i> of the valid candidates of a window, two per step (one per half-wave)
__device__ __forceinline__ float window_bases(const Cand& a, int64_t b, const Window& w, const float (&qf)[kMaxFPL]) {
  const int lane = lane_id();
  const int half = lane >> 5;
  float mine = 0.f;
  for (int c = 0; c < w.nvalid; c += 2) {
    const int i0 = w.first + c, i1 = i0 + 1;
    const int k0 = readlane_i(w.k, i0);
    const int k1 = readlane_i(w.k, i1 < a.C ? i1 : i0);
    const int64_t kk = half ? k1 : k0;
    float kf[kMaxFPL];
    key_feats(a, b * a.L + kk, kf);
    const float tot = half_sum(dot_feats(qf, kf, a.fpl));
    const float t0 = readlane_f(tot, 0), t1 = readlane_f(tot, 32);
    if (lane == i0) mine = t0;
    if (lane == i1) mine = t1;
  }
  return mine;
}

// ---------------------------------------------------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kWave * kWavesPerBlock) void k_cand_fwd(Cand a) {
  const int64_t tok = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (tok >= a.B * a.L) return;
  const int lane = lane_id();
  const int64_t b = tok / a.L, t = tok % a.L;
  float qf[kMaxFPL];
  query_feats(a, tok, qf);
  float4 acc[kMaxDCH];
#pragma unroll
  for (int ch = 0; ch < kMaxDCH; ++ch) acc[ch] = make_float4(0.f, 0.f, 0.f, 0.f);
  float pt = 0.f, best = -INFINITY, pico = 0.f, pctx = 0.f;
  const float* Vb = a.V + b * a.L * a.d;

  for (int tau = 0; tau < a.T; ++tau) {
    const Window w = query_window(a, b, t, tau);
    const float rate = a.gamma[tau] / (float)a.C;
    const float base = window_bases(a, b, w, qf);
    const float sc = w.valid ? score_of(a, b, t, w.k, base, rate, nullptr, nullptr) : -INFINITY;
    const bool hay = w.nvalid > 0;
    const float m = wave_max(sc);
    const float e = w.valid ? expf(sc - m) : 0.f;
    const float den = wave_sum(e);
    const float att = w.valid ? e / den : 0.f;
    const float peak = wave_max(att);
    if (lane == 0) {
      float* st = a.stats + (tok * a.T + tau) * 2;
      st[0] = hay ? m : 0.f;
      st[1] = hay ? den : 1.f;
    }
    if (hay) {
      pt += 1.f;
      best = fmaxf(best, m);
      pico += peak;
      if (tau >= a.T - a.Tc) pctx += 1.f;
    }
    // copy-gather: sum_k att_k V_k, four candidate rows in flight
    for (int c = 0; c < w.nvalid; c += 4) {
      int kc[4];
      float ac[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool ok = c + u < w.nvalid;
        const int ic = ok ? w.first + c + u : w.first;
        kc[u] = readlane_i(w.k, ic);
        const float av = readlane_f(att, ic);
        ac[u] = ok ? av : 0.f;
      }
#pragma unroll
      for (int ch = 0; ch < kMaxDCH; ++ch) {
        if (ch >= a.dch) break;
        const int dd = ch * 256 + lane * 4;
        if (dd < a.d) {
          float4 v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = ld4(Vb + (int64_t)kc[u] * a.d + dd);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            acc[ch].x += ac[u] * v[u].x;
            acc[ch].y += ac[u] * v[u].y;
            acc[ch].z += ac[u] * v[u].z;
            acc[ch].w += ac[u] * v[u].w;
          }
        }
      }
    }
  }
#pragma unroll
  for (int ch = 0; ch < kMaxDCH; ++ch) {
    if (ch >= a.dch) break;
    const int dd = ch * 256 + lane * 4;
    if (dd < a.d) *reinterpret_cast<float4*>(a.salida + tok * a.d + dd) = acc[ch];
  }
  if (lane == 0) {
    float* sg = a.signals + tok * 4;
    sg[0] = pt;
    sg[1] = pt > 0.f ? fmaxf(best, -1e9f) : -1e9f;
    sg[2] = pico;
    sg[3] = pctx;
  }
}

// dot of a 64-lane float4 row chunk set with a register copy, two rows reduced together:
// returns in every lane: lanes < 32 carry the sum for row 0, lanes >= 32 for row 1 (after half_sum)
__device__ __forceinline__ float pair_reduce(float p0, float p1) {
  const int lane = lane_id();
  const float keep = lane < 32 ? p0 : p1;
  const float give = lane < 32 ? p1 : p0;
  return half_sum(keep + __shfl_xor(give, 32, 64));
}

__device__ __forceinline__ float dot4(const float4& x, const float4& y) {
  return x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
}

// ---------------------------------------------------------------------------------------------------------------------
// backward, query pass
// ---------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kWave * kWavesPerBlock) void k_cand_bwd_q(Cand a) {
  const int64_t tok = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (tok >= a.B * a.L) return;
  const int lane = lane_id();
  const int half = lane >> 5;
  const int64_t b = tok / a.L, t = tok % a.L;
  float qf[kMaxFPL], gq[kMaxFPL];
  query_feats(a, tok, qf);
#pragma unroll
  for (int u = 0; u < kMaxFPL; ++u) gq[u] = 0.f;
  float4 dO[kMaxDCH];
#pragma unroll
  for (int ch = 0; ch < kMaxDCH; ++ch) {
    const int dd = ch * 256 + lane * 4;
    dO[ch] = (ch < a.dch && dd < a.d) ? ld4(a.dsal + tok * a.d + dd) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float* Vb = a.V + b * a.L * a.d;
  float dbq = 0.f;
  float dw[17];
#pragma unroll
  for (int c = 0; c < 17; ++c) dw[c] = 0.f;
  float* part = a.partials + tok * (a.T + a.K + 1);

  for (int tau = 0; tau < a.T; ++tau) {
    const Window w = query_window(a, b, t, tau);
    const float rate = a.gamma[tau] / (float)a.C;
    const float base = window_bases(a, b, w, qf);
    float dt = 0.f;
    int ell = 0;
    const float sc = w.valid ? score_of(a, b, t, w.k, base, rate, &dt, &ell) : -INFINITY;
    const float m = wave_max(sc);
    const float e = w.valid ? expf(sc - m) : 0.f;
    const float den = wave_sum(e);
    const float att = w.valid ? e / den : 0.f;
    // dp_i = <dO_q, V_k_i>, two candidates per reduction
    float dp = 0.f;
    for (int c = 0; c < w.nvalid; c += 2) {
      const int i0 = w.first + c;
      const bool two = c + 1 < w.nvalid;
      const int i1 = two ? i0 + 1 : i0;
      const int k0 = readlane_i(w.k, i0);
      const int k1 = readlane_i(w.k, i1);
      float p0 = 0.f, p1 = 0.f;
#pragma unroll
      for (int ch = 0; ch < kMaxDCH; ++ch) {
        const int dd = ch * 256 + lane * 4;
        if (ch < a.dch && dd < a.d) {
          p0 += dot4(dO[ch], ld4(Vb + (int64_t)k0 * a.d + dd));
          if (two) p1 += dot4(dO[ch], ld4(Vb + (int64_t)k1 * a.d + dd));
        }
      }
      const float r = pair_reduce(p0, p1);
      const float r0 = readlane_f(r, 0), r1 = readlane_f(r, 32);
      if (lane == i0) dp = r0;
      if (two && lane == i1) dp = r1;
    }
    const float D = wave_sum(att * dp);
    const float ds = w.valid ? att * (dp - D) : 0.f;
    if (lane == 0) a.qstats[tok * a.T + tau] = D;
    const float sds = wave_sum(ds);
    dbq += -rate * sds;
    const float sdt = wave_sum(ds * dt);
    if (lane == 0) part[tau] = sdt;
#pragma unroll
    for (int c = 0; c < 17; ++c)
      if (c <= a.K && ell == c) dw[c] += ds;
    // d phi_q, d Qc_q: sum_i ds_i [phi_k ; Kc_k], one candidate per half-wave
    for (int c = 0; c < w.nvalid; c += 2) {
      const int i0 = w.first + c;
      const bool two = c + 1 < w.nvalid;
      const int i1 = two ? i0 + 1 : i0;
      const int k0 = readlane_i(w.k, i0);
      const int k1 = readlane_i(w.k, i1);
      const float s0 = readlane_f(ds, i0);
      const float s1v = readlane_f(ds, i1);
      const float s1 = two ? s1v : 0.f;
      const int64_t kk = half ? k1 : k0;
      const float sk = half ? s1 : s0;
      float kf[kMaxFPL];
      key_feats(a, b * a.L + kk, kf);
#pragma unroll
      for (int u = 0; u < kMaxFPL; ++u) gq[u] += sk * kf[u];
    }
  }
  // combine the two halves and write the query-side gradients
#pragma unroll
  for (int u = 0; u < kMaxFPL; ++u) gq[u] += __shfl_xor(gq[u], 32, 64);
  if (half == 0) {
#pragma unroll
    for (int u = 0; u < kMaxFPL; ++u) {
      const int f = lane + 32 * u;
      if (u < a.fpl) {
        if (f < a.P) a.dphi[tok * a.P + f] = gq[u] * a.sp;
        else if (f < a.P + a.cf) a.dQc[tok * a.cf + (f - a.P)] = gq[u] * a.sc;
      }
    }
  }
  for (int c = 0; c <= a.K && c < 17; ++c) {
    const float v = wave_sum(dw[c]);
    if (lane == 0) part[a.T + c] = v;
  }
  if (lane == 0) a.dBt[tok] = (double)dbq;
}

// ---------------------------------------------------------------------------------------------------------------------
// backward, key pass
// ---------------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kWave * kWavesPerBlock) void k_cand_bwd_k(Cand a) {
  const int64_t tok = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (tok >= a.B * a.L) return;
  const int lane = lane_id();
  const int half = lane >> 5;
  const int64_t b = tok / a.L, k = tok % a.L;
  float kf[kMaxFPL], gk[kMaxFPL];
  key_feats(a, tok, kf);
#pragma unroll
  for (int u = 0; u < kMaxFPL; ++u) gk[u] = 0.f;
  float4 vk[kMaxDCH], dv[kMaxDCH];
#pragma unroll
  for (int ch = 0; ch < kMaxDCH; ++ch) {
    const int dd = ch * 256 + lane * 4;
    vk[ch] = (ch < a.dch && dd < a.d) ? ld4(a.V + tok * a.d + dd) : make_float4(0.f, 0.f, 0.f, 0.f);
    dv[ch] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float* dOb = a.dsal + b * a.L * a.d;
  float dla = 0.f, dbk = 0.f;

  for (int tau = 0; tau < a.T; ++tau) {
    const int64_t rowr = b * a.T + tau;
    const int s = a.rank[tok * a.T + tau];
    const int32_t* ids = a.ids_s + rowr * a.L;
    const int my = ids[s];
    const int64_t j = (int64_t)s + 1 + lane;
    const bool valid = lane < a.C && j < a.L && ids[j] == my;
    const int32_t q = valid ? a.order[rowr * a.L + j] : 0;
    const int nvalid = __popcll(__ballot(valid));     // valid lanes are the prefix [0, nvalid)
    if (nvalid == 0) continue;
    const float rate = a.gamma[tau] / (float)a.C;
    // base scores <q_i, k>: the query row is the one loaded per half-wave, pre-scaled as in the forward
    float base = 0.f;
    for (int c = 0; c < nvalid; c += 2) {
      const int q0 = readlane_i(q, c);
      const int q1 = readlane_i(q, c + 1 < a.C ? c + 1 : c);
      const int64_t qq = half ? q1 : q0;
      float qf[kMaxFPL];
      query_feats(a, b * a.L + qq, qf);
      const float tot = half_sum(dot_feats(qf, kf, a.fpl));
      const float t0 = readlane_f(tot, 0), t1 = readlane_f(tot, 32);
      if (lane == c) base = t0;
      if (lane == c + 1) base = t1;
    }
    float att = 0.f, D = 0.f;
    if (valid) {
      const float sc = score_of(a, b, q, k, base, rate, nullptr, nullptr);
      const float* st = a.stats_in + ((b * a.L + q) * a.T + tau) * 2;
      att = expf(sc - st[0]) / st[1];
      D = a.qstats[(b * a.L + q) * a.T + tau];
    }
    // dp_i = <dO_q_i, V_k> and dV_k += att_i dO_q_i from the same loads
    float dp = 0.f;
    for (int c = 0; c < nvalid; c += 2) {
      const bool two = c + 1 < nvalid;
      const int c1 = two ? c + 1 : c;
      const int q0 = readlane_i(q, c);
      const int q1 = readlane_i(q, c1);
      const float a0 = readlane_f(att, c);
      const float a1v = readlane_f(att, c1);
      const float a1 = two ? a1v : 0.f;
      float p0 = 0.f, p1 = 0.f;
#pragma unroll
      for (int ch = 0; ch < kMaxDCH; ++ch) {
        const int dd = ch * 256 + lane * 4;
        if (ch < a.dch && dd < a.d) {
          const float4 o0 = ld4(dOb + (int64_t)q0 * a.d + dd);
          p0 += dot4(o0, vk[ch]);
          dv[ch].x += a0 * o0.x; dv[ch].y += a0 * o0.y; dv[ch].z += a0 * o0.z; dv[ch].w += a0 * o0.w;
          if (two) {
            const float4 o1 = ld4(dOb + (int64_t)q1 * a.d + dd);
            p1 += dot4(o1, vk[ch]);
            dv[ch].x += a1 * o1.x; dv[ch].y += a1 * o1.y; dv[ch].z += a1 * o1.z; dv[ch].w += a1 * o1.w;
          }
        }
      }
      const float r = pair_reduce(p0, p1);
      const float r0 = readlane_f(r, 0), r1 = readlane_f(r, 32);
      if (lane == c) dp = r0;
      if (two && lane == c + 1) dp = r1;
    }
    const float ds = valid ? att * (dp - D) : 0.f;
    dla += ds;
    dbk += rate * ds;
    // d phi_k, d Kc_k: sum_i ds_i [phi_q * scale_phi ; Qc_q * scale_c]
    for (int c = 0; c < nvalid; c += 2) {
      const bool two = c + 1 < nvalid;
      const int c1 = two ? c + 1 : c;
      const int q0 = readlane_i(q, c);
      const int q1 = readlane_i(q, c1);
      const float s0 = readlane_f(ds, c);
      const float s1v = readlane_f(ds, c1);
      const float s1 = two ? s1v : 0.f;
      const int64_t qq = half ? q1 : q0;
      const float sq = half ? s1 : s0;
      float qf[kMaxFPL];
      query_feats(a, b * a.L + qq, qf);
#pragma unroll
      for (int u = 0; u < kMaxFPL; ++u) gk[u] += sq * qf[u];
    }
  }
#pragma unroll
  for (int ch = 0; ch < kMaxDCH; ++ch) {
    const int dd = ch * 256 + lane * 4;
    if (ch < a.dch && dd < a.d) *reinterpret_cast<float4*>(a.dV + tok * a.d + dd) = dv[ch];
  }
#pragma unroll
  for (int u = 0; u < kMaxFPL; ++u) gk[u] += __shfl_xor(gk[u], 32, 64);
  if (half == 0) {
#pragma unroll
    for (int u = 0; u < kMaxFPL; ++u) {
      const int f = lane + 32 * u;
      if (u < a.fpl) {
        if (f < a.P) a.dphi[tok * a.P + f] += gk[u];
        else if (f < a.P + a.cf) a.dKc[tok * a.cf + (f - a.P)] = gk[u];
      }
    }
  }
  const float sla = wave_sum(dla);
  const float sbk = wave_sum(dbk);
  if (lane == 0) {
    a.dla[tok] = sla;
    a.dBt[tok] += (double)sbk;
  }
}

// the candidate lists the kernels walk, materialized: (B, L, T, C) text positions (-1 = none, oldest first) and
// the suffix-match length of each against its query
__global__ __launch_bounds__(kWave * kWavesPerBlock) void k_cand_lists(Cand a, int32_t* __restrict__ pos,
                                                                       int32_t* __restrict__ ell) {
  const int64_t tok = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (tok >= a.B * a.L) return;
  const int lane = lane_id();
  const int64_t b = tok / a.L, t = tok % a.L;
  for (int tau = 0; tau < a.T; ++tau) {
    const Window w = query_window(a, b, t, tau);
    if (lane < a.C) {
      const int64_t o = (tok * a.T + tau) * a.C + lane;
      pos[o] = w.valid ? w.k : -1;
      ell[o] = w.valid ? suffix_match(a.sig + b * a.L, t, w.k, a.K) : -1;
    }
  }
}

static int check_args(const Cand& a, const char* what) {
  ASRN_REQUIRE(a.B >= 0 && a.L >= 0, "%s: bad sizes", what);
  ASRN_REQUIRE(a.L < (int64_t(1) << 31), "%s: L too long", what);
  ASRN_REQUIRE(a.d >= 4 && a.d % 4 == 0 && a.d <= 256 * kMaxDCH, "%s: d=%d must be a multiple of 4 in [4, %d]",
               what, a.d, 256 * kMaxDCH);
  ASRN_REQUIRE(a.C >= 1 && a.C <= 64, "%s: chunk C=%d must be in [1, 64]", what, a.C);
  ASRN_REQUIRE(a.P >= 1 && a.cf >= 1 && a.P + a.cf <= 32 * kMaxFPL, "%s: P + cf = %d must be <= %d", what,
               a.P + a.cf, 32 * kMaxFPL);
  ASRN_REQUIRE(a.K >= 0 && a.K <= 16, "%s: suffix K=%d must be in [0, 16]", what, a.K);
  ASRN_REQUIRE(a.T >= 1 && a.T <= 32 && a.Tc >= 0 && a.Tc <= a.T, "%s: T=%d Tc=%d", what, a.T, a.Tc);
  return 0;
}

static Cand make(const float* phi, const float* V, const float* Qc, const float* Kc, const float* sig,
                 const double* Bt, const float* la, const float* w_suf, const float* gamma, const int32_t* order,
                 const int32_t* ids_s, const int32_t* rank, int64_t B, int64_t L, int d, int P, int cf, int K, int T,
                 int Tc, int C, float sp, float sc) {
  Cand a = {};
  a.phi = phi; a.V = V; a.Qc = Qc; a.Kc = Kc; a.sig = sig; a.Bt = Bt; a.la = la; a.w_suf = w_suf;
  a.gamma = gamma; a.order = order; a.ids_s = ids_s; a.rank = rank;
  a.B = B; a.L = L; a.d = d; a.P = P; a.cf = cf; a.K = K; a.T = T; a.Tc = Tc; a.C = C;
  a.fpl = (P + cf + 31) / 32;
  a.dch = (d + 255) / 256;
  a.sp = sp; a.sc = sc;
  return a;
}

}  // namespace asrn

using namespace asrn;

extern "C" int asrn_candidates_fwd(const float* phi, const float* V, const float* Qc, const float* Kc,
                                   const float* sig, const double* Bt, const float* log_alfa, const float* w_suf,
                                   const float* gamma, const int32_t* order, const int32_t* ids_sorted,
                                   const int32_t* rank, int64_t B, int64_t L, int32_t d, int32_t P, int32_t cf,
                                   int32_t K, int32_t T, int32_t Tc, int32_t C, float scale_phi, float scale_c,
                                   float* salida, float* signals, float* stats, void* stream) {
  Cand a = make(phi, V, Qc, Kc, sig, Bt, log_alfa, w_suf, gamma, order, ids_sorted, rank, B, L, d, P, cf, K, T, Tc,
                C, scale_phi, scale_c);
  if (check_args(a, "asrn_candidates_fwd")) return 1;
  if (B == 0 || L == 0) return 0;
  a.salida = salida; a.signals = signals; a.stats = stats;
  const int64_t blocks = (B * L + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(k_cand_fwd, dim3((unsigned)blocks), dim3(kWave * kWavesPerBlock), 0, (hipStream_t)stream, a);
  return check_launch("asrn_candidates_fwd");
}

extern "C" int asrn_candidates_bwd(const float* phi, const float* V, const float* Qc, const float* Kc,
                                   const float* sig, const double* Bt, const float* log_alfa, const float* w_suf,
                                   const float* gamma, const int32_t* order, const int32_t* ids_sorted,
                                   const int32_t* rank, int64_t B, int64_t L, int32_t d, int32_t P, int32_t cf,
                                   int32_t K, int32_t T, int32_t Tc, int32_t C, float scale_phi, float scale_c,
                                   const float* dsalida, const float* stats, float* dphi, float* dV, float* dQc,
                                   float* dKc, double* dBt, float* dlog_alfa, float* qstats, float* partials,
                                   void* stream) {
  Cand a = make(phi, V, Qc, Kc, sig, Bt, log_alfa, w_suf, gamma, order, ids_sorted, rank, B, L, d, P, cf, K, T, Tc,
                C, scale_phi, scale_c);
  if (check_args(a, "asrn_candidates_bwd")) return 1;
  if (B == 0 || L == 0) return 0;
  a.dsal = dsalida; a.stats_in = stats; a.dphi = dphi; a.dV = dV; a.dQc = dQc; a.dKc = dKc; a.dBt = dBt;
  a.dla = dlog_alfa; a.qstats = qstats; a.partials = partials;
  const int64_t blocks = (B * L + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(k_cand_bwd_q, dim3((unsigned)blocks), dim3(kWave * kWavesPerBlock), 0, (hipStream_t)stream, a);
  if (check_launch("asrn_candidates_bwd/query")) return 1;
  hipLaunchKernelGGL(k_cand_bwd_k, dim3((unsigned)blocks), dim3(kWave * kWavesPerBlock), 0, (hipStream_t)stream, a);
  return check_launch("asrn_candidates_bwd/key");
}

extern "C" int asrn_candidate_lists(const float* sig, const int32_t* order, const int32_t* ids_sorted,
                                    const int32_t* rank, int64_t B, int64_t L, int32_t T, int32_t C, int32_t K,
                                    int32_t* pos, int32_t* ell, void* stream) {
  ASRN_REQUIRE(B >= 0 && L >= 0 && T >= 1 && C >= 1 && C <= 64 && K >= 0 && K <= 16,
               "asrn_candidate_lists: bad sizes B=%lld L=%lld T=%d C=%d K=%d", (long long)B, (long long)L, T, C, K);
  if (B == 0 || L == 0) return 0;
  Cand a = {};
  a.sig = sig; a.order = order; a.ids_s = ids_sorted; a.rank = rank;
  a.B = B; a.L = L; a.T = T; a.C = C; a.K = K;
  const int64_t blocks = (B * L + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(k_cand_lists, dim3((unsigned)blocks), dim3(kWave * kWavesPerBlock), 0, (hipStream_t)stream, a,
                     pos, ell);
  return check_launch("asrn_candidate_lists");
}
