// general.hpp — the conservative bin bounds of a general row, computed once per row by
// k_finalize from k_stream's per-chunk coarse histograms and read by k_collect / k_final.
//
// Each chunk bin (width 1/2 over d = m_chunk - l) lands somewhere in a range of global
// bins (width 1/CB_SCALE over d = m_row - l); placing every chunk bin at its earliest and
// at its latest global bin gives cumulative upper and lower bounds on the mass and count
// above any global bin, from which the top-k / top-p / min-p / draw thresholds are bounded
// to bin ranges. Integer (fixed-point) sums make the result independent of the order of
// the atomics.
#pragma once
#include "kernels.hpp"

namespace strim {

// First g in [lo, hi] with pred(g), hi + 1 if none, for a predicate monotone in g
// (false ... false true ... true). One wave: lane l tests bins l, l + 64, l + 128.
static_assert(NGB <= 3 * WAVE, "three bins per lane");
template <typename F>
__device__ __forceinline__ int first_true(int lo, int hi, F pred) {
  const int lane = threadIdx.x & (WAVE - 1);
  int res = hi + 1;
#pragma unroll
  for (int k = 2; k >= 0; --k) {
    const int g = lane + k * WAVE;
    const uint64_t bal = __ballot(g >= lo && g <= hi && g < NGB && pred(g));
    if (bal) res = k * WAVE + (int)__ffsll((long long)bal) - 1;
  }
  return res;
}

// Conservative bin bounds of a general row from the coarse chunk histograms
// (one wave, every lane computing the same scalars; the same arithmetic in every
// workgroup of the row gives the same result).
// cU/cL: cumulative fixed-point mass with each chunk bin placed at its earliest /
// latest possible global bin; kU/kL: the same for counts.
__device__ void compute_bounds(const Args& a, int r, const RowParams& p, float m, uint32_t N,
                               const unsigned long long* cU, const unsigned long long* cL,
                               const uint32_t* kU, const uint32_t* kL, Bounds& out) {
  const int lane = threadIdx.x & (WAVE - 1);
  Bounds bd;  // built in registers (uniform), stored by lane 0
  const double inv = 1.0 / FIX_SCALE, EPS = 1e-5;
  const double SLACK = (double)(a.W * NCB + 16) * 4.0 * inv;
  auto MU = [&](int g) { return g < 0 ? 0.0 : (double)cU[g] * inv * (1.0 + EPS) + SLACK; };
  auto ML = [&](int g) { return g < 0 ? 0.0 : (double)cL[g] * inv * (1.0 - EPS) - SLACK; };
  int s1 = NGB, e1 = NGB - 1;
  if (p.min_p > 0.0f) {
    const double thr = -p.lmp;
    const int gt = thr < 63.0 ? (int)(thr * (double)CB_SCALE) : NGB - 1;
    s1 = min(s1, max(0, gt - 1));
    e1 = min(e1, min(NGB - 1, gt + 1));
  }
  const bool topk = p.top_k > 0 && p.top_k < a.V;
  if (topk && N > (uint32_t)p.top_k) {
    const uint32_t K = (uint32_t)p.top_k;
    const int glo = first_true(0, NGB - 1, [&](int g) { return kU[g] >= K; });
    const int ghi = first_true(0, NGB - 1, [&](int g) { return kL[g] >= K; });
    s1 = min(s1, glo);
    e1 = min(e1, ghi);
  }
  int s = s1, e = e1;
  const bool topp = p.top_p < 1.0f;
  if (topp) {
    const double P = (double)p.top_p;
    const double hi = MU(e1), lo = ML(s1 - 1);
    const int lim = min(e1, s1 - 1);
    int ep = e1;
    if (lim >= 0) {
      const int f = first_true(0, lim, [&](int g) { return ML(g) > P * hi; });
      if (f <= lim) ep = f;
    }
    const int sp = first_true(0, NGB - 1, [&](int g) { return MU(g) > P * lo; });
    e = min(e1, ep);
    s = min(s1, sp);
  }
  if (s > e + 1) s = e + 1;
  const bool icdf = a.noise_mode == STRIM_NOISE_ICDF;
  const bool by_rank = (p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp;
  for (int q = 0; q < 3; ++q) { bd.rng[q][0] = 1; bd.rng[q][1] = 0; }
  int mode;
  if (kU[e1] <= (uint32_t)CAP) {
    mode = MODE_A;  // everything possibly pre-kept is collected
    bd.rng[0][0] = 0;
    bd.rng[0][1] = e1;
    s = 0;
  } else if (by_rank) {
    mode = MODE_NONE;
  } else {
    mode = MODE_B;
    bd.rng[0][0] = s;
    bd.rng[0][1] = e;
    if (s1 <= e1) { bd.rng[1][0] = s1; bd.rng[1][1] = e1; }
    if (icdf) {
      const double u = (double)row_uniform(a, r, p, 0);
      double wd = 0.0;
      if (a.verify) {
        int bb, jj;
        row_bj(a, r, bb, jj);
        const float ld = a.s.rs[r].l_draft;
        if (jj < a.k && ld > -INFINITY) wd = exp((double)ld - (double)m);
      }
      const double tlo = u * (ML(s - 1) - wd) - SLACK;
      const double thi = u * MU(e) + wd + SLACK;
      const int dlo = first_true(0, NGB - 1, [&](int g) { return MU(g) > tlo; });
      int dhi = first_true(0, NGB - 1, [&](int g) { return ML(g) > thi; });
      dhi = min(dhi, e);
      bd.rng[2][0] = dlo;
      bd.rng[2][1] = dhi;
    }
    // upper bound of the tokens in the collected bins: per contiguous run [lo, hi],
    // kU[hi] - kL[lo - 1] (never negative: kU >= kL bin by bin, and both are cumulative)
    uint32_t part = 0u;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int g = lane + k * WAVE;
      if (g >= NGB || !in_rng(bd, g)) continue;
      if (g + 1 >= NGB || !in_rng(bd, g + 1)) part += kU[g];
      if (g > 0 && !in_rng(bd, g - 1)) part -= kL[g - 1];
    }
    const uint32_t total = (uint32_t)wave_sum((int)part);
    if (total > (uint32_t)CAP) mode = MODE_NONE;
  }
  // non-collected intervals, split where the kept / pre-kept classification changes
  // (a new interval starts after a collected bin and at s and s1); more than NSEG
  // intervals leave the row to the exact resolution
  for (int q = 0; q < NSEG; ++q) { bd.seg_lo[q] = 1; bd.seg_hi[q] = 0; }
  if (mode != MODE_NONE) {
    uint64_t stm[3], enm[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int g = lane + k * WAVE;
      const bool out_g = g < NGB && !in_rng(bd, g);
      stm[k] = __ballot(out_g && (g == 0 || in_rng(bd, g - 1) || g == s || g == s1));
      enm[k] = __ballot(out_g && (g == NGB - 1 || in_rng(bd, g + 1) || g + 1 == s || g + 1 == s1));
    }
    // the q-th start and the q-th end delimit interval q (they alternate bin by bin)
    int q = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      uint64_t ms = stm[k];
      while (ms) {
        if (q < NSEG) bd.seg_lo[q] = k * WAVE + (int)__ffsll((long long)ms) - 1;
        ms &= ms - 1ull;
        ++q;
      }
    }
    if (q > NSEG) mode = MODE_NONE;
    q = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      uint64_t me = enm[k];
      while (me) {
        if (q < NSEG) bd.seg_hi[q] = k * WAVE + (int)__ffsll((long long)me) - 1;
        me &= me - 1ull;
        ++q;
      }
    }
  }
  bd.mode = mode;
  bd.s = s;
  bd.e = e;
  bd.s1 = s1;
  bd.e1 = e1;
  if (lane == 0) out = bd;
}

// LDS of general_bounds (overlaid on k_finalize's candidate keys).
struct GenShared {
  unsigned long long U[NGB], L[NGB];
  uint32_t kU[NGB], kL[NGB];
  float cm[256];  // per chunk: its maximum
  uint32_t n;     // live tokens of the row
};

// Bounds of row r into rs[r].bd, by one NT-thread workgroup whose thread t < W holds the
// statistics cs of chunk t (own = t < W). m is the row maximum.
template <int NT>
__device__ void general_bounds(const Args& a, int r, const RowParams& p, float m,
                               const ChunkStat& cs, bool own, GenShared& G) {
  static_assert(NT / WAVE >= 4 && NT >= 256, "four prefix waves; one chunk per thread");
  static_assert(NGB <= 3 * WAVE, "prefix layout");
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
  for (int g = t; g < NGB; g += NT) {
    G.U[g] = 0ull; G.L[g] = 0ull; G.kU[g] = 0u; G.kL[g] = 0u;
  }
  if (own) G.cm[t] = cs.m;
  if (t == 0) G.n = 0u;
  const int nw = wave_sum(own ? (int)cs.n : 0);
  __syncthreads();
  if (lane == 0) atomicAdd(&G.n, (uint32_t)nw);
  // every chunk bin spread over [glo, ghi] of the global bins (batches of loads from
  // clamped indices with no branch between them)
  constexpr int BB = 8;
  const int nbin = a.W * NCB;
  for (int e0 = t; e0 < nbin; e0 += BB * NT) {
    uint32_t cn[BB];
    unsigned long long hm[BB];
#pragma unroll
    for (int q = 0; q < BB; ++q) {
      const int e = e0 + q * NT < nbin ? e0 + q * NT : 0;
      const int64_t o = (int64_t)r * a.s.wmax * NCB + e;
      cn[q] = a.s.chc[o];
      hm[q] = a.s.chm[o];
    }
#pragma unroll
    for (int q = 0; q < BB; ++q) {
      const int e = e0 + q * NT;
      if (e >= nbin || !cn[q]) continue;
      const int cc = e / NCB, bb = e - cc * NCB;
      const double dlt = (double)m - (double)G.cm[cc];
      const double lo = (dlt + 0.5 * bb) * (1.0 - 2e-6) * CB_SCALE;
      const double hi = bb == NCB - 1 ? 1e300 : (dlt + 0.5 * (bb + 1)) * (1.0 + 2e-6) * CB_SCALE;
      const int glo = lo < (double)(NGB - 1) ? max(0, (int)floor(lo)) : NGB - 1;
      const int ghi = hi < (double)(NGB - 1) ? max(0, (int)floor(hi)) : NGB - 1;
      const double ms = (double)hm[q] * exp(-dlt);
      atomicAdd(&G.U[glo], (unsigned long long)(ms + 1.0));
      atomicAdd(&G.L[ghi], (unsigned long long)ms);
      atomicAdd(&G.kU[glo], cn[q]);
      atomicAdd(&G.kL[ghi], cn[q]);
    }
  }
  __syncthreads();
  // inclusive prefixes over the global bins, one array per wave: a lane owns bins
  // 3 lane .. 3 lane + 2
  if (w < 4) {
    const int g0 = 3 * lane;
    if (w < 2) {
      unsigned long long* arr = w == 0 ? G.U : G.L;
      unsigned long long v3[3], sum = 0ull;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        v3[q] = g0 + q < NGB ? arr[g0 + q] : 0ull;
        sum += v3[q];
      }
      unsigned long long run = wave_incl_scan_u64(sum) - sum;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        run += v3[q];
        if (g0 + q < NGB) arr[g0 + q] = run;
      }
    } else {
      uint32_t* arr = w == 2 ? G.kU : G.kL;
      uint32_t v3[3], sum = 0u;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        v3[q] = g0 + q < NGB ? arr[g0 + q] : 0u;
        sum += v3[q];
      }
      uint32_t run = wave_incl_scan_u32(sum) - sum;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        run += v3[q];
        if (g0 + q < NGB) arr[g0 + q] = run;
      }
    }
  }
  __syncthreads();
  if (w == 0) compute_bounds(a, r, p, m, G.n, G.U, G.L, G.kU, G.kL, a.s.rs[r].bd);
}

}  // namespace strim
