// exact.hpp — the exact streaming resolution of one row by one workgroup of NT threads.
//
// Used for the rows whose candidates do not fit a finalize's LDS (flat or tie-heavy rows,
// nuclei wider than the capacity, local candidate overflow). It needs nothing from the
// candidate pipeline: every decision re-streams the row's raw logits.
#pragma once

#include "select.hpp"

namespace strim {

// Rows whose candidates do not fit the finalize (flat or tie-heavy rows, nuclei wider
// than CAP, local candidate overflow) are decided here. Every decision is a weighted
// radix select over the order keys: level 0 bins d = m - l at 1/64 nat; deeper levels
// take 12 bits at a time of the compact key (fkey_desc(l) << 20 | id) inside the chosen
// bucket, until it holds at most XCOL tokens, which are gathered, sorted in LDS and
// resolved exactly. Each level is one streaming pass over the raw logits that recomputes
// the processing chain (history counts per window of NT * EPT tokens). Masses are fixed
// point, 2^43 per unit of exp(l - m), so every sum is exact and independent of order.
constexpr int XB = 4096;            // digits per level
constexpr int XCOL = 4096;          // bucket size resolved in LDS
constexpr double XFIX = 8796093022208.0;  // 2^43

struct XState {
  uint64_t below_m, key, key_w, tot_m;
  uint32_t below_c, cnt, tot_c, ncol;
  int32_t found, token;
};

// The tokens a select ranges over: allowed, passing min-p (lmp = log(min_p), -inf for
// none), with order key in [lo, bound], other than `excl`. rS != 0: the weights are the
// general-q residual max(0, p - q) scaled by the kept mass rS (see x_wt_q).
struct XUni {
  float m;
  double lmp;
  uint64_t lo, bound;
  int excl;
  uint64_t rS;
};

// The draft distribution q of a general-q verify row: softmax(draft logits / T) over the
// draft vocabulary, whose ids are the table's (membership bitmap dbits). A member id's
// table index is its rank among the members, wrank[id / 32] plus the member bits below
// it in its word (the table ascends), so v = draft_logit / T is read from the row's
// draft logits at that index.
struct XQ {
  const uint32_t* dbits;
  const uint32_t* wrank;
  const void* dlog;  // the row's draft logits [Vd], of dtype dt
  int32_t dt;
  float T;
  float mq;
  double Z;
};
// v at member id, given its membership word and rank word
__device__ __forceinline__ float xq_v(const XQ& q, int id, uint32_t bits, uint32_t rank) {
  const int i = (int)rank + __popc(bits & ((1u << (id & 31)) - 1u));
  const float x = q.dt == STRIM_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)q.dlog)[i])
                                           : ((const float*)q.dlog)[i];
  return x / q.T;
}
// The q of draft row qr (b * k + j) of a general-q verify launch (q_base: without its
// maximum and sum).
__device__ __forceinline__ XQ q_base(const Args& a, int qr) {
  XQ q;
  q.dbits = a.s.dbits;
  q.wrank = a.s.wrank;
  q.dt = a.dtype;
  q.dlog = a.dtype == STRIM_DTYPE_BF16
               ? (const void*)((const uint16_t*)a.dlog + (size_t)qr * (size_t)a.Vd)
               : (const void*)((const float*)a.dlog + (size_t)qr * (size_t)a.Vd);
  q.T = a.p[qr / a.k].temperature;
  q.mq = 0.0f;
  q.Z = 1.0;
  return q;
}
__device__ __forceinline__ XQ q_of_row(const Args& a, int qr) {
  const QStat qs = a.s.qst[qr];
  XQ q = q_base(a, qr);
  q.mq = qs.mq;
  q.Z = qs.Z;
  return q;
}
// q(id): exp(v - mq) / Z, 0 outside the table.
__device__ __forceinline__ double xq_prob(const XQ& q, int id) {
  const uint32_t bits = q.dbits[id >> 5];
  if (!((bits >> (id & 31)) & 1u)) return 0.0;
  return exp((double)xq_v(q, id, bits, q.wrank[id >> 5]) - (double)q.mq) / q.Z;
}

// The fields of Args the streaming passes read (the exact path is one out-of-line call,
// so the 3 KB launch block is not copied to private memory).
struct XArgs {
  const void* logits;
  int64_t row_stride;
  int32_t dtype, vec_ok, V, H, verify, k, noise_mode;
  const uint32_t* mask;
  int64_t mask_stride;
  const int32_t* hist;
  const int32_t* hist_len;
  const int32_t* drafts;
  const float* noise;
  int64_t noise_stride;
  int32_t has_q;  // a general-q verify row (q below)
  XQ q;
};

__device__ __forceinline__ bool x_in(const XUni& u, float l, int id) {
  if (!(l > -INFINITY) || !((double)l - (double)u.m >= u.lmp) || id == u.excl) return false;
  const uint64_t k = ckey(l, id);
  return k >= u.lo && k <= u.bound;
}
// Fixed-point weight of a token, round(2^43 * exp(l - m)), from the float exp of the
// float difference: within 2^-23 relative of the exact weight (far inside the 1e-6
// decision tolerance) and the same value in every pass, at a fraction of a double exp's
// cost (one workgroup computes it for every token of the row, once per pass).
__device__ __forceinline__ uint64_t x_weight(float l, float m) {
  return (uint64_t)(expf(l - m) * 8796093022208.0f + 0.5f);
}
// Weight of a universe token: exp(l - m) in fixed point, or, for a residual universe,
// max(0, W - round(q * rS)): the residual (p - q)^+ in units of the kept mass rS.
__device__ __forceinline__ uint64_t x_wt_q(const XUni& u, float l, double q) {
  const uint64_t W = x_weight(l, u.m);
  if (u.rS == 0ull || q == 0.0) return W;
  const uint64_t qS = (uint64_t)__double2ull_rn(q * (double)u.rS);
  return W > qS ? W - qS : 0ull;
}
// q from a streamed draft value (-inf: not in the table)
__device__ __forceinline__ double xq_of(const XQ& q, float v) {
  return v > -INFINITY ? exp((double)v - (double)q.mq) / q.Z : 0.0;
}
// Level-0 digit: floor(64 (m - l)), tail at XB - 1; monotone in the order.
__device__ __forceinline__ int x_dbin(float l, float m) {
  const double d = (double)m - (double)l;
  return d < (double)(XB - 1) / 64.0 ? (int)(d * 64.0) : XB - 1;
}
__device__ __forceinline__ uint64_t x_ck(float l, int id) {
  return ((uint64_t)fkey_desc(l) << 20) | (uint32_t)id;
}
// First fkey in [lo, hi] whose float satisfies a predicate that is monotone (false, then
// true) along the order; hi + 1 if none.
template <typename F>
__device__ __forceinline__ uint32_t x_first_fkey(uint32_t lo, uint32_t hi, F pred) {
  uint64_t L = lo, H = (uint64_t)hi + 1;
  while (L < H) {
    const uint64_t mid = (L + H) >> 1;
    if (pred(fkey_desc_inv((uint32_t)mid))) H = mid;
    else L = mid + 1;
  }
  return (uint32_t)L;
}

// One streaming pass over the row: fn(i0, l, qv) for every thread and window, with qv
// the draft values v of a general-q row's tokens (-inf outside the table; all -inf for
// other rows). Aligned rows keep xpd() windows of loads in flight; rows with penalties
// hold the history ids in registers (when they fit) and rebuild each window's counts in
// LDS while the next windows' loads are in flight. Unaligned rows load each window when
// they reach it.
// windows of loads in flight: 1024-thread workgroups have half the registers per thread
template <int NT>
constexpr int xpd() { return NT >= 1024 ? 2 : 4; }
template <int NT, bool BF16, bool Q, bool PEN, typename F>
__device__ __forceinline__ void x_pass_pipe(const XArgs& a, int r, int b, int j,
                                            const RowParams& p, uint32_t* s_cnt, F&& fn) {
  constexpr int XPD = xpd<NT>();
  constexpr int WIN = NT * EPT;
  const int t = threadIdx.x;
  int hid[hpt<NT>()];
  int hl = 0;
  if constexpr (PEN) {
    hist_load<NT>(a, b, hid);
    hl = hist_len(a, b);
    // the history ids arrive before the window loads are issued: inside the window loop
    // a load from before it would make every window wait for all of its loads
    __builtin_amdgcn_s_waitcnt(0);
  }
  const int64_t base = (int64_t)r * a.row_stride;
  const int nwin = (a.V + WIN - 1) / WIN;
  const uint8_t* mrow = a.mask ? (const uint8_t*)(a.mask + (int64_t)r * a.mask_stride)
                               : (const uint8_t*)a.logits;
  // the streamed arrays as global pointers (this runs inside an out-of-line call)
  const glb_t<const uint8_t>* lg = (const glb_t<const uint8_t>*)a.logits;
  const glb_t<const uint8_t>* mg = (const glb_t<const uint8_t>*)mrow;
  const glb_t<const uint32_t>* qdb = (const glb_t<const uint32_t>*)a.q.dbits;
  const glb_t<const uint32_t>* qrk = (const glb_t<const uint32_t>*)a.q.wrank;
  // (clang vector types: the HIP vector classes cannot be assigned from a global
  // reference)
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  struct Slot {
    u32x4 x0, x1;
    uint32_t mb, qb, qr;
  };
  Slot sl[XPD];
  // every load of a window from a clamped index, no branch between them; a segment that
  // ends past the row end (V not a multiple of 8) is left to the tail step below
  auto issue = [&](Slot& sd, int w) {
    const int i0 = w * WIN + t * EPT;
    const int ii = i0 + EPT <= a.V ? i0 : 0;
    if constexpr (BF16) {
      sd.x0 = *(const glb_t<const u32x4>*)(lg + 2 * (base + ii));
    } else {
      sd.x0 = *(const glb_t<const u32x4>*)(lg + 4 * (base + ii));
      sd.x1 = *(const glb_t<const u32x4>*)(lg + 4 * (base + ii + 4));
    }
    sd.mb = mg[a.mask ? (ii >> 3) : 0];
    if constexpr (Q) {
      sd.qb = qdb[ii >> 5];
      sd.qr = qrk[ii >> 5];
    }
  };
#pragma unroll
  for (int d = 0; d < XPD; ++d) issue(sl[d], d);
  for (int w = 0; w < nwin; w += XPD) {
#pragma unroll
    for (int d = 0; d < XPD; ++d) {
      if (w + d < nwin) {
        const int i0 = (w + d) * WIN + t * EPT;
        // this window's history counts (uniform: every thread takes the barriers)
        if constexpr (PEN) hist_count<NT, WIN>(a, b, j, (w + d) * WIN, hid, hl, s_cnt);
        const Slot& sd = sl[d];
        float x[EPT];
        if constexpr (BF16) {
          const uint32_t wv[4] = {sd.x0.x, sd.x0.y, sd.x0.z, sd.x0.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[2 * e] = __uint_as_float(wv[e] << 16);
            x[2 * e + 1] = __uint_as_float(wv[e] & 0xFFFF0000u);
          }
        } else {
          const uint32_t wv[8] = {sd.x0.x, sd.x0.y, sd.x0.z, sd.x0.w,
                                  sd.x1.x, sd.x1.y, sd.x1.z, sd.x1.w};
#pragma unroll
          for (int e = 0; e < EPT; ++e) x[e] = __uint_as_float(wv[e]);
        }
        if constexpr (PEN) {
          // the penalties as process_tokens applies them, one rounding per step
#pragma unroll
          for (int e = 0; e < EPT; ++e) {
            const uint32_t c = s_cnt[t * EPT + e];
            if (c > 0u) {
              float v = x[e];
              v = v > 0.0f ? v / p.rep : v * p.rep;
              v = v - p.freq * (float)c;
              x[e] = v - p.pres;
            }
          }
        }
        const uint32_t bits = a.mask ? ((uint32_t)sd.mb & 0xFFu) : 0xFFu;
        float l[EPT], qv[EPT];
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const bool ok = (i0 + EPT <= a.V) && ((bits >> e) & 1u);
          l[e] = ok ? (p.greedy ? x[e] : x[e] / p.T) : -INFINITY;
          qv[e] = -INFINITY;
          if constexpr (Q) {
            // (the members' draft logits: a dependent read of the row's draft logits,
            // which stay in the caches)
            const int id = i0 + e;
            if (i0 + EPT <= a.V && ((sd.qb >> (id & 31)) & 1u)) qv[e] = xq_v(a.q, id, sd.qb, sd.qr);
          }
        }
        fn(i0, l, qv);
        // every wave has read this window's counts before the next window's hist_count
        // clears them (its first step runs before its own barrier)
        if constexpr (PEN) __syncthreads();
      }
      issue(sl[d], w + d + XPD);
    }
  }
  // tail: the partial last segment, by its owner with element loads (all -inf elsewhere)
  if (a.V % EPT) {
    const int iP = a.V & ~(EPT - 1);
    const bool own = t == (iP % WIN) / EPT;
    const uint32_t bits = (own && a.mask) ? (uint32_t)mrow[iP >> 3] : 0xFFu;
    float l[EPT], qv[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int id = iP + e;
      const bool ok = own && id < a.V && ((bits >> e) & 1u);
      const int ic = ok ? id : 0;
      float x = BF16 ? bf16_to_f32(((const uint16_t*)a.logits)[base + ic])
                     : ((const float*)a.logits)[base + ic];
      if constexpr (PEN) {
        // the last window's counts are still in s_cnt (it holds the tail)
        const uint32_t c = s_cnt[(iP % WIN) + e];
        if (c > 0u) {
          x = x > 0.0f ? x / p.rep : x * p.rep;
          x = x - p.freq * (float)c;
          x = x - p.pres;
        }
      }
      l[e] = ok ? (p.greedy ? x : x / p.T) : -INFINITY;
      qv[e] = -INFINITY;
      if constexpr (Q) {
        if (ok && ((a.q.dbits[id >> 5] >> (id & 31)) & 1u))
          qv[e] = xq_v(a.q, id, a.q.dbits[id >> 5], a.q.wrank[id >> 5]);
      }
    }
    fn(iP, l, qv);
  }
}
// HQ: the caller may resolve general-q verify rows (the draft distribution's code is
// compiled only then).
template <int NT, bool HQ, typename F>
__device__ __forceinline__ void x_pass(const XArgs& a, int r, int b, int j, const RowParams& p,
                                       uint32_t* s_cnt, F&& fn) {
  const bool hq = HQ && a.has_q;
  if (a.vec_ok && !(hq && p.pen)) {
    if (a.dtype == STRIM_DTYPE_BF16) {
      if (hq) x_pass_pipe<NT, true, true, false>(a, r, b, j, p, s_cnt, fn);
      else if (p.pen) x_pass_pipe<NT, true, false, true>(a, r, b, j, p, s_cnt, fn);
      else x_pass_pipe<NT, true, false, false>(a, r, b, j, p, s_cnt, fn);
    } else {
      if (hq) x_pass_pipe<NT, false, true, false>(a, r, b, j, p, s_cnt, fn);
      else if (p.pen) x_pass_pipe<NT, false, false, true>(a, r, b, j, p, s_cnt, fn);
      else x_pass_pipe<NT, false, false, false>(a, r, b, j, p, s_cnt, fn);
    }
    return;
  }
  const int t = threadIdx.x;
  for (int w0 = 0; w0 < a.V; w0 += NT * EPT) {
    const int i0 = w0 + t * EPT;
    float x[EPT];
    load_tokens(a, r, i0, x);
    if (p.pen) build_counts_span<NT, NT * EPT>(a, b, j, w0, s_cnt);
    float l[EPT], qv[EPT];
    bool nf = false;
    process_tokens(a, r, i0, p, s_cnt + t * EPT, x, l, nf);
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      qv[e] = -INFINITY;
      if (hq && i0 + e < a.V) {
        const int id = i0 + e;
        if ((a.q.dbits[id >> 5] >> (id & 31)) & 1u)
          qv[e] = xq_v(a.q, id, a.q.dbits[id >> 5], a.q.wrank[id >> 5]);
      }
    }
    fn(i0, l, qv);
    if (p.pen) __syncthreads();  // the next window rebuilds the counts
  }
}

// Interval of one select level: mode 0 = level-0 bins, 1 = compact-key digits of
// [klo, khi] shifted right by `shift`, 2 = everything in digit 0.
struct XLevel {
  int mode, shift;
  uint64_t klo, khi;
};
__device__ __forceinline__ int x_digit(const XLevel& lv, float l, int id, float m) {
  if (lv.mode == 0) return x_dbin(l, m);
  if (lv.mode == 2) return 0;
  const uint64_t ck = x_ck(l, id);
  return (ck >= lv.klo && ck <= lv.khi) ? (int)((ck - lv.klo) >> lv.shift) : -1;
}

// Count and fixed-point mass per digit of the universe's tokens inside the level.
// Each thread accumulates runs of equal digits and flushes a run with one LDS atomic.
template <int NT, bool HQ>
__device__ __forceinline__ void x_hist(const XArgs& a, int r, int b, int j, const RowParams& p, const XUni& u,
                       const XLevel& lv, uint32_t* s_cnt, uint32_t* s_hc, uint64_t* s_hm) {
  for (int i = threadIdx.x; i < XB; i += NT) {
    s_hc[i] = 0u;
    s_hm[i] = 0ull;
  }
  __syncthreads();
  int cur = -1;
  uint32_t ac = 0u;
  uint64_t am = 0ull;
  x_pass<NT, HQ>(a, r, b, j, p, s_cnt, [&](int i0, const float (&l)[EPT], const float (&qv)[EPT]) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (!x_in(u, l[e], i0 + e)) continue;
      const int dg = x_digit(lv, l[e], i0 + e, u.m);
      if (dg < 0) continue;
      if (dg != cur) {
        if (cur >= 0) {
          atomicAdd(&s_hc[cur], ac);
          atomicAdd((unsigned long long*)&s_hm[cur], (unsigned long long)am);
        }
        cur = dg;
        ac = 0u;
        am = 0ull;
      }
      ac += 1u;
      am += x_wt_q(u, l[e], (HQ && u.rS != 0ull) ? xq_of(a.q, qv[e]) : 0.0);
    }
  });
  if (cur >= 0) {
    atomicAdd(&s_hc[cur], ac);
    atomicAdd((unsigned long long*)&s_hm[cur], (unsigned long long)am);
  }
  __syncthreads();
}

// Gathers the order keys of the universe's tokens inside the level's digit `dg` (all of
// them for mode 2) into s_col; returns their number (<= XCOL by construction).
template <int NT, bool HQ>
__device__ __forceinline__ int x_collect(const XArgs& a, int r, int b, int j, const RowParams& p, const XUni& u,
                         const XLevel& lv, int dg, uint32_t* s_cnt, uint64_t* s_col,
                         lds_t<XState>& s_x) {
  const int lane = threadIdx.x & (WAVE - 1);
  if (threadIdx.x == 0) s_x.ncol = 0u;
  __syncthreads();
  x_pass<NT, HQ>(a, r, b, j, p, s_cnt, [&](int i0, const float (&l)[EPT], const float (&)[EPT]) {
    uint32_t sel = 0u;
    int c = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (x_in(u, l[e], i0 + e) && x_digit(lv, l[e], i0 + e, u.m) == dg) {
        sel |= 1u << e;
        ++c;
      }
    int tot;
    const int ex = wave_excl_count(c, &tot);
    if (tot > 0) {
      uint32_t base = 0u;
      if (lane == 0) base = atomicAdd((uint32_t*)&s_x.ncol, (uint32_t)tot);
      base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
      uint32_t pos = base + (uint32_t)ex;
#pragma unroll
      for (int e = 0; e < EPT; ++e)
        if ((sel >> e) & 1u) {
          if (pos < (uint32_t)XCOL) s_col[pos] = ckey(l[e], i0 + e);
          ++pos;
        }
    }
  });
  __syncthreads();
  const int n = (int)s_x.ncol;
  return n < XCOL ? n : XCOL;
}

// Ascending in-place sort of s_col[0, n), n <= XCOL (keys are unique; s_col holds XCOL).
template <int NT>
__device__ __forceinline__ void x_sort(uint64_t* s_col, int n) {
  if (n <= NT) rank_sort<NT>(s_col, n);
  else bitonic_sort_lds<NT>(s_col, n);
}

// The LDS arrays of the exact resolution (address-space-typed: see lds_t).
struct XScratch {
  lds_t<uint64_t>* key_;  // XB u64 histogram masses, then the gathered bucket
  lds_t<uint32_t>* hc_;   // XB u32 histogram counts
  lds_t<uint32_t>* cnt_;  // NT * EPT u32 history counts of a window
  lds_t<uint64_t>* u2_;   // 2 * NT / WAVE
  lds_t<double>* dred_;
  lds_t<uint64_t>* ured_;
  lds_t<int>* ired_;
  __device__ __forceinline__ uint64_t* key() const { return (uint64_t*)key_; }
  __device__ __forceinline__ uint32_t* hc() const { return (uint32_t*)hc_; }
  __device__ __forceinline__ uint32_t* cnt() const { return (uint32_t*)cnt_; }
  __device__ __forceinline__ uint64_t* u2() const { return (uint64_t*)u2_; }
  __device__ __forceinline__ double* dred() const { return (double*)dred_; }
  __device__ __forceinline__ uint64_t* ured() const { return (uint64_t*)ured_; }
  __device__ __forceinline__ int* ired() const { return (int*)ired_; }
};
// An XScratch over a caller's LDS arrays.
__device__ __forceinline__ XScratch xscratch(uint64_t* key, uint32_t* hc, uint32_t* cnt,
                                             uint64_t* u2, double* dred, uint64_t* ured,
                                             int* ired) {
  return XScratch{(lds_t<uint64_t>*)key, (lds_t<uint32_t>*)hc, (lds_t<uint32_t>*)cnt,
                  (lds_t<uint64_t>*)u2, (lds_t<double>*)dred, (lds_t<uint64_t>*)ured,
                  (lds_t<int>*)ired};
}

// Weighted select: the last universe token x in the order whose universe mass before it
// (by_mass) or count before it is <= T, where T = floor(coef * total mass) of the
// universe, or T = cst when coef < 0. Result in s_x (found = 0 for an empty universe).
template <int NT, bool HQ>
__device__ __noinline__ void x_select(const XArgs& a_in, int r, int b, int j,
                                      const RowParams p_in, const XUni u_in, bool by_mass,
                                      double coef, uint64_t cst, const XScratch xs_in,
                                      lds_t<XState>& s_x) {
  // the uniform arguments in scalar registers (see uniform_copy)
  const XArgs a = uniform_copy(a_in);
  const RowParams p = uniform_copy(p_in);
  const XUni u = uniform_copy(u_in);
  const XScratch xs = uniform_copy(xs_in);
  r = __builtin_amdgcn_readfirstlane(r);
  b = __builtin_amdgcn_readfirstlane(b);
  j = __builtin_amdgcn_readfirstlane(j);
  constexpr int XQ = XB / NT;  // bins (and bucket positions) per thread
  const int t = threadIdx.x;
  XLevel lv{0, 0, 0ull, 0ull};
  uint64_t below_m = 0ull, below_c = 0ull, T = 0ull;
  int dsel = -1;
  for (;;) {
    x_hist<NT, HQ>(a, r, b, j, p, u, lv, xs.cnt(), xs.hc(), xs.key());
    uint32_t c4[XQ];
    uint64_t m4[XQ], lc = 0ull, lm = 0ull;
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      c4[q] = xs.hc()[XQ * t + q];
      m4[q] = xs.key()[XQ * t + q];
      lc += c4[q];
      lm += m4[q];
    }
    uint64_t exc, exm, totc, totm;
    block_excl_scan2_u64<NT>(lc, lm, xs.u2(), exc, exm, totc, totm);
    if (lv.mode == 0) {
      T = coef < 0.0 ? cst : (uint64_t)floor(coef * (double)totm);
      if (t == 0) {
        s_x.tot_c = (uint32_t)totc;
        s_x.tot_m = totm;
      }
    }
    int best = -1;
    uint64_t bc = 0ull, bm = 0ull;
    uint32_t bn = 0u;
    uint64_t fc = below_c + exc, fm = below_m + exm;
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      if (c4[q] > 0u && (by_mass ? fm : fc) <= T) {
        best = XQ * t + q;
        bc = fc;
        bm = fm;
        bn = c4[q];
      }
      fc += c4[q];
      fm += m4[q];
    }
    dsel = -block_min<NT>(-best, xs.ired());
    if (dsel < 0) {
      if (t == 0) s_x.found = 0;
      __syncthreads();
      return;
    }
    if (best == dsel) {
      s_x.below_c = (uint32_t)bc;
      s_x.below_m = bm;
      s_x.cnt = bn;
    }
    __syncthreads();
    below_c = s_x.below_c;
    below_m = s_x.below_m;
    const uint32_t cnt = s_x.cnt;
    __syncthreads();
    if (cnt <= (uint32_t)XCOL) break;
    // narrow to the chosen digit (every thread computes the same interval)
    XLevel nx;
    nx.mode = 1;
    if (lv.mode == 0) {
      const uint32_t f_m = fkey_desc(u.m), f_end = fkey_desc(-INFINITY);
      const float m = u.m;
      const uint32_t f_lo = x_first_fkey(f_m, f_end, [&](float l) { return x_dbin(l, m) >= dsel; });
      const uint32_t f_hi =
          x_first_fkey(f_m, f_end, [&](float l) { return x_dbin(l, m) >= dsel + 1; }) - 1u;
      nx.klo = (uint64_t)f_lo << 20;
      nx.khi = ((uint64_t)f_hi << 20) | 0xFFFFFull;
    } else {
      nx.klo = lv.klo + ((uint64_t)dsel << lv.shift);
      const uint64_t hi = nx.klo + ((1ull << lv.shift) - 1ull);
      nx.khi = hi < lv.khi ? hi : lv.khi;
    }
    const uint64_t width = nx.khi - nx.klo;
    const int bits = width == 0ull ? 0 : 64 - __clzll((long long)width);
    nx.shift = bits > 12 ? bits - 12 : 0;
    lv = nx;
  }
  // resolve the bucket exactly
  const int n = x_collect<NT, HQ>(a, r, b, j, p, u, lv, dsel, xs.cnt(), xs.key(), s_x);
  x_sort<NT>(xs.key(), n);
  uint64_t w4[XQ], lm = 0ull;
#pragma unroll
  for (int q = 0; q < XQ; ++q) {
    const int pos = XQ * t + q;
    w4[q] = 0ull;
    if (pos < n) {
      const uint64_t key = xs.key()[pos];
      const int id = (int)(uint32_t)key;
      w4[q] = x_wt_q(u, fkey_desc_inv((uint32_t)(key >> 32)),
                     (HQ && u.rS != 0ull) ? xq_prob(a.q, id) : 0.0);
      lm += w4[q];
    }
  }
  uint64_t ex0, exm, tot0, totm;
  block_excl_scan2_u64<NT>(0ull, lm, xs.u2(), ex0, exm, tot0, totm);
  int best = -1;
  uint64_t bm = 0ull, bw = 0ull;
  uint64_t fm = below_m + exm;
#pragma unroll
  for (int q = 0; q < XQ; ++q) {
    const int pos = XQ * t + q;
    if (pos < n) {
      if ((by_mass ? fm : below_c + (uint64_t)pos) <= T) {
        best = pos;
        bm = fm;
        bw = w4[q];
      }
      fm += w4[q];
    }
  }
  const int psel = -block_min<NT>(-best, xs.ired());
  if (t == 0) s_x.found = psel >= 0 ? 1 : 0;
  if (psel >= 0 && best == psel) {
    s_x.key = xs.key()[psel];
    s_x.key_w = bw;
    s_x.below_m = bm;
    s_x.below_c = (uint32_t)(below_c + (uint64_t)psel);
  }
  __syncthreads();
}

struct XOut {
  int status, token, accept;
  double sig;
  uint64_t last_key;
};

// The whole decision chain of one row from streaming passes (see above).
template <int NT, bool HQ>
__device__ __noinline__ XOut exact_row(const XArgs a, int r, int b, int j, const RowParams p, float m, int arg,
                          int draft, bool vdr, float l_draft, const XScratch xs, lds_t<XState>& s_x) {
  const int V = a.V;
  const bool topk = p.top_k > 0 && p.top_k < V;
  const bool topp = p.top_p < 1.0f;
  const bool keep_ties = (p.flags & STRIM_FLAG_TOPK_KEEP_TIES) != 0;
  const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
  const bool by_rank = (p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp;
  const bool cand_sorted = no_lse ? topp : (topk || topp);
  XUni u{m, p.min_p > 0.0f ? p.lmp : -INFINITY, 0ull, ~0ull, -1, 0ull};
  // general-q verify rows draw from the residual (p - q)^+ over the whole kept set
  const bool resid = HQ && vdr && a.has_q;
  uint64_t S = 0ull;
  bool haveS = false;
  uint32_t nkeep = 0u;
  if (topk) {
    const uint64_t K1 = (uint64_t)(p.top_k - 1);
    x_select<NT, HQ>(a, r, b, j, p, u, false, -1.0, K1, xs, s_x);
    if (!s_x.found) return XOut{STRIM_EEMPTY, -1, 0, 0.0, 0ull};
    if (keep_ties) {
      u.bound = (s_x.key & 0xFFFFFFFF00000000ull) | 0xFFFFFFFFull;
    } else {
      u.bound = s_x.key;
      S = s_x.below_m + s_x.key_w;
      haveS = true;
      nkeep = s_x.below_c + 1u;
    }
  }
  if (topp) {
    const double P = (double)p.top_p;
    x_select<NT, HQ>(a, r, b, j, p, u, true, P, 0ull, xs, s_x);
    if (!s_x.found) return XOut{STRIM_EEMPTY, -1, 0, 0.0, 0ull};
    u.bound = s_x.key;
    S = s_x.below_m + s_x.key_w;
    haveS = true;
    nkeep = s_x.below_c + 1u;
  }
  double w_d = 0.0;
  uint64_t W_d = 0ull;
  if (vdr && l_draft > -INFINITY && x_in(u, l_draft, draft)) {
    w_d = exp((double)l_draft - (double)m);
    W_d = x_weight(l_draft, m);
  }
  XUni ud = u;
  ud.excl = vdr && !resid ? draft : -1;
  if (resid && !haveS) {
    const XLevel all{2, 0, 0ull, 0ull};
    x_hist<NT, HQ>(a, r, b, j, p, u, all, xs.cnt(), xs.hc(), xs.key());
    S = xs.key()[0];
    haveS = true;
    __syncthreads();
  }
  int token = -1;
  if (a.noise_mode == STRIM_NOISE_ICDF) {
    const double uu = (double)row_uniform(a, r, p, 0);
    if (resid) {
      ud.rS = S;
      x_select<NT, HQ>(a, r, b, j, p, ud, true, uu, 0ull, xs, s_x);
      // an all-zero residual draws the first kept token
      token = (s_x.found && s_x.tot_m > 0ull) ? (int)(uint32_t)s_x.key : arg;
    } else {
      x_select<NT, HQ>(a, r, b, j, p, ud, true, uu, 0ull, xs, s_x);
      S = s_x.tot_m + W_d;
      // an empty residual (only the draft kept) draws the first kept token
      token = s_x.found ? (int)(uint32_t)s_x.key : arg;
    }
  } else {
    if (!haveS) {
      const XLevel all{2, 0, 0ull, 0ull};
      x_hist<NT, HQ>(a, r, b, j, p, u, all, xs.cnt(), xs.hc(), xs.key());
      S = xs.key()[0];
      __syncthreads();
    }
    const double lse = log((double)S / XFIX);
    const uint64_t pkey = mix64(p.seed, p.position);
    double bsc = -INFINITY;
    uint64_t btk = ~0ull;
    int bid = -1;
    auto take = [&](float l, int id, int64_t nidx, uint64_t tk, double q) {
      const float uq = a.noise ? a.noise[(int64_t)r * a.noise_stride + nidx]
                               : philox_uniform(pkey, (uint64_t)nidx);
      double base = no_lse ? (double)l : ((double)l - (double)m) - lse;
      if (resid) {
        // residual score: log(p - q) where q > 0, excluded where p <= q
        if (q != 0.0) {
          const double rr = exp(base) - q;
          if (!(rr > 0.0)) return;
          base = log(rr);
        }
      }
      const double sc = base + gumbel64(uq);
      if (bid < 0 || sc > bsc || (sc == bsc && tk < btk)) {
        bsc = sc;
        btk = tk;
        bid = id;
      }
    };
    if (by_rank) {
      // noise indexed by the rank in the order: the kept set is walked in rank order,
      // XCOL keys at a time (a count select finds each bucket's last key, a gather pass
      // collects and sorts the bucket)
      const XLevel all{2, 0, 0ull, 0ull};
      XUni ub = ud;
      uint32_t below = 0u;
      while (below < nkeep) {
        x_select<NT, HQ>(a, r, b, j, p, ub, false, -1.0, (uint64_t)(XCOL - 1), xs, s_x);
        if (!s_x.found) break;
        XUni uc = ub;
        uc.bound = s_x.key;
        const int n = x_collect<NT, HQ>(a, r, b, j, p, uc, all, 0, xs.cnt(), xs.key(), s_x);
        x_sort<NT>(xs.key(), n);
        for (int pos = threadIdx.x; pos < n; pos += NT) {
          const uint64_t key = xs.key()[pos];
          take(fkey_desc_inv((uint32_t)(key >> 32)), (int)(uint32_t)key,
               (int64_t)below + pos, key, resid ? xq_prob(a.q, (int)(uint32_t)key) : 0.0);
        }
        __syncthreads();
        if (n <= 0) break;
        below += (uint32_t)n;
        ub.lo = uc.bound + 1ull;
      }
    } else {
      x_pass<NT, HQ>(a, r, b, j, p, xs.cnt(), [&](int i0, const float (&l)[EPT], const float (&qv)[EPT]) {
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if (x_in(ud, l[e], i0 + e))
            take(l[e], i0 + e, i0 + e, cand_sorted ? ckey(l[e], i0 + e) : (uint64_t)(i0 + e),
                 resid ? xq_of(a.q, qv[e]) : 0.0);
      });
    }
    block_argmax_score<NT>(bsc, btk, bid, xs.dred(), xs.ured(), xs.ired(), (int*)&s_x.token);
    token = s_x.token >= 0 ? s_x.token : arg;
  }
  int acc = 0;
  const double sig = (double)S / XFIX;
  if (vdr) {
    const float ua = row_uniform(a, r, p, a.noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V : 1);
    double ratio = w_d / sig;
    if (resid) {
      // accept iff u < p(d) / q(d)
      const double qd = xq_prob(a.q, draft);
      ratio = qd > 0.0 ? ratio / qd : (ratio > 0.0 ? INFINITY : 0.0);
    }
    acc = ((double)ua < ratio) ? 1 : 0;
  }
  uint64_t last = u.bound;
  if (last == ~0ull && p.min_p > 0.0f) {
    const double lmp = u.lmp;
    const uint32_t f_thr = x_first_fkey(fkey_desc(m), fkey_desc(-INFINITY), [&](float l) {
                             return !((double)l - (double)m >= lmp);
                           }) - 1u;
    last = ((uint64_t)f_thr << 32) | 0xFFFFFFFFull;
  }
  return XOut{STRIM_OK, token, acc, sig, last};
}


}  // namespace strim
