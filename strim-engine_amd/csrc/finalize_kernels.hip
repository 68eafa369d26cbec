// finalize_kernels.hip — k_finalize: the per-row decision from k_stream's results.
//
// One workgroup per row:
//   greedy rows      argmax of the merged chunk maxima;
//   fast rows        (0 < top-k <= 256, or min-p >= e^-8) from the chunks' candidates:
//                    min-p on the row maximum, a radix select of the k-th key, a sort of
//                    the survivors, the top-p cut and the draw, all in LDS;
//   unfiltered Gumbel rows  from the chunks' two best scores;
//   general-q draft rows    checked and handed to the residual draw (qres_kernels.hip)
//                    or k_final's exact resolution.
// The other general rows are k_gfinal's (gfinal_kernels.hip), which runs beside it.
// A row whose candidates do not fit the LDS finalize is decided here by the exact
// streaming resolution (exact.hpp).
#include "exact.hpp"

namespace strim {

// ---------------------------------------------------------------------------------
// finalize of one row (k_finalize)
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void finish_row(const Args& a, int r, int status, int token,
                                           int accept, double sig, float m, uint64_t last_key,
                                           int phase) {
  if (threadIdx.x != 0) return;
  RowState* rs = &a.s.rs[r];
  rs->status = status;
  rs->token = token;
  rs->accept = accept;
  rs->sum_kept = sig;
  rs->m = m;
  rs->last_key = last_key;
  rs->phase = phase;
  if (!a.verify && phase == PH_DONE) {
    a.out_ids[r] = status == STRIM_OK ? token : -1;
    if (a.out_status) a.out_status[r] = status;
  }
}

// LDS of one k_finalize workgroup.
constexpr int FSEG = FCAP_FAST / (FTPB / WAVE);  // survivors per wave segment in phase 2
struct FinalShared {
  uint64_t key[FCAP_FAST];  // the row's surviving candidate keys (32 KB)
  uint32_t rpre[256];       // per chunk: first position of its candidates past the
                            // speculative depth, within its 64-chunk block (add the block
                            // offsets in off[])
  uint16_t rcnt[256];       // per chunk: candidates written by k_stream
  uint32_t hist[256];       // d-histogram / radix digits
  float v[FTPB / WAVE], g[FTPB / WAVE];
  int i[FTPB / WAVE], f[FTPB / WAVE];
  uint32_t off[FTPB / WAVE], cnt[FTPB / WAVE], seg[FTPB / WAVE];
  double d[FTPB / WAVE];
  uint64_t u[FTPB / WAVE];
  int misc[8];
  // the exact streaming resolution (rows whose candidates overflow): its histogram
  // masses and gathered buckets use key[] (XB entries)
  uint32_t xhc[XB];
  uint32_t xcnt[FTPB * EPT];
  uint64_t xu2[2 * FTPB / WAVE];
  XState x;
};
static_assert(FCAP_FAST >= XB && FCAP_FAST >= XCOL, "the exact path reuses the candidate keys");

// Histogram bin of d = m - l at `scale` bins per nat (last bin open) for the top-k cut;
// monotone in l.
__device__ __forceinline__ int dbin(float m, float l, float scale) {
  return (int)fminf((m - l) * scale, 255.0f);
}

// Decides a row whose candidates overflow the finalize by the exact streaming
// resolution (all threads of the workgroup call it). Inlined: only exact_row is an
// out-of-line call, taking the few launch fields it needs by value, so the 3 KB launch
// block is never copied to private memory.
__device__ __forceinline__ void finalize_exact(const Args& a, int r, int b, int j,
                                            const RowParams& p, float m, int arg, int draft,
                                            bool vdr, float l_draft, FinalShared& S) {
  const XScratch xs = xscratch(S.key, S.xhc, S.xcnt, S.xu2, S.d, S.u, S.i);
  XArgs xa;
  xa.logits = a.logits;
  xa.row_stride = a.row_stride;
  xa.dtype = a.dtype;
  xa.vec_ok = a.vec_ok;
  xa.V = a.V;
  xa.H = a.H;
  xa.verify = a.verify;
  xa.k = a.k;
  xa.noise_mode = a.noise_mode;
  xa.mask = a.mask;
  xa.mask_stride = a.mask_stride;
  xa.hist = a.hist;
  xa.hist_len = a.hist_len;
  xa.drafts = a.drafts;
  xa.noise = a.noise;
  xa.noise_stride = a.noise_stride;
  xa.has_q = 0;  // general-q rows are decided by k_final
  __syncthreads();
  const XOut xo = exact_row<FTPB, false>(xa, r, b, j, p, m, arg, draft, vdr, l_draft, xs,
                                  *(lds_t<XState>*)&S.x);
  finish_row(a, r, xo.status, xo.token, xo.accept, xo.sig, m, xo.last_key, PH_DONE);
}

// One row per 256-thread workgroup, in three phases with two barriers:
//   1. merge the chunk statistics (max, argmax, flags, k-th value bound G, candidate
//      counts);
//   2. every thread gathers candidate positions t, t + 256, ... (eight loads in flight;
//      a binary search over the wave-region prefixes finds each slot), divides by T,
//      prunes with min-p on the row maximum and with G, compacts the survivors into its
//      wave's LDS segment and, for top-k rows, counts them in a histogram of m - l over
//      the survivors' span;
//   3. wave 0 alone: top-k (from the histogram), sort, top-p, draw, with wave-wide
//      operations only.
// The row's global inputs that do not depend on its parameters, requested before the
// parameters are waited for: the chunk statistics (one chunk per thread), the first
// entries of every candidate region (a speculative gather; the region counts arrive with
// the statistics, so the common row needs one memory round trip, not two), the noise
// and the draft. There is no branch between the loads (see load_chunk); a missing
// optional input reads the row's own state instead and is ignored.
constexpr int PRE_E = 8;  // speculative candidate entries per thread
struct RowPre {
  ChunkStat cs;
  Cand c[PRE_E];
  float n0, n1, l_draft;
  int draft;
  int kd;          // speculative depth K per chunk region (even)
  uint32_t kmag;   // entry e lies in region umulhi(e, kmag) = e / K
};
__device__ __forceinline__ RowPre prefetch_row(const Args& a, int r, int b, int j) {
  RowPre f;
  const int t = threadIdx.x;
  f.cs = a.s.cstat[(int64_t)r * a.s.wmax + (t < a.W ? t : 0)];
  // depth K: the largest even number with K * chunks <= the entries of the workgroup, at
  // least 2 (one 16-byte load), at most a region. e / K = umulhi(e, ceil(2^32 / K)) is
  // exact while e * K < 2^32.
  const int kd = min(SLOT, max(2, ((FTPB * PRE_E) / a.W) & ~1));
  const uint32_t kmag = 0xFFFFFFFFu / (uint32_t)kd + 1u;
  f.kd = kd;
  f.kmag = kmag;
  const Cand* slots = a.s.slot + (int64_t)r * a.s.wmax * SLOT;
#pragma unroll
  for (int q = 0; q < PRE_E / 2; ++q) {
    const int e = t * PRE_E + 2 * q;
    const int g = (int)__umulhi((uint32_t)e, kmag), o = e - g * kd;
    const uint4 v = *(const uint4*)(slots + (g < a.W ? (int64_t)g * SLOT + o : 0));
    f.c[2 * q] = Cand{__uint_as_float(v.x), (int32_t)v.y};
    f.c[2 * q + 1] = Cand{__uint_as_float(v.z), (int32_t)v.w};
  }
  RowState* rsp = &a.s.rs[r];
  const bool gum = a.noise && a.noise_mode != STRIM_NOISE_ICDF;
  const float* nz = a.noise ? a.noise + (int64_t)r * a.noise_stride : (const float*)rsp;
  f.n0 = nz[gum ? a.V : 0];
  f.n1 = nz[gum ? a.V : 1];
  const bool vdr = a.verify && j < a.k;
  const int32_t* dp = vdr ? a.drafts + (int64_t)b * a.k + j : (const int32_t*)rsp;
  const int d = *dp;
  f.draft = vdr ? d : -1;
  const float ld = rsp->l_draft;
  f.l_draft = vdr ? ld : -INFINITY;
  return f;
}

// What the exact streaming resolution needs when a row cannot be finished in LDS.
struct ExactReq {
  int need;
  float m;
  int arg, draft;
  float l_draft;
};

__device__ __forceinline__ ExactReq finalize_row(const Args& a, int r, int b, int j,
                                                 const RowParams& p, const RowPre& pf,
                                                 FinalShared& S) {
  const ExactReq done{0, 0.0f, -1, -1, 0.0f};
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  const int V = a.V, W = a.W;
  const bool vdr = a.verify && j < a.k;  // a verify row with a draft
  const int draft = pf.draft;
  const float l_draft = pf.l_draft;
  float u_draw = 0.0f, u_acc = 0.0f;
  if (a.noise && !p.greedy) {
    if (a.noise_mode == STRIM_NOISE_ICDF) u_draw = pf.n0;
    u_acc = pf.n1;
  } else if (!a.noise) {
    // the row's own uniforms, computed while the prefetched loads are in flight (they
    // depend on the parameters alone)
    const uint64_t pk = mix64(p.seed, p.position);
    u_draw = philox_uniform(pk, 0);
    u_acc = philox_uniform(pk, a.noise_mode == STRIM_NOISE_GUMBEL ? (uint64_t)V : 1u);
  }

  // ---- phase 1: chunk statistics (W <= 256: one chunk per thread) -----------------
  // (threads past the row's chunks select neutral values; no branch around the loads)
  const ChunkStat& cs = pf.cs;
  const bool own = t < W;
  int ff = own ? (cs.flags | (cs.n > 0 ? 4 : 0)) : 0;
  // one candidate region per chunk, SLOT entries: the first K entries of the regions
  // below npre were gathered speculatively, the rest ("residual" entries) are gathered by
  // position in phase 2
  const int kd = pf.kd, npre = (FTPB * PRE_E) / kd;
  auto depth = [&](int g) { return g < npre ? (uint32_t)kd : 0u; };
  const uint32_t ce = own ? cs.ncand : 0u;
  if (ce > (uint32_t)SLOT) ff |= 2;  // the region overflowed
  const uint32_t ctot = ce <= (uint32_t)SLOT ? ce : 0u;
  const uint32_t rtot = ctot > depth(t) ? ctot - depth(t) : 0u;
  float mv = own ? cs.m : -INFINITY, gv = own ? cs.g : -INFINITY;
  int mi = own ? cs.arg : -1;
  wave_argmax(mv, mi);
  ff = wave_or_i(ff);
  gv = wave_max_f(gv);
  const uint32_t wall = (uint32_t)wave_sum((int)ctot);
  uint32_t wtot;
  const uint32_t wex = wave_excl_scan_u32(rtot, &wtot);
  if (own) {
    S.rpre[t] = wex;
    S.rcnt[t] = (uint16_t)ctot;
  }
  if (t < 256) S.hist[t] = 0u;
  if (lane == 0) {
    S.v[w] = mv;
    S.i[w] = mi;
    S.f[w] = ff;
    S.g[w] = gv;
    S.off[w] = wtot;
    S.cnt[w] = wall;
  }
  __syncthreads();
  float m = S.v[0], G = S.g[0];
  int arg = S.i[0], flags = S.f[0];
  uint32_t n_c = 0u, n_r = 0u;  // all candidates; residual entries
#pragma unroll
  for (int q = 0; q < FTPB / WAVE; ++q) {
    if (q > 0) {
      argmax_merge(m, arg, S.v[q], S.i[q]);
      flags |= S.f[q];
      G = fmaxf(G, S.g[q]);
    }
    n_c += S.cnt[q];
    n_r += S.off[q];
  }

  int status = STRIM_OK;
  if (vdr && (draft < 0 || draft >= V)) status = STRIM_EINVAL;
  if (status == STRIM_OK && (flags & 1)) status = STRIM_ENONFINITE;
  if (status == STRIM_OK && !(flags & 4)) status = STRIM_EEMPTY;
  if (status != STRIM_OK) {
    finish_row(a, r, status, -1, 0, 0.0, m, 0ull, PH_DONE);
    return done;
  }
  if (p.greedy) {
    finish_row(a, r, STRIM_OK, arg, vdr && arg == draft, 1.0, m, 0ull, PH_DONE);
    return done;
  }
  if (vdr && a.dlog) {
    // general-q draft row: the draft distribution from k_qprep's slices (its maximum, the
    // draft's table index, fp64 Z = sum exp(v - mq)), published for the residual draw;
    // the draft must be in a valid table (the first draft row's slices checked it)
    const int qr = b * a.k + j;
    const QPart* pp = a.s.qpp + (size_t)qr * QSPLIT;
    float mq = -INFINITY;
    int td = -1, bad = 0;
#pragma unroll
    for (int q = 0; q < QSPLIT; ++q) {
      mq = fmaxf(mq, pp[q].m);
      td = max(td, pp[q].td);
      bad |= a.s.qpp[q].bad;
    }
    // Z = sum over the slices of z exp(m - mq): one slice per lane of wave 0
    double z = 0.0;
    if (w == 0) {
      const QPart& pq = pp[lane < QSPLIT ? lane : 0];
      z = wave_sum(lane < QSPLIT && pq.m > -INFINITY ? pq.z * exp((double)pq.m - (double)mq)
                                                     : 0.0);
      if (t == 0) a.s.qst[qr] = QStat{mq, td, z};
    }
    if (bad || td < 0) {
      finish_row(a, r, STRIM_EINVAL, -1, 0, 0.0, m, 0ull, PH_DONE);
      return done;
    }
    // unfiltered rows: the grid-wide residual draw (qres_kernels.hip); the others: k_final's
    // exact resolution (the row's first maximum is kept as the fallback token)
    const bool unfiltered = !(p.top_k > 0 && p.top_k < V) && !(p.top_p < 1.0f) && !(p.min_p > 0.0f);
    uint64_t wq = 0ull;
    if (unfiltered && own) {
      // the residual draw's plain mass per chunk, round(2^43 sum exp(l - m)), from
      // k_stream's chunk sums (fp64 over float terms: within a few 1e-7 of the sum of
      // the per-token fixed-point weights)
      const double wc = cs.n > 0 ? cs.S * exp((double)cs.m - (double)m) : 0.0;
      wq = (unsigned long long)__double2ull_rn(wc * XFIX);
      a.s.qpart[(size_t)qr * a.s.wmax + t] = wq;
    }
    if (unfiltered && a.qskip) {
      // Only (accepted, token) is asked for: the accept test runs here, on the same
      // numbers as the residual pick's (the row mass is the integer sum of the chunk masses above),
      // so the residual draw runs only for a sequence's first rejected row.
      const uint64_t sw = wave_sum_u64(wq);
      if (lane == 0) S.u[w] = sw;
      __syncthreads();
      if (t == 0) {
        uint64_t Sq = 0ull;
#pragma unroll
        for (int q = 0; q < FTPB / WAVE; ++q) Sq += S.u[q];
        const double sig = (double)Sq / XFIX;
        const double w_d = l_draft > -INFINITY ? exp((double)l_draft - (double)m) : 0.0;
        double ratio = w_d / sig;
        const uint32_t dw = a.s.dbits[draft >> 5];
        const bool in_tab = (dw >> (draft & 31)) & 1u;
        const double qd =
            in_tab ? exp((double)xq_v(q_base(a, qr), draft, dw, a.s.wrank[draft >> 5]) -
                         (double)mq) / z
                   : 0.0;
        ratio = qd > 0.0 ? ratio / qd : (ratio > 0.0 ? INFINITY : 0.0);
        const float ua =
            a.noise ? pf.n1
                    : philox_uniform(mix64(p.seed, p.position),
                                     a.noise_mode == STRIM_NOISE_GUMBEL ? (uint64_t)V : 1u);
        const int acc = ((double)ua < ratio) ? 1 : 0;
        finish_row(a, r, STRIM_OK, acc ? draft : arg, acc, sig, m, 0ull, acc ? PH_DONE : PH_QRES);
      }
      return done;
    }
    finish_row(a, r, STRIM_OK, arg, 0, 0.0, m, 0ull, unfiltered ? PH_QRES : PH_EXACT);
    return done;
  }
  const bool topk = p.top_k > 0 && p.top_k < V;
  const bool topp = p.top_p < 1.0f;
  const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
  const bool by_rank = (p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp;
  const bool cand_sorted = no_lse ? topp : (topk || topp);
  const uint64_t pkey = mix64(p.seed, p.position);
  const int excl_id = vdr ? draft : -1;

  // ---- unfiltered Gumbel rows: the chunks' two best tokens ------------------------
  // (and a chunk's near ties of its second best, as its candidates; flag 8: a chunk had
  // more near ties than its candidate region holds, the exact resolution decides)
  if (p.cls == CLS_GENERAL && a.noise_mode == STRIM_NOISE_GUMBEL && row_nofilter(p, V) &&
      (flags & 8))
    return ExactReq{1, m, arg, draft, l_draft};
  if (p.cls == CLS_GENERAL && a.noise_mode == STRIM_NOISE_GUMBEL && row_nofilter(p, V)) {
    const double wc = (t < W && cs.n > 0) ? cs.S * exp((double)cs.m - (double)m) : 0.0;
    const double sig = block_sum_f64<FTPB>(wc, S.d);
    const double lse = log(sig);
    double bsc = -INFINITY;
    uint64_t btk = ~0ull;
    int bid = -1;
    auto take = [&](int id, float l) {
      if (id < 0 || id == excl_id) return;
      const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + id]
                              : philox_uniform(pkey, (uint64_t)id);
      const double base = no_lse ? (double)l : ((double)l - (double)m) - lse;
      const double sc = base + gumbel64(u);
      if (bid < 0 || sc > bsc || (sc == bsc && (uint64_t)id < btk)) {
        bsc = sc; btk = (uint64_t)id; bid = id;
      }
    };
    if (t < W) {
      const ChunkPart pt = a.s.part[(int64_t)r * a.s.wmax + t];
      take(pt.id0, pt.l0);
      take(pt.id1, pt.l1);
      const Cand* near = a.s.slot + ((int64_t)r * a.s.wmax + t) * SLOT;
      for (uint32_t e = 0; e < cs.ncand; ++e) take(near[e].id, near[e].l);
    }
    block_argmax_score<FTPB>(bsc, btk, bid, S.d, S.u, S.i, &S.misc[3]);
    int token = S.misc[3];
    int acc = 0;
    if (vdr) {
      const double w_d = l_draft > -INFINITY ? exp((double)l_draft - (double)m) : 0.0;
      acc = ((double)u_acc < w_d / sig) ? 1 : 0;
      if (token < 0) token = arg;  // the draft is the only allowed token
    }
    finish_row(a, r, STRIM_OK, token, acc, sig, m, ~0ull, PH_DONE);
    return done;
  }
  // General rows are k_gfinal's (this kernel returns before the row for them); should one
  // arrive here, the exact resolution decides it.
  if (p.cls != CLS_FAST) return ExactReq{1, m, arg, draft, l_draft};
  if ((flags & 2) || n_c > (uint32_t)FCAND) {
    return ExactReq{1, m, arg, draft, l_draft};
  }

  // ---- phase 2: gather, divide, prune, compact --------------------------------------
  // every kept token has v >= G (the k-th value bound), minus the l-tie margin
  const float Gm = topk && G > -INFINITY ? G - (fabsf(G) * 1e-6f + 1e-30f) : -INFINITY;
  const bool minp = p.min_p > 0.0f;
  const double lmp = p.lmp;
  // top-k histogram of d = m - l over the survivors' span (bounded by G or min-p)
  float dspan = 16.0f;
  if (Gm > -INFINITY) dspan = fminf(dspan, m - Gm / p.T);
  if (minp) dspan = fminf(dspan, (float)-lmp);
  const float scale = 255.0f / fmaxf(dspan * 1.0001f, 1e-6f);
  const Cand* slots = a.s.slot + (int64_t)r * a.s.wmax * SLOT;
  // global position of region rg's first residual entry
  auto gpre = [&](int rg) {
    uint32_t o = S.rpre[rg];
    const int blk = rg >> 6;  // 64 chunks per wave of phase 1
#pragma unroll
    for (int q = 0; q < FTPB / WAVE; ++q)
      if (q < blk) o += S.off[q];
    return o;
  };
  constexpr int GB = 8;  // loads in flight per thread per batch
  uint32_t n_w = 0u;     // survivors in this wave's segment
  // Candidates below the v-space bound of G and min-p (most of them: the chunks bound
  // min-p on their own maximum) leave after one compare, without the division.
  const float vthr = fmaxf(Gm, minp ? minp_vlo(m, p) : -INFINITY);
  // One candidate of this lane (id < 0: none), called by the whole wave: the v-space
  // pretest only; (v, id) pairs that pass are compacted into the wave's LDS segment.
  // The division and the exact tests run once per survivor after the gathers.
  auto take = [&](const Cand cd) {
    const bool k = cd.id >= 0 && cd.l >= vthr;
    const uint64_t msk = __ballot(k);
    if (msk) {
      const uint32_t dst = n_w + (uint32_t)lanes_below(msk);
      if (k && dst < (uint32_t)FSEG)
        S.key[w * FSEG + dst] = ((uint64_t)__float_as_uint(cd.l) << 32) | (uint32_t)cd.id;
      n_w += (uint32_t)__popcll(msk);
    }
  };
  // the speculative entries, valid below their region's count
  {
#pragma unroll
    for (int i = 0; i < PRE_E; ++i) {
      const int e = t * PRE_E + i;
      const int g = (int)__umulhi((uint32_t)e, pf.kmag), o = e - g * kd;
      const bool ok = g < W && o < (int)S.rcnt[g < W ? g : 0];
      take(ok ? pf.c[i] : Cand{-INFINITY, -1});
    }
  }
  // the residual entries, by position
  for (int base = 0; base < (int)n_r; base += GB * FTPB) {
    Cand cd[GB];
#pragma unroll
    for (int q = 0; q < GB; ++q) {
      const int pos = base + q * FTPB + t;
      cd[q] = Cand{-INFINITY, -1};
      if (pos < (int)n_r) {
        int lo = 0, hi = W - 1;  // last region whose first position <= pos
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if ((int)gpre(mid) <= pos) lo = mid;
          else hi = mid - 1;
        }
        cd[q] = slots[(int64_t)lo * SLOT + depth(lo) + (pos - (int)gpre(lo))];
      }
    }
#pragma unroll
    for (int q = 0; q < GB; ++q) take(cd[q]);
  }
  // l = v / T as the oracle rounds it, min-p on the row maximum and the top-k histogram
  // for the wave's pretest survivors, compacted in place into order keys
  if (n_w <= (uint32_t)FSEG) {
    uint64_t* seg = S.key + w * FSEG;
    uint32_t n2 = 0u;
    for (uint32_t base = 0; base < n_w; base += WAVE) {
      const uint32_t i = base + (uint32_t)lane;
      bool k = i < n_w;
      const uint64_t raw = k ? seg[i] : 0ull;
      const int id = (int)(uint32_t)raw;
      const float l = k ? __uint_as_float((uint32_t)(raw >> 32)) / p.T : -INFINITY;
      k = k && l > -INFINITY && (!minp || ((double)l - (double)m) >= lmp);
      const uint64_t msk = __ballot(k);
      wave_sync();  // every read of the block precedes the writes (positions only fall)
      if (k) seg[n2 + (uint32_t)lanes_below(msk)] = ckey(l, id);
      if (k && topk) atomicAdd(&S.hist[dbin(m, l, scale)], 1u);
      n2 += (uint32_t)__popcll(msk);
      wave_sync();
    }
    n_w = n2;
  }
  if (lane == 0) S.seg[w] = n_w;
  __syncthreads();
  uint32_t segn[FTPB / WAVE];
  int over = 0;
  uint32_t n_s = 0u;
#pragma unroll
  for (int q = 0; q < FTPB / WAVE; ++q) {
    segn[q] = S.seg[q];
    over |= segn[q] > (uint32_t)FSEG;
    n_s += segn[q];
  }
  if (over) {
    return ExactReq{1, m, arg, draft, l_draft};
  }
  if (w != 0) return done;  // phase 3 is one wave
  // concatenate the wave segments
  {
    uint32_t o = segn[0];
#pragma unroll
    for (int q = 1; q < FTPB / WAVE; ++q) {
      for (uint32_t i = lane; i < segn[q]; i += WAVE) S.key[o + i] = S.key[q * FSEG + i];
      o += segn[q];
    }
    wave_sync();
  }
  int n = (int)n_s;

  // ---- phase 3a: top-k -- the survivors up to the histogram bin holding the k-th ----
  bool sorted = false;
  if (topk && n > p.top_k) {
    const uint4 h = *(const uint4*)&S.hist[4 * lane];
    const uint32_t own = h.x + h.y + h.z + h.w;
    uint32_t tot;
    uint32_t cum = wave_excl_scan_u32(own, &tot);
    const uint32_t hs[4] = {h.x, h.y, h.z, h.w};
    int bl = 256;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (bl == 256 && cum + hs[e] >= (uint32_t)p.top_k) bl = 4 * lane + e;
      cum += hs[e];
    }
    const int bstar = wave_min_i(bl);
    // keep the keys in bins <= bstar (a superset of the top k)
    uint32_t n2 = 0u;
    for (int base = 0; base < n; base += WAVE) {
      const int pos = base + lane;
      const uint64_t kv = pos < n ? S.key[pos] : ~0ull;
      const bool keep = pos < n && dbin(m, fkey_desc_inv((uint32_t)(kv >> 32)), scale) <= bstar;
      const uint64_t msk = __ballot(keep);
      wave_sync();
      if (keep) S.key[n2 + (uint32_t)lanes_below(msk)] = kv;
      n2 += (uint32_t)__popcll(msk);
      wave_sync();
    }
    n = (int)n2;
    uint64_t kth;
    if (n <= WAVE) {
      wave_rank_sort(S.key, n);
      kth = S.key[p.top_k - 1];
    } else if (n <= 1024) {
      wave_sort_lds(S.key, n);
      kth = S.key[p.top_k - 1];
    } else {
      kth = wave_radix_kth(S.key, n, (uint32_t)p.top_k, S.hist);
      uint32_t n3 = 0u;
      for (int base = 0; base < n; base += WAVE) {
        const int pos = base + lane;
        const uint64_t kv = pos < n ? S.key[pos] : ~0ull;
        const bool keep = pos < n && (uint32_t)(kv >> 32) <= (uint32_t)(kth >> 32);
        const uint64_t msk = __ballot(keep);
        wave_sync();
        if (keep) S.key[n3 + (uint32_t)lanes_below(msk)] = kv;
        n3 += (uint32_t)__popcll(msk);
        wave_sync();
      }
      n = (int)n3;
      wave_sort_lds(S.key, n);
    }
    sorted = true;
    // the kept prefix: k keys, or with ties every key sharing the k-th value
    const bool ties = (p.flags & STRIM_FLAG_TOPK_KEEP_TIES) != 0;
    const uint64_t bound = ties ? (kth | 0xFFFFFFFFull) : kth;
    int c = 0;
    for (int base = 0; base < n; base += WAVE) {
      const int pos = base + lane;
      c += (pos < n && S.key[pos] <= bound) ? 1 : 0;
    }
    n = wave_sum(c);
  }
  // ---- phase 3b: sort the survivors ---------------------------------------------
  if (!sorted) {
    if (n <= WAVE) {
      wave_rank_sort(S.key, n);
    } else {
      wave_sort_lds(S.key, n);
    }
  }

  // ---- phase 3c: top-p over the sorted survivors ----------------------------------
  // lane owns positions [lane*Qn, lane*Qn + Qn); with n <= 64 (Qn = 1) its weight is
  // computed once
  const int Qn = (n + WAVE - 1) / WAVE;
  const int p0 = lane * Qn, p1 = min(n, p0 + Qn);
  const uint64_t* keys = S.key;
  auto weight = [&](int q) {
    return exp((double)fkey_desc_inv((uint32_t)(keys[q] >> 32)) - (double)m);
  };
  const double w0 = p0 < p1 ? weight(p0) : 0.0;
  double loc = w0;
  for (int q = p0 + 1; q < p1; ++q) loc += weight(q);
  double S_pre;
  const double ex = wave_excl_scan_f64(loc, &S_pre);
  int n_keep = n;
  if (topp) {
    const double P = (double)p.top_p;
    int fd = n;
    double run = ex;
    for (int q = p0; q < p1; ++q) {
      if (run / S_pre - P > 0.0) {
        fd = q;
        break;
      }
      run += q == p0 ? w0 : weight(q);
    }
    n_keep = wave_min_i(fd);
  }
  const int k1 = min(p1, n_keep);
  loc = 0.0;
  for (int q = p0; q < k1; ++q) loc += q == p0 ? w0 : weight(q);
  double S_kept;
  const double exk = wave_excl_scan_f64(loc, &S_kept);
  const uint64_t last_key = keys[n_keep - 1];

  // the draft of a verify row: kept iff its key is inside the kept prefix
  double w_d = 0.0;
  uint64_t key_d = ~0ull;
  if (vdr && l_draft > -INFINITY) {
    key_d = ckey(l_draft, draft);
    if (key_d <= last_key) w_d = exp((double)l_draft - (double)m);
  }

  // ---- phase 3d: draw -----------------------------------------------------------
  int token;
  if (a.noise_mode == STRIM_NOISE_ICDF) {
    const double tgt = (double)u_draw * (S_kept - w_d);
    int best = n_keep;
    double run = exk;
    for (int q = p0; q < k1; ++q) {
      const uint64_t key = keys[q];
      const double wq = q == p0 ? w0 : weight(q);
      double before = run;
      if (key_d < key) before -= w_d;
      if ((int)(uint32_t)key != excl_id && wq > 0.0 && before + wq > tgt) {
        best = q;
        break;
      }
      run += wq;
    }
    int bp = wave_min_i(best);
    if (bp >= n_keep) {
      // rounding pushed the target past the end, or the residual is empty (only the
      // draft kept): the last kept token other than the draft, else the first kept
      bp = n_keep - 1;
      if ((int)(uint32_t)keys[bp] == excl_id) bp = bp > 0 ? bp - 1 : 0;
      if (S_kept - w_d <= 0.0) bp = 0;
    }
    token = (int)(uint32_t)keys[bp];
  } else {
    const double lse = log(S_kept);
    double bsc = -INFINITY;
    uint64_t btk = ~0ull;
    int bid = -1;
    for (int q = p0; q < k1; ++q) {
      const uint64_t key = keys[q];
      const int id = (int)(uint32_t)key;
      if (id == excl_id) continue;
      const float l = fkey_desc_inv((uint32_t)(key >> 32));
      const int64_t nidx = by_rank ? (int64_t)q : (int64_t)id;
      const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + nidx]
                              : philox_uniform(pkey, (uint64_t)nidx);
      const double base = no_lse ? (double)l : ((double)l - (double)m) - lse;
      const double sc = base + gumbel64(u);
      const uint64_t tk = cand_sorted ? key : (uint64_t)id;
      if (bid < 0 || sc > bsc || (sc == bsc && tk < btk)) { bsc = sc; btk = tk; bid = id; }
    }
    token = wave_argmax_score(bsc, btk, bid);
    if (token < 0) token = (int)(uint32_t)keys[0];  // every score -inf / only the draft kept
  }
  const int acc = vdr && ((double)u_acc < w_d / S_kept) ? 1 : 0;
  finish_row(a, r, STRIM_OK, token, acc, S_kept, m, last_key, PH_DONE);
  return done;
}

// ---------------------------------------------------------------------------------
// k_finalize: one workgroup per row, after k_stream (the kernel boundary makes every
// chunk's results visible; an in-kernel device-scope release per workgroup costs far
// more on gfx950 than the second launch)
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(FTPB) void k_finalize(Args a) {
  __shared__ FinalShared S;
  // the launch fields of the prefetch, read together (see k_stream)
  asm volatile("" ::"s"(a.s.cstat), "s"(a.s.wmax), "s"(a.s.slot), "s"(a.s.rs), "s"(a.W),
               "s"(a.V), "s"(a.noise), "s"(a.noise_stride), "s"(a.noise_mode), "s"(a.verify),
               "s"(a.k), "s"(a.drafts));
  const int r = blockIdx.x;
  int b, j;
  row_bj(a, r, b, j);
  const RowPre pf = prefetch_row(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  // the general rows are k_gfinal's
  if (gfinal_row(a.p[b], a.V, a.noise_mode, a.dlog != nullptr && a.verify && j < a.k)) return;
  const ExactReq q = finalize_row(a, r, b, j, p, pf, S);
  // one call site for the exact resolution (an out-of-line call), reached by every
  // thread of a row that needs it
  if (q.need) finalize_exact(a, r, b, j, p, q.m, q.arg, q.draft, a.verify && j < a.k, q.l_draft, S);
}

hipError_t launch_finalize(const Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  return launch_args((const void*)k_finalize, dim3((unsigned)a.R), dim3(FTPB), a, st, e0, e1);
}

}  // namespace strim
