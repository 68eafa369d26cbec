// stream_kernels.hip — k_stream: the single streaming pass over the logits, and
// k_finalize: the per-row decision from the chunks' results.
//
// A 256-thread workgroup owns one (row, chunk of 4096 tokens); thread t owns the two
// 8-token segments t and t + 256, so every wave-wide load is 1 KB (bf16) of contiguous
// logits. All global loads of a workgroup (logits, allow-bits, history ids) are issued
// before its first barrier. The workgroup writes its chunk statistics and candidates;
// k_finalize (one workgroup per row) then decides the row:
//   greedy rows      argmax of the merged chunk maxima;
//   fast rows        (0 < top-k <= 256, or min-p >= e^-8) from the chunks' candidates:
//                    min-p on the row maximum, a radix select of the k-th key, a sort of
//                    the survivors, the top-p cut and the draw, all in LDS;
//   unfiltered Gumbel rows  from the chunks' two best scores;
//   general rows     left to k_collect / k_final (pass-1 histograms are written here).
// A row whose candidates do not fit the LDS finalize is decided there by the exact
// streaming resolution (exact.hpp).
#include "exact.hpp"

namespace strim {

constexpr int SSEG = CHUNK / (STPB * EPT);  // 8-token segments per thread
static_assert(SSEG == 2, "k_stream geometry");

// LDS of one k_stream workgroup.
struct StreamShared {
  uint32_t cnt[CHUNK];          // history counts of the chunk's tokens (16 KB)
  uint32_t hc[NCB];
  unsigned long long hm[NCB];
  uint32_t lad[2 * WAVE];
  float v[STPB / WAVE];
  int i[STPB / WAVE], n[STPB / WAVE], f[STPB / WAVE];
  uint32_t off[STPB / WAVE];
  double d[STPB / WAVE];
  float tf[4 * STPB / WAVE];
  int ti[2 * STPB / WAVE];
};

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
constexpr int FSEG = FCAP / (STPB / WAVE);  // survivors per wave segment in phase 2
struct FinalShared {
  uint64_t key[FCAP];       // the row's surviving candidate keys (32 KB)
  uint32_t rpre[4 * 256];   // per wave region: first candidate position within its
                            // 64-chunk block (add the block offsets in off[])
  uint32_t hist[256];       // d-histogram / radix digits
  float v[STPB / WAVE], g[STPB / WAVE];
  int i[STPB / WAVE], f[STPB / WAVE];
  uint32_t off[STPB / WAVE], cnt[STPB / WAVE];
  double d[STPB / WAVE];
  uint64_t u[STPB / WAVE];
  int misc[8];
  // the exact streaming resolution (rows whose candidates overflow): its histogram
  // masses and gathered buckets use key[] (XB entries)
  uint32_t xhc[XB];
  uint32_t xcnt[STPB * EPT];
  uint64_t xu2[2 * STPB / WAVE];
  XState x;
};
static_assert(FCAP >= XB && FCAP >= XCOL, "the exact path reuses the candidate keys");

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
  XScratch xs;
  xs.key = S.key;
  xs.hc = S.xhc;
  xs.cnt = S.xcnt;
  xs.u2 = S.xu2;
  xs.dred = S.d;
  xs.ured = S.u;
  xs.ired = S.i;
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
  __syncthreads();
  const XOut xo = exact_row<STPB>(xa, r, b, j, p, m, arg, draft, vdr, l_draft, xs, S.x);
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
__device__ void finalize_row(const Args& a, int r, int b, int j, const RowParams& p,
                             FinalShared& S) {
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
  const int V = a.V, W = a.W;
  const bool vdr = a.verify && j < a.k;  // a verify row with a draft
  RowState* rsp = &a.s.rs[r];
  // the row's remaining global inputs, requested before anything waits
  const int draft = vdr ? a.drafts[(int64_t)b * a.k + j] : -1;
  const float l_draft = vdr ? rsp->l_draft : -INFINITY;
  float u_draw = 0.0f, u_acc = 0.0f;
  if (a.noise && !p.greedy) {
    const float* nz = a.noise + (int64_t)r * a.noise_stride;
    if (a.noise_mode == STRIM_NOISE_ICDF) {
      u_draw = nz[0];
      u_acc = nz[1];
    } else {
      u_acc = nz[V];
    }
  }

  // ---- phase 1: chunk statistics (W <= 256: one chunk per thread) -----------------
  ChunkStat cs{-INFINITY, -1, 0, 0, 0.0, 0u, -INFINITY};
  if (t < W) cs = a.s.cstat[(int64_t)r * a.s.wmax + t];
  uint32_t ctot = 0u;
  int ff = cs.flags | (cs.n > 0 ? 4 : 0);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t ce = (cs.nslot >> (8 * e)) & 255u;
    if (ce > (uint32_t)SLOTW) ff |= 2;  // a wave region overflowed
    ctot += ce;
  }
  float mv = cs.m, gv = cs.g;
  int mi = cs.arg;
  wave_argmax(mv, mi);
  ff = wave_or_i(ff);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) gv = fmaxf(gv, __shfl_xor(gv, o, WAVE));
  uint32_t wtot;
  const uint32_t wex = wave_excl_scan_u32(ctot, &wtot);
  if (t < W) {
    uint32_t o = wex;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      S.rpre[4 * t + e] = o;
      o += (cs.nslot >> (8 * e)) & 255u;
    }
  }
  if (t < 256) S.hist[t] = 0u;
  if (lane == 0) {
    S.v[w] = mv;
    S.i[w] = mi;
    S.f[w] = ff;
    S.g[w] = gv;
    S.off[w] = wtot;
  }
  __syncthreads();
  float m = S.v[0], G = S.g[0];
  int arg = S.i[0], flags = S.f[0];
  uint32_t n_c = 0u;
#pragma unroll
  for (int q = 0; q < STPB / WAVE; ++q) {
    if (q > 0) {
      argmax_merge(m, arg, S.v[q], S.i[q]);
      flags |= S.f[q];
      G = fmaxf(G, S.g[q]);
    }
    n_c += S.off[q];
  }

  int status = STRIM_OK;
  if (vdr && (draft < 0 || draft >= V)) status = STRIM_EINVAL;
  if (status == STRIM_OK && (flags & 1)) status = STRIM_ENONFINITE;
  if (status == STRIM_OK && !(flags & 4)) status = STRIM_EEMPTY;
  if (status != STRIM_OK) {
    finish_row(a, r, status, -1, 0, 0.0, m, 0ull, PH_DONE);
    return;
  }
  if (p.greedy) {
    finish_row(a, r, STRIM_OK, arg, vdr && arg == draft, 1.0, m, 0ull, PH_DONE);
    return;
  }
  const bool topk = p.top_k > 0 && p.top_k < V;
  const bool topp = p.top_p < 1.0f;
  const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
  const bool by_rank = (p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp;
  const bool cand_sorted = no_lse ? topp : (topk || topp);
  const uint64_t pkey = mix64(p.seed, p.position);
  const int excl_id = vdr ? draft : -1;
  if (!a.noise) {
    u_draw = philox_uniform(pkey, 0);
    u_acc = philox_uniform(pkey, a.noise_mode == STRIM_NOISE_GUMBEL ? (uint64_t)V : 1u);
  }

  // ---- unfiltered Gumbel rows: the chunks' two best tokens ------------------------
  if (p.cls == CLS_GENERAL && a.noise_mode == STRIM_NOISE_GUMBEL && row_nofilter(p, V)) {
    const double wc = (t < W && cs.n > 0) ? cs.S * exp((double)cs.m - (double)m) : 0.0;
    const double sig = block_sum_f64<STPB>(wc, S.d);
    const double lse = log(sig);
    double bsc = -INFINITY;
    uint64_t btk = ~0ull;
    int bid = -1;
    if (t < W) {
      const ChunkPart pt = a.s.part[(int64_t)r * a.s.wmax + t];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int id = h == 0 ? pt.id0 : pt.id1;
        const float l = h == 0 ? pt.l0 : pt.l1;
        if (id < 0 || id == excl_id) continue;
        const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + id]
                                : philox_uniform(pkey, (uint64_t)id);
        const double base = no_lse ? (double)l : ((double)l - (double)m) - lse;
        const double sc = base + gumbel64(u);
        if (bid < 0 || sc > bsc || (sc == bsc && (uint64_t)id < btk)) {
          bsc = sc; btk = (uint64_t)id; bid = id;
        }
      }
    }
    block_argmax_score<STPB>(bsc, btk, bid, S.d, S.u, S.i, &S.misc[3]);
    int token = S.misc[3];
    int acc = 0;
    if (vdr) {
      const double w_d = l_draft > -INFINITY ? exp((double)l_draft - (double)m) : 0.0;
      acc = ((double)u_acc < w_d / sig) ? 1 : 0;
      if (token < 0) token = arg;  // the draft is the only allowed token
    }
    finish_row(a, r, STRIM_OK, token, acc, sig, m, ~0ull, PH_DONE);
    return;
  }
  if (p.cls != CLS_FAST) {
    finish_row(a, r, STRIM_OK, -1, 0, 0.0, m, 0ull, PH_PENDING);
    return;
  }
  if ((flags & 2) || n_c > (uint32_t)FCAND) {
    finalize_exact(a, r, b, j, p, m, arg, draft, vdr, l_draft, S);
    return;
  }

  // ---- phase 2: gather, divide, prune, compact --------------------------------------
  // every kept token has v >= G (the k-th value bound), minus the l-tie margin
  const float Gm = topk && G > -INFINITY ? G - (fabsf(G) * 1e-6f + 1e-30f) : -INFINITY;
  const bool minp = p.min_p > 0.0f;
  const double lmp = minp ? log((double)p.min_p) : 0.0;
  // top-k histogram of d = m - l over the survivors' span (bounded by G or min-p)
  float dspan = 16.0f;
  if (Gm > -INFINITY) dspan = fminf(dspan, m - Gm / p.T);
  if (minp) dspan = fminf(dspan, (float)-lmp);
  const float scale = 255.0f / fmaxf(dspan * 1.0001f, 1e-6f);
  const Cand* slots = a.s.slot + (int64_t)r * a.s.wmax * SLOT;
  const int nreg = 4 * W;
  // global position of region rg's first candidate
  auto gpre = [&](int rg) {
    uint32_t o = S.rpre[rg];
    const int blk = rg >> 8;  // 64 chunks (256 regions) per wave of phase 1
#pragma unroll
    for (int q = 0; q < STPB / WAVE; ++q)
      if (q < blk) o += S.off[q];
    return o;
  };
  constexpr int GB = 8;  // loads in flight per thread per batch
  uint32_t n_w = 0u;     // survivors in this wave's segment
  for (int base = 0; base < (int)n_c; base += GB * STPB) {
    Cand cd[GB];
#pragma unroll
    for (int q = 0; q < GB; ++q) {
      const int pos = base + q * STPB + t;
      cd[q] = Cand{-INFINITY, -1};
      if (pos < (int)n_c) {
        int lo = 0, hi = nreg - 1;  // last region whose first position <= pos
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if ((int)gpre(mid) <= pos) lo = mid;
          else hi = mid - 1;
        }
        cd[q] = slots[(int64_t)lo * SLOTW + (pos - (int)gpre(lo))];
      }
    }
#pragma unroll
    for (int q = 0; q < GB; ++q) {
      // l = v / T as the oracle rounds it
      bool k = cd[q].id >= 0 && cd[q].l >= Gm;
      const float l = k ? cd[q].l / p.T : -INFINITY;
      k = k && l > -INFINITY && (!minp || ((double)l - (double)m) >= lmp);
      const uint64_t msk = __ballot(k);
      if (msk) {
        const uint32_t dst = n_w + (uint32_t)lanes_below(msk);
        if (k && dst < (uint32_t)FSEG) S.key[w * FSEG + dst] = ckey(l, cd[q].id);
        if (k && topk) atomicAdd(&S.hist[dbin(m, l, scale)], 1u);
        n_w += (uint32_t)__popcll(msk);
      }
    }
  }
  if (lane == 0) S.off[w] = n_w;
  __syncthreads();
  uint32_t segn[STPB / WAVE];
  int over = 0;
  uint32_t n_s = 0u;
#pragma unroll
  for (int q = 0; q < STPB / WAVE; ++q) {
    segn[q] = S.off[q];
    over |= segn[q] > (uint32_t)FSEG;
    n_s += segn[q];
  }
  if (over) {
    finalize_exact(a, r, b, j, p, m, arg, draft, vdr, l_draft, S);
    return;
  }
  if (w != 0) return;  // phase 3 is one wave
  // concatenate the wave segments
  {
    uint32_t o = segn[0];
#pragma unroll
    for (int q = 1; q < STPB / WAVE; ++q) {
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
      const uint64_t kv = wave_sort_u64(lane < n ? S.key[lane] : ~0ull);
      wave_sync();
      S.key[lane] = kv;
      wave_sync();
      kth = shfl_u64(kv, p.top_k - 1);
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
      const uint64_t kv = wave_sort_u64(lane < n ? S.key[lane] : ~0ull);
      wave_sync();
      S.key[lane] = kv;
      wave_sync();
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
}

// ---------------------------------------------------------------------------------
// k_stream
// ---------------------------------------------------------------------------------
// Ladder rung of dv = vmax - v >= 0 read from the float's bits: exponent and the top
// three mantissa bits, so consecutive rungs differ by 2^(1/8) in dv. Rung 0 holds
// dv < 2^-10, the last rung everything from 2^5.875 on. Monotone in dv.
constexpr int VRUNG = 128;
constexpr uint32_t VRUNG0 = (127u - 10u) << 3;
__device__ __forceinline__ int dv_rung(float dv) {
  const int r = (int)(__float_as_uint(dv) >> 20) - (int)VRUNG0;
  return r < 0 ? 0 : (r > VRUNG - 1 ? VRUNG - 1 : r);
}
// Smallest dv above rung r (r < VRUNG - 1).
__device__ __forceinline__ float dv_rung_end(int r) {
  return __uint_as_float(((uint32_t)r + 1u + VRUNG0) << 20);
}

// The 8 tokens [i0, i0 + 8) of row r as float32 (bf16 widened exactly). FULL: the
// chunk lies inside the row and rows are 16-byte aligned, so one or two vector loads.
template <int DT, bool FULL>
__device__ __forceinline__ void load_seg(const Args& a, int r, int i0, float (&x)[EPT]) {
  const int64_t base = (int64_t)r * a.row_stride;
  if constexpr (DT == STRIM_DTYPE_BF16) {
    const uint16_t* xb = (const uint16_t*)a.logits + base;
    if constexpr (FULL) {
      const uint4 v = *(const uint4*)(xb + i0);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[2 * e] = __uint_as_float(w[e] << 16);
        x[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) x[e] = (i0 + e < a.V) ? bf16_to_f32(xb[i0 + e]) : -INFINITY;
    }
  } else {
    const float* xf = (const float*)a.logits + base;
    if constexpr (FULL) {
      const float4 v0 = *(const float4*)(xf + i0);
      const float4 v1 = *(const float4*)(xf + i0 + 4);
      x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w;
      x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) x[e] = (i0 + e < a.V) ? xf[i0 + e] : -INFINITY;
    }
  }
}

// DT: logits dtype; VEC: rows are 16-byte aligned; PEN: some row of the launch has
// penalties; MASK: allow-bits are given. The host picks the instantiation, so each
// launch runs straight-line per-token code.
template <int DT, bool VEC, bool PEN, bool MASK>
__global__ __launch_bounds__(STPB) void k_stream(Args a) {
  __shared__ StreamShared S;
  uint32_t* s_cnt = S.cnt;

  int r, c;
  map_block(r, c);
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
  const int c0 = c * CHUNK;
  const bool full = VEC && c0 + CHUNK <= a.V;
  int i0[SSEG];
  float v[SSEG][EPT];
  uint32_t bits[SSEG];
#pragma unroll
  for (int s = 0; s < SSEG; ++s) {
    i0[s] = c0 + (s * STPB + t) * EPT;
    if (full) load_seg<DT, true>(a, r, i0[s], v[s]);
    else load_seg<DT, false>(a, r, i0[s], v[s]);
    bits[s] = 0xFFu;
    if constexpr (MASK) {
      if (a.mask && i0[s] < a.V)
        bits[s] = ((const uint8_t*)(a.mask + (int64_t)r * a.mask_stride))[i0[s] >> 3];
    }
  }
  for (int q = t; q < VRUNG; q += STPB) S.lad[q] = 0u;
  if (t < NCB) {
    S.hc[t] = 0u;
    S.hm[t] = 0ull;
  }
  const bool pen = PEN && p.pen;
  if (pen) build_counts_pre<STPB, CHUNK>(a, b, j, c0, s_cnt);

  // ---- penalties and mask, before temperature ("v space") ------------------------
  // Dividing by T > 0 is monotone, so maxima and candidate bounds are found on v; only
  // the chunk maximum and (in k_finalize) the candidates are divided. Tokens past the
  // row end load as -inf (not allowed).
  bool nf = false;
  float vmax = -INFINITY;
  int vid = -1;
#pragma unroll
  for (int s = 0; s < SSEG; ++s) {
    uint32_t cnt[EPT];
    if (pen) {
      const uint4 c4a = *(const uint4*)(s_cnt + (i0[s] - c0));
      const uint4 c4b = *(const uint4*)(s_cnt + (i0[s] - c0) + 4);
      cnt[0] = c4a.x; cnt[1] = c4a.y; cnt[2] = c4a.z; cnt[3] = c4a.w;
      cnt[4] = c4b.x; cnt[5] = c4b.y; cnt[6] = c4b.z; cnt[7] = c4b.w;
    }
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      float y = v[s][e];
      if (pen && cnt[e] > 0u) {
        y = y > 0.0f ? y / p.rep : y * p.rep;
        y = y - p.freq * (float)cnt[e];
        y = y - p.pres;
      }
      if constexpr (MASK) y = ((bits[s] >> e) & 1u) ? y : -INFINITY;
      nf |= !(y < INFINITY);  // NaN or +inf in an allowed position
      v[s][e] = y;
      // ids rise with (s, e): a strict compare keeps the first maximum
      if (y > vmax) {
        vmax = y;
        vid = i0[s] + e;
      }
    }
  }
  if (a.verify && j < a.k) {
    const int d = a.drafts[(int64_t)b * a.k + j];
#pragma unroll
    for (int s = 0; s < SSEG; ++s) {
      const int o = d - i0[s];
      if (o >= 0 && o < EPT) {
        float ld = -INFINITY;
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if (e == o) ld = v[s][e];
        a.s.rs[r].l_draft = (ld > -INFINITY && !p.greedy) ? ld / p.T : ld;
      }
    }
  }
  if (c == 0 && t == 0) a.s.ncand[r] = 0u;

  // ---- chunk max (first id on ties), allowed count, non-finite flag ---------------
  wave_argmax(vmax, vid);
  int n = vmax > -INFINITY ? 1 : 0;  // "some token allowed"; general rows count below
  const int f = __any(nf) ? 1 : 0;
  if (lane == 0) {
    S.v[w] = vmax;
    S.i[w] = vid;
    S.n[w] = n;
    S.f[w] = f;
  }
  __syncthreads();
  float vm = S.v[0];
  int a_w = S.i[0], n_w = S.n[0], f_w = S.f[0];
#pragma unroll
  for (int q = 1; q < STPB / WAVE; ++q) {
    argmax_merge(vm, a_w, S.v[q], S.i[q]);
    n_w |= S.n[q];
    f_w |= S.f[q];
  }
  // chunk max after temperature; an overflow to +inf is a non-finite logit, one to -inf
  // leaves nothing allowed
  const float m_w = (p.greedy || !(vm > -INFINITY)) ? vm : vm / p.T;
  if (m_w == INFINITY) f_w = 1;
  if (!(m_w > -INFINITY)) n_w = 0;
  ChunkStat cs{m_w, a_w, n_w, f_w, 0.0, 0u, -INFINITY};
  const bool live = n_w > 0 && !f_w;

  if (p.cls == CLS_FAST && live) {
    // Local candidates, in v space: every token that can pass min-p (on the row maximum
    // m >= m_w) and the chunk's top-k, written as (v, id) to the wave's slot region.
    const bool topk = p.top_k > 0 && p.top_k < a.V;
    // v >= vlo keeps every token with v / T >= m_w + log(min_p) (rounding margin 4e-7)
    float vlo = -INFINITY;
    if (p.min_p > 0.0f) {
      const double L = (double)m_w + log((double)p.min_p);
      const double tl = L * (double)p.T;
      vlo = (float)(tl - fabs(tl) * 4e-7 - 1e-37);
    }
    if (topk) {
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if (v[s][e] >= vlo && v[s][e] > -INFINITY) atomicAdd(&S.lad[dv_rung(vm - v[s][e])], 1u);
      __syncthreads();
      // every wave finds the first rung whose cumulative count reaches k (lane owns
      // rungs 2 lane and 2 lane + 1)
      const uint32_t h0 = S.lad[2 * lane], h1 = S.lad[2 * lane + 1];
      uint32_t cum = h0 + h1;
#pragma unroll
      for (int o = 1; o < WAVE; o <<= 1) {
        const uint32_t u = (uint32_t)__shfl_up((int)cum, o, WAVE);
        if (lane >= o) cum += u;
      }
      const uint64_t reach = __ballot(cum >= (uint32_t)p.top_k);
      if (reach) {
        const int ln = (int)__ffsll((long long)reach) - 1;
        const uint32_t before = (uint32_t)__shfl((int)(cum - h0 - h1), ln, WAVE);
        const uint32_t hl0 = (uint32_t)__shfl((int)h0, ln, WAVE);
        const int rstar = 2 * ln + (before + hl0 >= (uint32_t)p.top_k ? 0 : 1);
        if (rstar < VRUNG - 1) {
          // v > vm - end(rstar) holds the rung; the margin (a few ulps of the values
          // involved) keeps tokens whose l = v / T ties with one inside it
          const float bnd = dv_rung_end(rstar);
          const float thr = vm - bnd;
          const float margin = (fabsf(vm) + fabsf(thr)) * 1e-6f + bnd * 1.6e-5f + 1e-30f;
          vlo = fmaxf(vlo, thr - margin);
          // the rungs up to rstar hold >= k tokens of the window, all with v >= g
          cs.g = thr - margin;
        }
      }
    }
    uint32_t sel[SSEG];
    int mycnt = 0;
#pragma unroll
    for (int s = 0; s < SSEG; ++s) {
      sel[s] = 0u;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const float y = v[s][e];
        if (y >= vlo && y > -INFINITY) {
          sel[s] |= 1u << e;
          ++mycnt;
        }
      }
    }
    // each wave writes its candidates to its own region of the chunk (no atomics, no
    // barrier); the region counts travel in cs.nslot, one byte per wave
    int wtot;
    const int wex = wave_excl_count32(mycnt, &wtot);
    if (wtot <= SLOTW) {
      Cand* dst = a.s.slot + (((int64_t)r * a.s.wmax + c) * 4 + w) * SLOTW;
      int pos = wex;
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if ((sel[s] >> e) & 1u) dst[pos++] = Cand{v[s][e], i0[s] + e};
    }
    if (lane == 0) S.off[w] = wtot <= SLOTW ? (uint32_t)wtot : 255u;
    __syncthreads();
    cs.nslot = S.off[0] | (S.off[1] << 8) | (S.off[2] << 16) | (S.off[3] << 24);
  } else if (p.cls == CLS_GENERAL && live) {
    // processed logits; chunk sum exp(l - m_w) and a coarse histogram of m_w - l
    // (k_collect's bounds)
    float (&l)[SSEG][EPT] = v;  // v is not needed after this
#pragma unroll
    for (int s = 0; s < SSEG; ++s)
#pragma unroll
      for (int e = 0; e < EPT; ++e) l[s][e] = v[s][e] > -INFINITY ? v[s][e] / p.T : -INFINITY;
    double ssum = 0.0;
    int na = 0;
#pragma unroll
    for (int s = 0; s < SSEG; ++s)
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if (!(l[s][e] > -INFINITY)) continue;
        ++na;
        const float d = m_w - l[s][e];
        const float wgt = expf(-d);
        ssum += (double)wgt;
        const int bb = d < 32.0f ? (int)(d * CB_SCALE) : NCB - 1;
        atomicAdd(&S.hc[bb], 1u);
        const unsigned long long fx = __float2ull_rn(wgt * FIX_SCALE_F);
        if (fx) atomicAdd(&S.hm[bb], fx);
      }
    cs.S = block_sum_f64<STPB>(ssum, S.d);
    na = wave_sum(na);
    if (lane == 0) S.n[w] = na;
    __syncthreads();
    cs.n = S.n[0] + S.n[1] + S.n[2] + S.n[3];
    if (t < NCB) {
      const int64_t o = ((int64_t)r * a.s.wmax + c) * NCB + t;
      a.s.chc[o] = S.hc[t];
      a.s.chm[o] = S.hm[t];
    }
    // unfiltered Gumbel rows: the chunk's two best tokens decide the draw directly
    if (a.noise_mode == STRIM_NOISE_GUMBEL && row_nofilter(p, a.V)) {
      const uint64_t key = mix64(p.seed, p.position);
      float s0 = -INFINITY, s1 = -INFINITY, l0 = 0.f, l1 = 0.f;
      int id0 = -1, id1 = -1;
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          if (!(l[s][e] > -INFINITY)) continue;
          const int id = i0[s] + e;
          const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + id]
                                  : philox_uniform(key, (uint64_t)id);
          top2_merge(s0, l0, id0, s1, l1, id1, l[s][e] + gumbel32(u), l[s][e], id, -INFINITY,
                     0.f, -1);
        }
      block_top2<STPB>(s0, l0, id0, s1, l1, id1, S.tf, S.ti);
      if (t == 0) {
        ChunkPart& pt = a.s.part[(int64_t)r * a.s.wmax + c];
        pt.l0 = l0; pt.id0 = id0; pt.l1 = l1; pt.id1 = id1;
      }
    }
  }
  if (t == 0) a.s.cstat[(int64_t)r * a.s.wmax + c] = cs;
}

// Launches the k_stream instantiation matching the call: dtype, alignment, whether
// any row has penalties, whether a mask is given.
hipError_t launch_stream(const Args& a, dim3 grid, hipStream_t st, bool any_pen) {
  const bool vec = a.vec_ok != 0, mask = a.mask != nullptr;
#define STRIM_STREAM(DT, VEC, PEN, MASK) \
  hipLaunchKernelGGL((k_stream<DT, VEC, PEN, MASK>), grid, dim3(STPB), 0, st, a)
  if (a.dtype == STRIM_DTYPE_BF16) {
    if (!vec) STRIM_STREAM(STRIM_DTYPE_BF16, false, true, true);
    else if (any_pen) {
      if (mask) STRIM_STREAM(STRIM_DTYPE_BF16, true, true, true);
      else STRIM_STREAM(STRIM_DTYPE_BF16, true, true, false);
    } else {
      if (mask) STRIM_STREAM(STRIM_DTYPE_BF16, true, false, true);
      else STRIM_STREAM(STRIM_DTYPE_BF16, true, false, false);
    }
  } else {
    if (!vec) STRIM_STREAM(STRIM_DTYPE_F32, false, true, true);
    else if (any_pen) {
      if (mask) STRIM_STREAM(STRIM_DTYPE_F32, true, true, true);
      else STRIM_STREAM(STRIM_DTYPE_F32, true, true, false);
    } else {
      if (mask) STRIM_STREAM(STRIM_DTYPE_F32, true, false, true);
      else STRIM_STREAM(STRIM_DTYPE_F32, true, false, false);
    }
  }
#undef STRIM_STREAM
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// k_finalize: one workgroup per row, after k_stream (the kernel boundary makes every
// chunk's results visible; an in-kernel device-scope release per workgroup costs far
// more on gfx950 than the second launch)
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(STPB) void k_finalize(Args a) {
  __shared__ FinalShared S;
  const int r = blockIdx.x;
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  finalize_row(a, r, b, j, p, S);
}

}  // namespace strim
