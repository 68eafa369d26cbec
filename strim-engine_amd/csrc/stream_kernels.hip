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
// A row whose candidates do not fit the LDS finalize is marked for k_final's exact path.
#include "select.hpp"

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
// Histogram bin of d = m - l (1/16 nat, last bin open) for k_finalize's top-k cut;
// monotone in l.
__device__ __forceinline__ int dbin(float m, float l) {
  return (int)fminf((m - l) * 16.0f, 255.0f);
}
struct FinalShared {
  uint64_t key[FCAP];       // the row's surviving candidate keys (32 KB)
  uint16_t owner[FCAND];    // candidate position -> wave region (4 * chunk + wave)
  uint32_t rpre[4 * 256];   // first position of each wave region
  uint32_t hist[256];       // radix digits / d-histogram
  float v[STPB / WAVE];
  int i[STPB / WAVE], n[STPB / WAVE], f[STPB / WAVE];
  float g[STPB / WAVE];
  uint32_t off[STPB / WAVE];
  double d[STPB / WAVE];
  uint64_t u[STPB / WAVE];
  int misc[8];
  uint32_t nsurv;
};

// One row per 256-thread workgroup. All threads merge the chunk statistics and gather
// the candidates (every load in flight at once), pruning with the row maximum (min-p)
// and with G = max over chunks of the certified k-th value bound; the survivors are
// decided by wave 0 alone with wave-wide operations (no further barriers).
__device__ void finalize_row(const Args& a, int r, int b, int j, const RowParams& p,
                             FinalShared& S) {
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
  const int V = a.V, W = a.W;
  const bool vdr = a.verify && j < a.k;  // a verify row with a draft
  RowState* rsp = &a.s.rs[r];

  // ---- merge the chunk statistics (W <= 256: one chunk per thread) ----------------
  ChunkStat cs{-INFINITY, -1, 0, 0, 0.0, 0u, -INFINITY};
  if (t < W) cs = a.s.cstat[(int64_t)r * a.s.wmax + t];
  float mv = cs.m, gv = cs.g;
  int mi = cs.arg, nn = cs.n, ff = cs.flags;
  wave_argmax(mv, mi);
  nn = wave_sum(nn);
  ff = wave_or_i(ff);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) gv = fmaxf(gv, __shfl_xor(gv, o, WAVE));
  if (lane == 0) {
    S.v[w] = mv;
    S.i[w] = mi;
    S.n[w] = nn;
    S.f[w] = ff;
    S.g[w] = gv;
  }
  if (t < 256) S.hist[t] = 0u;
  if (t == 0) S.nsurv = 0u;
  __syncthreads();
  float m = S.v[0], G = S.g[0];
  int arg = S.i[0], n_all = S.n[0], flags = S.f[0];
#pragma unroll
  for (int q = 1; q < STPB / WAVE; ++q) {
    argmax_merge(m, arg, S.v[q], S.i[q]);
    n_all += S.n[q];
    flags |= S.f[q];
    G = fmaxf(G, S.g[q]);
  }

  int status = STRIM_OK, draft = -1;
  if (vdr) {
    draft = a.drafts[(int64_t)b * a.k + j];
    if (draft < 0 || draft >= V) status = STRIM_EINVAL;
  }
  if (status == STRIM_OK && flags) status = STRIM_ENONFINITE;
  if (status == STRIM_OK && n_all == 0) status = STRIM_EEMPTY;
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
  const float l_draft = vdr ? rsp->l_draft : -INFINITY;

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
      const float ua = row_uniform(a, r, p, (int64_t)V);
      acc = ((double)ua < w_d / sig) ? 1 : 0;
      if (token < 0) token = arg;  // the draft is the only allowed token
    }
    finish_row(a, r, STRIM_OK, token, acc, sig, m, ~0ull, PH_DONE);
    return;
  }
  if (p.cls != CLS_FAST) {
    finish_row(a, r, STRIM_OK, -1, 0, 0.0, m, 0ull, PH_PENDING);
    return;
  }

  // ---- fast rows: gather, divide, prune and compact the candidates -------------------
  // chunk c's candidates sit in four per-wave regions of SLOTW entries; cs.nslot holds
  // the four counts as bytes (255 = the wave overflowed its region)
  uint32_t ctot = 0u;
  int over = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t ce = t < W ? (cs.nslot >> (8 * e)) & 255u : 0u;
    if (ce > (uint32_t)SLOTW) over = 1;
    ctot += ce;
  }
  uint32_t n_c;
  const uint32_t pre = block_excl_scan_u32<STPB>(over ? 0u : ctot, S.off, &n_c);
  over = block_or<STPB>(over, S.i);
  if (over || n_c > (uint32_t)FCAND) {
    finish_row(a, r, STRIM_OK, -1, 0, 0.0, m, 0ull, PH_EXACT);
    return;
  }
  if (t < W) {
    // the owner table maps each candidate position to its region
    uint32_t o = pre;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t ce = (cs.nslot >> (8 * e)) & 255u;
      S.rpre[4 * t + e] = o;
      for (uint32_t i = 0; i < ce; ++i) S.owner[o + i] = (uint16_t)(4 * t + e);
      o += ce;
    }
  }
  __syncthreads();
  // every kept token has v >= G (the k-th value bound), minus the l-tie margin
  const float Gm = topk && G > -INFINITY ? G - (fabsf(G) * 1e-6f + 1e-30f) : -INFINITY;
  const Cand* slots = a.s.slot + (int64_t)r * a.s.wmax * SLOT;
  const bool minp = p.min_p > 0.0f;
  const double lmp = minp ? log((double)p.min_p) : 0.0;
  constexpr int GQ = FCAP / STPB;
  for (int base = 0; base < (int)n_c; base += FCAP) {
    Cand cd[GQ];
#pragma unroll
    for (int q = 0; q < GQ; ++q) {
      const int pos = base + q * STPB + t;
      cd[q] = Cand{-INFINITY, -1};
      if (pos < (int)n_c) {
        const int rg = S.owner[pos];
        cd[q] = slots[(int64_t)rg * SLOTW + (pos - (int)S.rpre[rg])];
      }
    }
#pragma unroll
    for (int q = 0; q < GQ; ++q) {
      // l = v / T as the oracle rounds it
      bool keep = cd[q].id >= 0 && cd[q].l >= Gm;
      const float l = keep ? cd[q].l / p.T : -INFINITY;
      keep = keep && l > -INFINITY && (!minp || ((double)l - (double)m) >= lmp);
      const uint64_t msk = __ballot(keep);
      if (msk) {
        uint32_t wbase = 0u;
        if (lane == 0) wbase = atomicAdd(&S.nsurv, (uint32_t)__popcll(msk));
        wbase = (uint32_t)__builtin_amdgcn_readfirstlane((int)wbase);
        const uint32_t dst = wbase + (uint32_t)lanes_below(msk);
        if (keep && dst < (uint32_t)FCAP) S.key[dst] = ckey(l, cd[q].id);
        // histogram of d = m - l for the top-k cut
        if (keep && topk) atomicAdd(&S.hist[dbin(m, l)], 1u);
      }
    }
  }
  __syncthreads();
  int n = (int)S.nsurv;
  if (n > FCAP) {
    finish_row(a, r, STRIM_OK, -1, 0, 0.0, m, 0ull, PH_EXACT);
    return;
  }
  if (w != 0) return;  // the rest is one wave

  // ---- top-k: the survivors up to the histogram bin holding the k-th, sorted ---------
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
    // keep the keys in bins <= bstar (a superset of the top k, ordered by key)
    uint32_t n2 = 0u;
    for (int base = 0; base < n; base += WAVE) {
      const int pos = base + lane;
      const uint64_t kv = pos < n ? S.key[pos] : ~0ull;
      const float l = fkey_desc_inv((uint32_t)(kv >> 32));
      const bool keep = pos < n && dbin(m, l) <= bstar;
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
    int cnt = 0;
    for (int base = 0; base < n; base += WAVE) {
      const int pos = base + lane;
      cnt += (pos < n && S.key[pos] <= bound) ? 1 : 0;
    }
    n = wave_sum(cnt);
  }
  // sort the survivors
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

  // ---- top-p over the sorted survivors: lane owns positions [lane*Qn, lane*Qn + Qn) --
  const int Qn = (n + WAVE - 1) / WAVE;
  const int p0 = lane * Qn, p1 = min(n, p0 + Qn);
  const uint64_t* keys = S.key;
  double loc = 0.0;
  for (int q = p0; q < p1; ++q)
    loc += exp((double)fkey_desc_inv((uint32_t)(keys[q] >> 32)) - (double)m);
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
      run += exp((double)fkey_desc_inv((uint32_t)(keys[q] >> 32)) - (double)m);
    }
    n_keep = wave_min_i(fd);
  }
  const int k1 = min(p1, n_keep);
  loc = 0.0;
  for (int q = p0; q < k1; ++q)
    loc += exp((double)fkey_desc_inv((uint32_t)(keys[q] >> 32)) - (double)m);
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

  // ---- draw ---------------------------------------------------------------------
  int token;
  if (a.noise_mode == STRIM_NOISE_ICDF) {
    const float u = row_uniform(a, r, p, 0);
    const double tgt = (double)u * (S_kept - w_d);
    int best = n_keep;
    double run = exk;
    for (int q = p0; q < k1; ++q) {
      const uint64_t key = keys[q];
      const double wq = exp((double)fkey_desc_inv((uint32_t)(key >> 32)) - (double)m);
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
  int acc = 0;
  if (vdr) {
    const float ua = row_uniform(a, r, p, a.noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V : 1);
    acc = ((double)ua < w_d / S_kept) ? 1 : 0;
  }
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
  int i0[SSEG];
  float v[SSEG][EPT];
  uint32_t bits[SSEG];
#pragma unroll
  for (int s = 0; s < SSEG; ++s) {
    i0[s] = c0 + (s * STPB + t) * EPT;
    load_tokens(a, r, i0[s], v[s]);
    bits[s] = load_mask8(a, r, i0[s]);
  }
  for (int q = t; q < VRUNG; q += STPB) S.lad[q] = 0u;
  if (t < NCB) {
    S.hc[t] = 0u;
    S.hm[t] = 0ull;
  }
  if (p.pen) build_counts_pre<STPB, CHUNK>(a, b, j, c0, s_cnt);

  // ---- penalties and mask, before temperature ("v space") ------------------------
  // Dividing by T > 0 is monotone, so maxima and candidate bounds are found on v; only
  // the chunk maximum and (in k_finalize) the candidates are divided.
  bool nf = false;
  float vmax = -INFINITY;
  int vid = -1, n = 0;
#pragma unroll
  for (int s = 0; s < SSEG; ++s) {
    const uint32_t* cnt = s_cnt + (i0[s] - c0);
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      float y = v[s][e];
      if (p.pen) {
        const uint32_t cc = cnt[e];
        if (cc > 0u) {
          y = y > 0.0f ? y / p.rep : y * p.rep;
          y = y - p.freq * (float)cc;
          y = y - p.pres;
        }
      }
      const bool ok = (i0[s] + e < a.V) && ((bits[s] >> e) & 1u);
      y = ok ? y : -INFINITY;
      nf |= !(y < INFINITY) && ok;  // NaN or +inf in an allowed position
      v[s][e] = y;
      n += y > -INFINITY ? 1 : 0;
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
  n = wave_sum(n);
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
    n_w += S.n[q];
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
#pragma unroll
    for (int s = 0; s < SSEG; ++s)
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if (!(l[s][e] > -INFINITY)) continue;
        const float d = m_w - l[s][e];
        const float wgt = expf(-d);
        ssum += (double)wgt;
        const int bb = d < 32.0f ? (int)(d * CB_SCALE) : NCB - 1;
        atomicAdd(&S.hc[bb], 1u);
        const unsigned long long fx = __float2ull_rn(wgt * FIX_SCALE_F);
        if (fx) atomicAdd(&S.hm[bb], fx);
      }
    cs.S = block_sum_f64<STPB>(ssum, S.d);
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
