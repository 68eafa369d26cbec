// sample_kernels.hip — the general path (k_collect, k_final), the validation output
// (k_probs) and the verify combine.
//
// General rows (top-p alone, no filter, very small min-p, large top-k) cannot bound their
// candidates from a chunk's own maximum. k_finalize derives conservative bin bounds from
// k_stream's 64-bin coarse histograms once per row (general.hpp); k_collect collects the
// tokens of the undecided bins and sums the rest exactly; k_final sorts the candidates in LDS by (l desc, id asc) and takes every
// decision in fp64. Rows whose candidates overflow either finalize are decided by k_final's
// exact streaming resolution.
#include "exact.hpp"

namespace strim {

// ---------------------------------------------------------------------------------
// k_collect: general rows
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(TPB) void k_collect(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  __shared__ unsigned long long s_sm[TPB / WAVE][NSEG];
  __shared__ uint32_t s_sc[TPB / WAVE][NSEG];
  __shared__ float s_tf[4 * TPB / WAVE];
  __shared__ int s_ti[2 * TPB / WAVE];

  int r, c;
  map_block(r, c);
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  if (p.cls != CLS_GENERAL) return;
  if (a.noise_mode == STRIM_NOISE_GUMBEL && row_nofilter(p, a.V)) return;
  if (a.s.rs[r].phase != PH_PENDING) return;  // decided, or a general-q row (k_final)
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
  const int c0 = c * CHUNK, i0 = c0 + t * EPT;

  float x[EPT];
  load_tokens(a, r, i0, x);
  // the row maximum and the bin bounds, from k_finalize
  const float m = a.s.rs[r].m;
  const Bounds bd = a.s.rs[r].bd;
  if (bd.mode == MODE_NONE) return;
  if (p.pen) build_counts(a, b, j, c0, s_cnt);

  float l[EPT];
  bool nf = false;
  process_tokens(a, r, i0, p, s_cnt + (i0 & (CHUNK - 1)), x, l, nf);
  const bool want_top = bd.mode == MODE_B && a.noise_mode == STRIM_NOISE_GUMBEL;
  const uint64_t key = mix64(p.seed, p.position);
  unsigned long long sm[NSEG];
  uint32_t sc[NSEG];
#pragma unroll
  for (int q = 0; q < NSEG; ++q) { sm[q] = 0ull; sc[q] = 0u; }
  uint32_t sel = 0u;
  int mycnt = 0;
  float s0 = -INFINITY, s1 = -INFINITY, l0 = 0.f, l1 = 0.f;
  int id0 = -1, id1 = -1;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (!(l[e] > -INFINITY)) continue;
    const float d = m - l[e];
    const int g = gbin(d);
    if (in_rng(bd, g)) {
      sel |= 1u << e;
      ++mycnt;
      continue;
    }
    const int q = seg_of(bd, g);
    const unsigned long long fx = __float2ull_rn(expf(-d) * FIX_SCALE_F);
#pragma unroll
    for (int qq = 0; qq < NSEG; ++qq)
      if (qq == q) { sm[qq] += fx; sc[qq] += 1u; }
    if (want_top && g < bd.s) {
      const int id = i0 + e;
      const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + id]
                              : philox_uniform(key, (uint64_t)id);
      top2_merge(s0, l0, id0, s1, l1, id1, l[e] + gumbel32(u), l[e], id, -INFINITY, 0.f, -1);
    }
  }
  // append the collected tokens (one atomic per wave)
  int tot;
  const int wex = wave_excl_count(mycnt, &tot);
  if (tot > 0) {
    unsigned base = 0;
    if (lane == 0) base = atomicAdd(&a.s.ncand[r], (unsigned)tot);
    base = (unsigned)__builtin_amdgcn_readlane((int)base, 0);
    unsigned pos = base + (unsigned)wex;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if ((sel >> e) & 1u) {
        if (pos < (unsigned)CAP) a.s.cand[(int64_t)r * CAP + pos] = Cand{l[e], i0 + e};
        ++pos;
      }
  }
  // per-interval sums of the tokens not collected
#pragma unroll
  for (int q = 0; q < NSEG; ++q) {
    sm[q] = wave_sum_u64(sm[q]);
    sc[q] = wave_sum(sc[q]);
  }
  if (lane == 0)
#pragma unroll
    for (int q = 0; q < NSEG; ++q) { s_sm[w][q] = sm[q]; s_sc[w][q] = sc[q]; }
  if (want_top) block_top2<TPB>(s0, l0, id0, s1, l1, id1, s_tf, s_ti);
  else __syncthreads();
  if (t == 0) {
    ChunkPart& pt = a.s.part[(int64_t)r * a.s.wmax + c];
    for (int q = 0; q < NSEG; ++q) {
      unsigned long long tm = 0ull;
      uint32_t tc = 0u;
      for (int ww = 0; ww < TPB / WAVE; ++ww) { tm += s_sm[ww][q]; tc += s_sc[ww][q]; }
      pt.mass[q] = tm;
      pt.cnt[q] = tc;
    }
    pt.l0 = l0; pt.id0 = want_top ? id0 : -1;
    pt.l1 = l1; pt.id1 = want_top ? id1 : -1;
  }
}

// ---------------------------------------------------------------------------------
// k_final
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(FIN_T) void k_final(Args a) {
  __shared__ uint64_t s_key[CAP];
  __shared__ double s_w[CAP];
  __shared__ double s_dred[FIN_T / WAVE];
  __shared__ uint64_t s_ured[FIN_T / WAVE];
  __shared__ int s_ired[FIN_T / WAVE];
  __shared__ int s_int[8];
  __shared__ float s_kth;
  __shared__ uint32_t s_pre[256];
  __shared__ uint32_t s_ns[256];
  __shared__ double s_segm[NSEG];
  __shared__ uint32_t s_segc[NSEG];
  __shared__ int s_segk[NSEG];  // 2 = kept, 1 = pre-kept only, 0 = neither
  __shared__ uint32_t s_bcb[NGB];   // per global bin g: seg_before(g), tabulated
  __shared__ double s_bpb[NGB], s_bkb[NGB];
  __shared__ Bounds s_bd;
  __shared__ uint64_t s_u2[2 * FIN_T / WAVE];
  __shared__ XState s_x;

  const int r = blockIdx.x;
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  const int t = threadIdx.x;
  const int V = a.V;
  const bool verify_draft_row = a.verify && j < a.k;
  RowState* rsp = &a.s.rs[r];
  // k_finalize decided every row except the general rows (PENDING)
  const int phase = rsp->phase;
  if (phase == PH_DONE) return;

  // k_finalize has checked the row (status, draft) and left its maximum and first argmax
  const float m = rsp->m;
  const int arg = rsp->token;
  int status = STRIM_OK;
  int draft = -1;
  if (verify_draft_row) {
    draft = a.drafts[(int64_t)b * a.k + j];
    if (draft < 0 || draft >= V) status = STRIM_EINVAL;
  }
  if (status == STRIM_OK && !p.greedy && phase == PH_PENDING) {
    if (t == 0) s_bd = rsp->bd;
    __syncthreads();
  }
  // rows the candidate path cannot hold go to the exact streaming resolution
  bool exact = status == STRIM_OK && !p.greedy && (phase == PH_EXACT || s_bd.mode == MODE_NONE);
  auto finish = [&](int stt, int token, int accept, double sig, uint64_t lk) {
    if (t == 0) {
      rsp->status = stt;
      rsp->token = token;
      rsp->accept = accept;
      rsp->sum_kept = sig;
      rsp->m = m;
      rsp->last_key = lk;
      if (!a.verify) {
        a.out_ids[r] = stt == STRIM_OK ? token : -1;
        if (a.out_status) a.out_status[r] = stt;
      }
    }
  };
  if (status != STRIM_OK) {
    finish(status, -1, 0, 0.0, 0ull);
    return;
  }
  if (p.greedy) {
    finish(STRIM_OK, arg, verify_draft_row && arg == draft, 1.0, 0ull);
    return;
  }
  const int W = a.W;
  const bool topk = p.top_k > 0 && p.top_k < V;
  const bool topp = p.top_p < 1.0f;
  const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
  const bool by_rank = (p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp;
  const bool cand_sorted = no_lse ? topp : (topk || topp);
  const uint64_t pkey = mix64(p.seed, p.position);
  const int excl_id = verify_draft_row ? draft : -1;

  if (!exact) do {
  // ---- gather candidates --------------------------------------------------------
  int n = 0;
  {
    n = (int)a.s.ncand[r];
    if (n > CAP) {
      exact = true;
      break;
    }
    // per-chunk interval sums staged in LDS (s_w is free until the masses are computed),
    // then summed in chunk order by one thread per interval
    unsigned long long* st_m = (unsigned long long*)s_w;   // [NSEG][W]
    uint32_t* st_c = (uint32_t*)(st_m + NSEG * W);          // [NSEG][W]
    for (int e = t; e < W * NSEG; e += FIN_T) {
      const int cc = e / NSEG, q = e - cc * NSEG;
      const ChunkPart& pt = a.s.part[(int64_t)r * a.s.wmax + cc];
      st_m[q * W + cc] = pt.mass[q];
      st_c[q * W + cc] = pt.cnt[q];
    }
    __syncthreads();
    if (t < NSEG) {
      unsigned long long tm = 0ull;
      uint32_t tc = 0u;
      for (int cc = 0; cc < W; ++cc) {
        tm += st_m[t * W + cc];
        tc += st_c[t * W + cc];
      }
      s_segm[t] = (double)tm * (1.0 / FIX_SCALE);
      s_segc[t] = tc;
      const bool valid = s_bd.seg_lo[t] <= s_bd.seg_hi[t];
      s_segk[t] = !valid ? 0 : (s_bd.seg_hi[t] < s_bd.s ? 2 : (s_bd.seg_hi[t] < s_bd.s1 ? 1 : 0));
    }
    __syncthreads();
  }
  uint64_t kk[FIN_Q];
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    const int idx = q * FIN_T + t;
    kk[q] = ~0ull;
    if (idx < n) {
      const Cand cd = a.s.cand[(int64_t)r * CAP + idx];
      kk[q] = ckey(cd.l, cd.id);
    }
  }
  if (t == 0) s_kth = -INFINITY;
  sort_keys(kk, n, s_key, (uint64_t*)s_w);

  // ---- per-position data lives in LDS: keys in s_key, fp64 masses in s_w ----------
  const bool minp = p.min_p > 0.0f;
  const double lmp = p.lmp;
  const bool keep_ties = (p.flags & STRIM_FLAG_TOPK_KEEP_TIES) != 0;
  // non-collected tokens before global coarse bin g: count, pre-kept mass, kept mass,
  // summed in interval order once per bin
  for (int g = t; g < NGB; g += FIN_T) {
    uint32_t cb = 0u;
    double pb = 0.0, kb = 0.0;
#pragma unroll
    for (int s = 0; s < NSEG; ++s)
      if (s_bd.seg_lo[s] <= s_bd.seg_hi[s] && s_bd.seg_hi[s] < g) {
        cb += s_segc[s];
        if (s_segk[s] >= 1) pb += s_segm[s];
        if (s_segk[s] == 2) kb += s_segm[s];
      }
    s_bcb[g] = cb;
    s_bpb[g] = pb;
    s_bkb[g] = kb;
  }
  __syncthreads();
  auto seg_before = [&](int g, uint32_t& cb, double& pb, double& kb) {
    cb = s_bcb[g];
    pb = s_bpb[g];
    kb = s_bkb[g];
  };
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    const int pos = t * FIN_Q + q;
    if (pos >= n) break;
    const uint64_t key = s_key[pos];
    const float l = fkey_desc_inv((uint32_t)(key >> 32));
    s_w[pos] = exp((double)l - (double)m);
    if (topk && keep_ties) {
      uint32_t cb;
      double pb, kb;
      seg_before(gbin(m - l), cb, pb, kb);
      if (cb + (uint32_t)pos == (uint32_t)(p.top_k - 1)) s_kth = l;
    }
  }
  __syncthreads();
  const float kth = s_kth;
  double seg_pre = 0.0, seg_kept = 0.0;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
      if (s_segk[s] >= 1) seg_pre += s_segm[s];
      if (s_segk[s] == 2) seg_kept += s_segm[s];
    }

  // ---- pre-filters (min-p, top-k): a prefix of the order ---------------------------
  int first_bad = n;
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    const int pos = t * FIN_Q + q;
    if (pos >= n) break;
    const uint64_t key = s_key[pos];
    const float l = fkey_desc_inv((uint32_t)(key >> 32));
    bool ok = true;
    if (minp) ok = ((double)l - (double)m) >= lmp;
    if (ok && topk) {
      if (keep_ties) {
        ok = l >= kth;
      } else {
        uint32_t cb;
        double pb, kb;
        seg_before(gbin(m - l), cb, pb, kb);
        ok = cb + (uint32_t)pos < (uint32_t)p.top_k;
      }
    }
    if (!ok && pos < first_bad) first_bad = pos;
  }
  const int n_pre = block_min<FIN_T>(first_bad, s_ired);

  // ---- top-p over the pre-kept set ---------------------------------------------------
  double loc = 0.0;
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    const int pos = t * FIN_Q + q;
    if (pos < n_pre) loc += s_w[pos];
  }
  double tot_pre;
  const double ex = block_excl_scan_f64<FIN_T>(loc, s_dred, &tot_pre);
  const double sig_pre = seg_pre + tot_pre;
  int n_keep = n_pre;
  if (topp) {
    const double P = (double)p.top_p;
    int fd = n;
    double run = ex;
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q) {
      const int pos = t * FIN_Q + q;
      if (pos >= n_pre) break;
      uint32_t cb;
      double pb, kb;
      seg_before(gbin(m - fkey_desc_inv((uint32_t)(s_key[pos] >> 32))), cb, pb, kb);
      const double before = pb + run;
      if (before / sig_pre - P > 0.0 && pos < fd) fd = pos;
      run += s_w[pos];
    }
    n_keep = block_min<FIN_T>(min(fd, n_pre), s_ired);
  }
  loc = 0.0;
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    const int pos = t * FIN_Q + q;
    if (pos < n_keep) loc += s_w[pos];
  }
  double tot_keep;
  const double exk = block_excl_scan_f64<FIN_T>(loc, s_dred, &tot_keep);
  const double sig_k = seg_kept + tot_keep;
  const uint64_t last_key = n_keep > 0 ? s_key[n_keep - 1] : 0ull;

  // the draft (verify rows): kept? and its mass
  double w_d = 0.0;
  uint64_t key_d = ~0ull;
  if (verify_draft_row && rsp->l_draft > -INFINITY) {
    const float ld = rsp->l_draft;
    key_d = ckey(ld, draft);
    bool kept_d;
    const int g = gbin(m - ld);
    kept_d = in_rng(s_bd, g) ? (last_key != 0ull && key_d <= last_key) : (g < s_bd.s);
    if (kept_d) w_d = exp((double)ld - (double)m);
  }

  // ---- draw --------------------------------------------------------------------------
  int token = -1;
  if (a.noise_mode == STRIM_NOISE_ICDF) {
    const float u = row_uniform(a, r, p, 0);
    const double sig_r = sig_k - w_d;
    const double tgt = (double)u * sig_r;
    int best = n;
    double run = exk;
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q) {
      const int pos = t * FIN_Q + q;
      if (pos >= n_keep) break;
      const uint64_t key = s_key[pos];
      uint32_t cb;
      double pb, kb;
      seg_before(gbin(m - fkey_desc_inv((uint32_t)(key >> 32))), cb, pb, kb);
      double before = kb + run;
      if (key_d < key) before -= w_d;
      const double wq = ((int)(uint32_t)key == excl_id) ? 0.0 : s_w[pos];
      if (wq > 0.0 && before + wq > tgt && pos < best) best = pos;
      run += s_w[pos];
    }
    int bp = block_min<FIN_T>(best, s_ired);
    if (bp >= n_keep) {
      // rounding pushed the target past the last collected kept token
      const bool all_collected = s_bd.mode == MODE_A;
      bp = (all_collected && n_keep > 0) ? n_keep - 1 : -1;
      if (bp >= 0 && (int)(uint32_t)s_key[bp] == excl_id) bp = bp > 0 ? bp - 1 : -1;
    }
    if (bp < 0) {
      exact = true;
      break;
    }
    token = (int)(uint32_t)s_key[bp];
  } else {
    const double lse = log(sig_k);
    double bsc = -INFINITY;
    uint64_t btk = ~0ull;
    int bid = -1;
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q) {
      const int pos = t * FIN_Q + q;
      if (pos >= n_keep) break;
      const uint64_t key = s_key[pos];
      const int id = (int)(uint32_t)key;
      if (id == excl_id) continue;
      const float l = fkey_desc_inv((uint32_t)(key >> 32));
      int64_t nidx = id;
      if (by_rank) {
        uint32_t cb;
        double pb, kb;
        seg_before(gbin(m - l), cb, pb, kb);
        nidx = (int64_t)(cb + (uint32_t)pos);
      }
      const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + nidx]
                              : philox_uniform(pkey, (uint64_t)nidx);
      const double base = no_lse ? (double)l : ((double)l - (double)m) - lse;
      const double sc = base + gumbel64(u);
      const uint64_t tk = cand_sorted ? key : (uint64_t)id;
      if (bid < 0 || sc > bsc || (sc == bsc && tk < btk)) { bsc = sc; btk = tk; bid = id; }
    }
    if (s_bd.mode == MODE_B) {
      for (int cc = t; cc < W; cc += FIN_T) {
        const ChunkPart pt = a.s.part[(int64_t)r * a.s.wmax + cc];
        for (int h = 0; h < 2; ++h) {
          const int id = h == 0 ? pt.id0 : pt.id1;
          const float l = h == 0 ? pt.l0 : pt.l1;
          if (id < 0 || id == excl_id) continue;
          const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + id]
                                  : philox_uniform(pkey, (uint64_t)id);
          const double base = no_lse ? (double)l : ((double)l - (double)m) - lse;
          const double sc = base + gumbel64(u);
          const uint64_t tk = cand_sorted ? ckey(l, id) : (uint64_t)id;
          if (bid < 0 || sc > bsc || (sc == bsc && tk < btk)) { bsc = sc; btk = tk; bid = id; }
        }
      }
    }
    block_argmax_score<FIN_T>(bsc, btk, bid, s_dred, s_ured, s_ired, &s_int[3]);
    token = s_int[3];
    if (token < 0) token = n_keep > 0 ? (int)(uint32_t)s_key[0] : -1;  // every score -inf
    if (token < 0) {
      exact = true;
      break;
    }
  }
  int acc = 0;
  if (verify_draft_row) {
    const double p_d = w_d / sig_k;
    const float ua = row_uniform(a, r, p, a.noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V : 1);
    acc = ((double)ua < p_d) ? 1 : 0;
  }
  finish(STRIM_OK, token, acc, sig_k, last_key);
  return;
  } while (0);

  // ---- exact streaming resolution ---------------------------------------------------
  XScratch xs;
  xs.key = s_key;
  xs.hc = (uint32_t*)(s_key + XB);
  xs.cnt = (uint32_t*)s_w;
  xs.u2 = s_u2;
  xs.dred = s_dred;
  xs.ured = s_ured;
  xs.ired = s_ired;
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
  xa.has_q = phase == PH_EXACT ? 1 : 0;
  if (xa.has_q) {
    // the draft distribution q of a general-q verify row (k_qprep)
    const int qr = b * a.k + j;
    const QStat qs = a.s.qst[qr];
    xa.q.dbits = a.s.dbits;
    xa.q.vq = a.s.vq + (size_t)qr * (size_t)a.s.wmax * CHUNK;
    xa.q.mq = qs.mq;
    xa.q.Z = qs.Z;
  }
  const XOut xo = exact_row<FIN_T>(xa, r, b, j, p, m, arg, draft, verify_draft_row,
                            verify_draft_row ? rsp->l_draft : -INFINITY, xs, s_x);
  if (t == 0 && phase == PH_PENDING) rsp->bd.mode = MODE_A;  // kept set = order prefix up to last_key
  finish(xo.status, xo.token, xo.accept, xo.sig, xo.last_key);
}

// ---------------------------------------------------------------------------------
// k_probs: processed distribution (validation output)
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(TPB) void k_probs(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  int r, c;
  map_block(r, c);
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  const RowState rs = a.s.rs[r];
  const int c0 = c * CHUNK, i0 = c0 + (int)threadIdx.x * EPT;
  float* out = a.out_probs + (int64_t)r * a.V;
  if (rs.status != STRIM_OK || p.greedy) {
    for (int e = 0; e < EPT; ++e)
      if (i0 + e < a.V) out[i0 + e] = (rs.status == STRIM_OK && i0 + e == rs.token) ? 1.0f : 0.0f;
    return;
  }
  float x[EPT];
  load_tokens(a, r, i0, x);
  if (p.pen) build_counts(a, b, j, c0, s_cnt);
  float l[EPT];
  bool nf = false;
  process_tokens(a, r, i0, p, s_cnt + (i0 & (CHUNK - 1)), x, l, nf);
  const bool general_b = p.cls == CLS_GENERAL && rs.bd.mode == MODE_B &&
                         !(a.noise_mode == STRIM_NOISE_GUMBEL && row_nofilter(p, a.V));
  for (int e = 0; e < EPT; ++e) {
    const int i = i0 + e;
    if (i >= a.V) break;
    float pv = 0.0f;
    if (l[e] > -INFINITY) {
      bool kept;
      const uint64_t ky = ckey(l[e], i);
      if (general_b) {
        const int g = gbin(rs.m - l[e]);
        kept = in_rng(rs.bd, g) ? (rs.last_key != 0ull && ky <= rs.last_key) : (g < rs.bd.s);
      } else {
        kept = rs.last_key != 0ull && ky <= rs.last_key;
      }
      if (kept) pv = (float)(exp((double)l[e] - (double)rs.m) / rs.sum_kept);
    }
    out[i] = pv;
  }
}

// ---------------------------------------------------------------------------------
// k_verify_combine: leading accepts and the decided token per sequence
// ---------------------------------------------------------------------------------
__global__ void k_verify_combine(Args a) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  const int k = a.k;
  int status = STRIM_OK, n = 0, token = -1;
  bool alive = true;
  // SpecSampling.verify consumes only the rows its accept chain reaches, 0 .. n
  // (SpecSampling.swift:101-105): a row error counts for the sequence only when the chain
  // reaches that row; later rows report theirs in the per-row outputs alone
  for (int j = 0; j <= k; ++j) {
    const RowState& rs = a.s.rs[(int64_t)b * (k + 1) + j];
    if (rs.status != STRIM_OK) {
      if (alive) {
        status = rs.status;
        alive = false;
      }
      if (a.out_row_accept && j < k) a.out_row_accept[(int64_t)b * k + j] = 0;
      if (a.out_row_token) a.out_row_token[(int64_t)b * (k + 1) + j] = -1;
      continue;
    }
    const int acc = j < k ? rs.accept : 0;
    if (a.out_row_accept && j < k) a.out_row_accept[(int64_t)b * k + j] = acc;
    if (a.out_row_token) a.out_row_token[(int64_t)b * (k + 1) + j] = rs.token;
    if (alive) {
      if (j < k && acc) ++n;
      else {
        alive = false;
        token = rs.token;
      }
    }
  }
  if (status != STRIM_OK) {
    n = 0;
    token = -1;
  }
  a.out_accepted[b] = n;
  a.out_token[b] = token;
  if (a.out_status) a.out_status[b] = status;
}

// ---------------------------------------------------------------------------------
// k_qprep: general-q verify inputs (runs before k_stream)
// ---------------------------------------------------------------------------------
// Lower bound of `id` in the ascending table [0, n).
__device__ __forceinline__ int table_lower_bound(const int32_t* tab, int n, int id) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (tab[mid] < id) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// QPT-thread workgroups. Blocks [0, B*k*QSPLIT): slice sp of draft row qr (blk = qr *
// QSPLIT + sp, 1/QSPLIT of the table each): the slice maximum of v = draft_logit / T
// (fp32 division, as the target's temperature), the slice's sum of exp(v - max) in fp64,
// the table index of the row's draft token if the slice holds it, and v stored at each
// table id of the row's dense array (the draft distribution of SpecSampling's general-q
// extension); row 0's slices also check that the table is strictly ascending inside
// [0, V). k_qcombine merges the slices. Blocks after them: one thread per table entry
// builds the membership bitmap: the first entry of each 32-id word writes the word's
// bits and zeroes the empty words before it (the last entry also those after it), so
// every word is written once.
__global__ __launch_bounds__(QPT) void k_qprep(Args a) {
  __shared__ float s_m[QPT / WAVE];
  __shared__ double s_d[QPT / WAVE];
  __shared__ int s_bad[QPT / WAVE];
  const int t = threadIdx.x;
  const int nq = a.B * a.k, Vd = a.Vd;
  const int blk = blockIdx.x;
  if (blk < nq * QSPLIT) {
    // slice sp of draft row qr: table entries [lo, hi)
    const int qr = blk / QSPLIT, sp = blk - qr * QSPLIT;
    const int span = (Vd + QSPLIT - 1) / QSPLIT;
    const int lo = min(Vd, sp * span), hi = min(Vd, lo + span);
    const int b = qr / a.k, j = qr % a.k;
    const int d = a.drafts[(int64_t)b * a.k + j];
    const float T = a.p[b].temperature;
    const size_t base = (size_t)qr * (size_t)Vd;
    float* vq = a.s.vq + (size_t)qr * (size_t)a.s.wmax * CHUNK;
    auto ld = [&](int i) -> float {
      return a.dtype == STRIM_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)a.dlog)[base + i])
                                         : ((const float*)a.dlog)[base + i];
    };
    // batches of QB entries per thread: every load of a batch is issued before its
    // stores (a store could alias a later load, which would serialise the loop). One
    // pass: the table check (row 0), the draft's table index, v = logit / T at each id
    // and the maximum.
    constexpr int QB = 4;
    const bool live = T > 0.0f;
    float mx = -INFINITY;
    int bad = 0, td = -1;
    for (int i0 = lo + t; i0 < hi; i0 += QB * QPT) {
      float v[QB];
      int id[QB], idn[QB];
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        const int i = i0 + q * QPT < hi ? i0 + q * QPT : lo;
        v[q] = ld(i);
        id[q] = a.dtable[i];
        idn[q] = a.dtable[i + 1 < Vd ? i + 1 : i];
      }
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        const int i = i0 + q * QPT;
        if (i >= hi) continue;
        if (id[q] < 0 || id[q] >= a.V || (i + 1 < Vd && !(id[q] < idn[q]))) bad = 1;
        if (id[q] == d) td = i;
        if (live) {
          v[q] = v[q] / T;
          mx = fmaxf(mx, v[q]);
          if (id[q] >= 0 && id[q] < a.V) vq[id[q]] = v[q];
        }
      }
    }
    if (qr == 0) bad = block_or<QPT>(bad, s_bad);
    td = -block_min<QPT>(-td, s_bad);  // at most one entry holds the draft
    QPart q{-INFINITY, td, 0.0, bad, 0};
    if (live) {
      mx = wave_max_f(mx);
      if ((t & (WAVE - 1)) == 0) s_m[t / WAVE] = mx;
      __syncthreads();
      mx = s_m[0];
#pragma unroll
      for (int w = 1; w < QPT / WAVE; ++w) mx = fmaxf(mx, s_m[w]);
      double z = 0.0;
      for (int i0 = lo + t; i0 < hi; i0 += QB * QPT) {
        float v[QB];
#pragma unroll
        for (int w = 0; w < QB; ++w) v[w] = ld(i0 + w * QPT < hi ? i0 + w * QPT : lo);
#pragma unroll
        for (int w = 0; w < QB; ++w)
          if (i0 + w * QPT < hi) z += exp((double)(v[w] / T) - (double)mx);
      }
      z = block_sum_f64<QPT>(z, s_d);
      q.m = mx;
      q.z = z;
    }
    if (t == 0) a.s.qpp[blk] = q;
    return;
  }
  const int i = (blk - nq * QSPLIT) * QPT + t;
  if (i >= Vd) return;
  const int words = (a.V + 31) / 32;
  const int id = a.dtable[i];
  if (id < 0 || id >= a.V) return;  // an invalid table: every general-q row is rejected
  const int w = id >> 5;
  const int pw = i > 0 ? (a.dtable[i - 1] >> 5) : -1;
  if (pw == w) return;
  uint32_t bits = 0u;
  for (int e = i; e < Vd; ++e) {
    const int ide = a.dtable[e];
    if (ide < 0 || (ide >> 5) != w) break;
    bits |= 1u << (ide & 31);
  }
  a.s.dbits[w] = bits;
  for (int z = max(pw + 1, 0); z < w; ++z) a.s.dbits[z] = 0u;
  if (i == Vd - 1)
    for (int z = w + 1; z < words; ++z) a.s.dbits[z] = 0u;
}

// k_qcombine: one thread per draft row merges its QSPLIT slices into the row's QStat
// (maximum, Z rescaled to it, the draft's index) and row 0's table check into qflag.
__global__ void k_qcombine(Args a) {
  const int t = threadIdx.x;
  const int nq = a.B * a.k;
  if (t >= nq) return;
  const QPart* pp = a.s.qpp + (size_t)t * QSPLIT;
  const float T = a.p[t / a.k].temperature;
  float m = -INFINITY;
  int td = -1, bad = 0;
  for (int s = 0; s < QSPLIT; ++s) {
    m = fmaxf(m, pp[s].m);
    td = max(td, pp[s].td);
    bad |= pp[s].bad;
  }
  double z = 0.0;
  for (int s = 0; s < QSPLIT; ++s)
    if (pp[s].m > -INFINITY) z += pp[s].z * exp((double)pp[s].m - (double)m);
  QStat q{-INFINITY, -1, 0.0};
  if (T > 0.0f) {
    q.mq = m;
    q.td = td;
    q.Z = z;
  }
  a.s.qst[t] = q;
  if (t == 0) *a.s.qflag = bad ? 0 : 1;
}

}  // namespace strim
