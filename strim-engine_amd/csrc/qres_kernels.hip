// qres_kernels.hip — the residual draw of general-q verify rows on the whole chip.
//
// An unfiltered general-q draft row with an icdf draw (phase QRES) draws from the
// residual max(0, p - q) over every allowed token, in the token order (l descending, id
// ascending), with the fixed-point masses of the exact streaming resolution (exact.hpp:
// 2^43 per unit of exp(l - m), so every sum is exact and independent of order): the
// drawn token is the last one whose residual mass before it is <= T = floor(u R), R the
// row's residual mass. The exact resolution makes these passes with one workgroup per
// row; here each pass runs on a (chunks, rows) grid. The row's plain mass S (2^43 units
// of exp(l - m)) comes from k_stream's fp64 chunk sums, placed per chunk by k_finalize:
//   k_qhist     per chunk: residual weights (they need S), counts and masses in QNB
//               coarse bins of d = m - l (1/4 nat; monotone along the order)
//   k_qpick     per row: R, T, the last non-empty bin whose mass before it is <= T
//   k_qcollect  per chunk: the tokens of that bin
//   k_qfinal    per row: sorts them, finds the token, the p(d) / q(d) accept
// A bin with more than CAP tokens leaves the row to k_final's exact resolution.
//
// With Gumbel noise the draw is the argmax over the row of log(p - q) + g (log p where
// q = 0, tokens with p <= q excluded), ties to the smaller id:
//   k_qgumbel   per chunk: the chunk's best (score, id); the sequence's last workgroup
//               to finish then takes each row's best over the chunks and the p(d) / q(d)
//               accept, then the sequence's accept chain when nothing follows.
#include "exact.hpp"

namespace strim {

// Coarse bin of a token: floor(4 (m - l)), the last bin open.
__device__ __forceinline__ int q_bin(float l, float m) {
  const double d = (double)m - (double)l;
  return d < (double)(QNB - 1) / 4.0 ? (int)(d * 4.0) : QNB - 1;
}

// The draft distribution of draft row qr = b * k + j (k_qprep).
// With a.qskip (only (accepted, token) asked for), k_finalize has taken every draft
// row's accept test, and a row in phase QRES needs its residual draw only when every
// earlier row of its sequence was accepted (the first rejection); the draws of later
// rows are not read.
__device__ __forceinline__ bool q_needed(const Args& a, int b, int j) {
  if (!a.qskip) return true;
  for (int q = 0; q < j; ++q) {
    const RowState& rs = a.s.rs[(int64_t)b * (a.k + 1) + q];
    if (rs.status != STRIM_OK || !rs.accept) return false;
  }
  return true;
}


// Residual weight of a token of plain weight W: max(0, W - round(q S)) where q > 0
// (x_wt's rule with the kept mass S).
__device__ __forceinline__ uint64_t q_resid(uint64_t W, double q, uint64_t S) {
  if (q == 0.0) return W;
  const uint64_t qS = (uint64_t)__double2ull_rn(q * (double)S);
  return W > qS ? W - qS : 0ull;
}

// The processed logits of this thread's EPT tokens of chunk c, as k_stream computes
// them (every thread of the workgroup calls it: the history counts use barriers).
__device__ __forceinline__ void q_tokens(const Args& a, int r, int b, int j, const RowParams& p,
                                         int c, uint32_t* s_cnt, float (&l)[EPT]) {
  const int c0 = c * CHUNK, i0 = c0 + (int)threadIdx.x * EPT;
  float x[EPT];
  load_tokens(a, r, i0, x);
  if (p.pen) build_counts(a, b, j, c0, s_cnt);
  bool nf = false;
  process_tokens(a, r, i0, p, s_cnt + (i0 & (CHUNK - 1)), x, l, nf);
}

template <int NT>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* scratch) {
  v = wave_sum_u64(v);
  if ((threadIdx.x & (WAVE - 1)) == 0) scratch[threadIdx.x / WAVE] = v;
  __syncthreads();
  uint64_t s = 0ull;
#pragma unroll
  for (int q = 0; q < NT / WAVE; ++q) s += scratch[q];
  __syncthreads();
  return s;
}

__global__ __launch_bounds__(TPB) void k_qhist(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  __shared__ uint64_t s_red[TPB / WAVE];
  __shared__ uint32_t s_hc[QNB];
  __shared__ uint64_t s_hm[QNB];
  int r, c;
  map_block(a, r, c);
  int b, j;
  row_bj(a, r, b, j);
  if (a.s.rs[r].phase != PH_QRES) return;
  const int t = threadIdx.x, qr = b * a.k + j;
  const RowParams p = load_params(a, b, j);
  const float m = a.s.rs[r].m;
  // S: the plain masses of the row's chunks (integers, so any order)
  const uint64_t sp = t < a.W ? a.s.qpart[(size_t)qr * a.s.wmax + t] : 0ull;
  float l[EPT];
  q_tokens(a, r, b, j, p, c, s_cnt, l);
  if (t < QNB) {
    s_hc[t] = 0u;
    s_hm[t] = 0ull;
  }
  const uint64_t S = block_sum_u64<TPB>(sp, s_red);
  const XQ q = q_of_row(a, qr);
  const int i0 = c * CHUNK + t * EPT;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (!(l[e] > -INFINITY)) continue;
    const uint64_t rr = q_resid(x_weight(l[e], m), xq_prob(q, i0 + e), S);
    const int g = q_bin(l[e], m);
    atomicAdd(&s_hc[g], 1u);
    atomicAdd((unsigned long long*)&s_hm[g], (unsigned long long)rr);
  }
  __syncthreads();
  if (t < QNB) {
    const size_t o = ((size_t)qr * a.s.wmax + c) * QNB + t;
    a.s.qhc[o] = s_hc[t];
    a.s.qhm[o] = s_hm[t];
  }
}

// One row per QNB-thread workgroup: thread g owns coarse bin g.
__global__ __launch_bounds__(QNB) void k_qpick(Args a) {
  __shared__ uint64_t s_red[QNB / WAVE];
  __shared__ uint64_t s_u2[2 * QNB / WAVE];
  __shared__ int s_i[QNB / WAVE];
  __shared__ uint32_t s_bc;
  __shared__ uint64_t s_bm;
  const int r = blockIdx.x;
  int b, j;
  row_bj(a, r, b, j);
  RowState* rs = &a.s.rs[r];
  if (rs->phase != PH_QRES) return;
  const int t = threadIdx.x, qr = b * a.k + j, W = a.W;
  const RowParams p = load_params(a, b, j);
  const uint64_t sp = t < W ? a.s.qpart[(size_t)qr * a.s.wmax + t] : 0ull;
  uint32_t cc = 0u;
  uint64_t cm = 0ull;
  for (int c = 0; c < W; ++c) {
    const size_t o = ((size_t)qr * a.s.wmax + c) * QNB + t;
    cc += a.s.qhc[o];
    cm += a.s.qhm[o];
  }
  const uint64_t S = block_sum_u64<QNB>(sp, s_red);
  uint64_t exc, exm, totc, totm;
  block_excl_scan2_u64<QNB>(cc, cm, s_u2, exc, exm, totc, totm);
  const double uu = (double)row_uniform(a, r, p, 0);
  const uint64_t T = (uint64_t)floor(uu * (double)totm);
  // the last non-empty bin whose residual mass before it is <= T
  const int mine = (cc > 0u && exm <= T) ? t : -1;
  const int best = -block_min<QNB>(-mine, s_i);
  if (t == best) {
    s_bc = cc;
    s_bm = exm;
  }
  __syncthreads();
  if (t == 0) {
    rs->qS = S;
    rs->qR = totm;
    rs->qT = T;
    rs->qbin = best;
    rs->qbelow = best >= 0 ? s_bm : 0ull;
    if (best >= 0 && s_bc > (uint32_t)CAP) rs->phase = PH_EXACT;  // k_final resolves it
  }
}

__global__ __launch_bounds__(TPB) void k_qcollect(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  int r, c;
  map_block(a, r, c);
  int b, j;
  row_bj(a, r, b, j);
  const RowState* rs = &a.s.rs[r];
  if (rs->phase != PH_QRES) return;
  const int qbin = rs->qbin;
  if (qbin < 0) return;
  const int t = threadIdx.x, lane = t & (WAVE - 1);
  const RowParams p = load_params(a, b, j);
  const float m = rs->m;
  float l[EPT];
  q_tokens(a, r, b, j, p, c, s_cnt, l);
  const int i0 = c * CHUNK + t * EPT;
  uint32_t sel = 0u;
  int mycnt = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e)
    if (l[e] > -INFINITY && q_bin(l[e], m) == qbin) {
      sel |= 1u << e;
      ++mycnt;
    }
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
}

__global__ __launch_bounds__(FIN_T) void k_qfinal(Args a) {
  __shared__ uint64_t s_key[CAP];
  __shared__ uint64_t s_tmp[CAP];
  __shared__ uint64_t s_u2[2 * FIN_T / WAVE];
  __shared__ int s_i[FIN_T / WAVE];
  const int r = blockIdx.x;
  int b, j;
  row_bj(a, r, b, j);
  RowState* rs = &a.s.rs[r];
  if (rs->phase != PH_QRES) return;
  const int t = threadIdx.x, qr = b * a.k + j;
  const RowParams p = load_params(a, b, j);
  const float m = rs->m;
  const uint64_t S = rs->qS, R = rs->qR, T = rs->qT, below = rs->qbelow;
  const int qbin = rs->qbin, arg = rs->token;
  const int draft = a.drafts[(int64_t)b * a.k + j];
  const float l_draft = rs->l_draft;
  const XQ q = q_of_row(a, qr);
  int token = arg;
  if (qbin >= 0) {
    const int n = min((int)a.s.ncand[r], CAP);
    uint64_t kk[FIN_Q];
#pragma unroll
    for (int e = 0; e < FIN_Q; ++e) {
      const int idx = e * FIN_T + t;
      kk[e] = ~0ull;
      if (idx < n) {
        const Cand cd = a.s.cand[(int64_t)r * CAP + idx];
        kk[e] = ckey(cd.l, cd.id);
      }
    }
    sort_keys(kk, n, s_key, s_tmp);
    // residual weights in order; thread t owns positions FIN_Q t .. FIN_Q t + FIN_Q - 1
    uint64_t w[FIN_Q], lm = 0ull;
#pragma unroll
    for (int e = 0; e < FIN_Q; ++e) {
      const int pos = FIN_Q * t + e;
      w[e] = 0ull;
      if (pos < n) {
        const uint64_t key = s_key[pos];
        const int id = (int)(uint32_t)key;
        w[e] = q_resid(x_weight(fkey_desc_inv((uint32_t)(key >> 32)), m), xq_prob(q, id), S);
        lm += w[e];
      }
    }
    uint64_t ex0, exm, tot0, totm;
    block_excl_scan2_u64<FIN_T>(0ull, lm, s_u2, ex0, exm, tot0, totm);
    // the last token whose residual mass before it is <= T
    int best = -1;
    uint64_t fm = below + exm;
#pragma unroll
    for (int e = 0; e < FIN_Q; ++e) {
      const int pos = FIN_Q * t + e;
      if (pos < n) {
        if (fm <= T) best = pos;
        fm += w[e];
      }
    }
    best = -block_min<FIN_T>(-best, s_i);
    // an all-zero residual draws the row's first maximum
    if (best >= 0 && R > 0ull) token = (int)(uint32_t)s_key[best];
  }
  // accept iff u < p(d) / q(d)
  const double sig = (double)S / XFIX;
  const double w_d = l_draft > -INFINITY ? exp((double)l_draft - (double)m) : 0.0;
  double ratio = w_d / sig;
  const double qd = xq_prob(q, draft);
  ratio = qd > 0.0 ? ratio / qd : (ratio > 0.0 ? INFINITY : 0.0);
  const float ua = row_uniform(a, r, p, 1);
  const int acc = ((double)ua < ratio) ? 1 : 0;
  if (t == 0) {
    rs->status = STRIM_OK;
    rs->token = token;
    rs->accept = acc;
    rs->sum_kept = sig;
    rs->last_key = ~0ull;
    rs->phase = PH_DONE;
  }
}

// (score, id) argmax, larger score first, then the smaller id; id < 0 is empty.
__device__ __forceinline__ void q_take(double& a, int& ai, double b, int bi) {
  if (bi >= 0 && (ai < 0 || b > a || (b == a && bi < ai))) {
    a = b;
    ai = bi;
  }
}
__device__ __forceinline__ void q_wave_best(double& sc, int& id) {
#define STRIM_Q_STEP(C) q_take(sc, id, dpp_d<C>(sc), dpp_i<C>(id))
  STRIM_Q_STEP(DPP_XOR1);
  STRIM_Q_STEP(DPP_XOR2);
  STRIM_Q_STEP(DPP_HALF_MIRROR);
  STRIM_Q_STEP(DPP_MIRROR);
#undef STRIM_Q_STEP
  double bs = rl_d(sc, 0);
  int bi = rl_i(id, 0);
  q_take(bs, bi, rl_d(sc, 16), rl_i(id, 16));
  q_take(bs, bi, rl_d(sc, 32), rl_i(id, 32));
  q_take(bs, bi, rl_d(sc, 48), rl_i(id, 48));
  sc = bs;
  id = bi;
}

// The residual draws of sequence b and its accept chain, in the last k_qgumbel workgroup
// of the sequence to finish: wave w takes draft rows j = w, w + NW, ... (those in phase
// QRES) and reduces their chunks' results; with COMBINE (no later kernel decides rows of
// the call) the sequence's accept chain follows, reading the picked rows from LDS.
template <bool COMBINE, int NW>
__device__ __forceinline__ void qg_pick(const Args& a, int b, RowOut* s_out, int* s_mine,
                                        const double* s_sig, bool pre, int jq) {
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  const int k1 = a.k + 1;
  // the chunks' best of draft row j: its token (the row's first maximum when nothing
  // scores), and the row's plain mass sum over the chunks when sp is asked for
  auto best = [&](int j, uint64_t* sp_out) -> int {
    const int qr = b * a.k + j;
    uint64_t sp = 0ull;
    double bsc = -INFINITY;
    int bid = -1;
    for (int c = lane; c < a.W; c += WAVE) {
      if (sp_out) sp += a.s.qpart[(size_t)qr * a.s.wmax + c];
      const size_t o = ((size_t)qr * a.s.wmax + c) * QNB;
      q_take(bsc, bid, __longlong_as_double((long long)a.s.qhm[o]), (int)a.s.qhc[o]);
    }
    q_wave_best(bsc, bid);
    if (sp_out) *sp_out = wave_sum_u64(sp);
    return bid;
  };
  auto done = [&](int j, int token, int acc, double sig) {
    RowState* rs = &a.s.rs[b * k1 + j];
    rs->status = STRIM_OK;
    rs->token = token;
    rs->accept = acc;
    rs->sum_kept = sig;
    rs->last_key = ~0ull;
    rs->phase = PH_DONE;
    s_out[j] = RowOut{STRIM_OK, acc, token};
  };
  if (pre) {
    // qskip: the routing loaded every row's outcome into s_out and each draft row's mass
    // into s_sig; only row jq (the first rejection) draws, and k_finalize took its accept
    // test (not accepted) and kept its mass
    if (jq >= 0 && w == 0) {
      const int bid = best(jq, nullptr);
      if (lane == 0) done(jq, bid >= 0 ? bid : s_out[jq].token, 0, s_sig[jq]);
    }
  } else {
    // every draft row's state in one load, one lane a row (k <= 64): with qskip only the
    // first rejected row takes its draw (q_needed)
    int st = STRIM_OK, ac = 1, ph = PH_DONE;
    if (lane < a.k) {
      const RowState& rq = a.s.rs[(int64_t)b * k1 + lane];
      st = rq.status;
      ac = rq.accept;
      ph = rq.phase;
    }
    const uint64_t m_rej = __ballot(!(st == STRIM_OK && ac));
    const int first_rej = m_rej ? (int)__ffsll((long long)m_rej) - 1 : WAVE;
    for (int j = w; j < a.k; j += NW) {
      const int r = b * k1 + j;
      RowState* rs = &a.s.rs[r];
      const bool mine =
          __builtin_amdgcn_readlane(ph, j) == PH_QRES && (!a.qskip || j == first_rej);
      if (lane == 0) s_mine[j] = mine ? 1 : 0;
      if (!mine) continue;
      const int qr = b * a.k + j;
      int acc;
      double sig;
      uint64_t S = 0ull;
      const int bid = best(j, a.qskip ? nullptr : &S);
      if (a.qskip) {
        // k_finalize took the accept test (a first rejection: not accepted) and kept the
        // row's mass
        acc = rs->accept;
        sig = rs->sum_kept;
      } else {
        const RowParams p = load_params(a, b, j);
        const float m = rs->m;
        const int draft = a.drafts[(int64_t)b * a.k + j];
        const float l_draft = rs->l_draft;
        const XQ q = q_of_row(a, qr);
        sig = (double)S / XFIX;
        const double w_d = l_draft > -INFINITY ? exp((double)l_draft - (double)m) : 0.0;
        double ratio = w_d / sig;
        const double qd = xq_prob(q, draft);
        ratio = qd > 0.0 ? ratio / qd : (ratio > 0.0 ? INFINITY : 0.0);
        const float ua = row_uniform(a, r, p, (int64_t)a.V);
        acc = ((double)ua < ratio) ? 1 : 0;
      }
      if (lane == 0) done(j, bid >= 0 ? bid : rs->token, acc, sig);
    }
  }
  if constexpr (COMBINE) {
    __syncthreads();
    if (t == 0)
      verify_combine_one(a, b, [&](int j) {
        if (pre || (j < a.k && s_mine[j])) return s_out[j];
        const RowState& rs = a.s.rs[(int64_t)b * k1 + j];
        return RowOut{rs.status, rs.accept, rs.token};
      });
  }
}

// One chunk of a residual draw: the chunk's best (score, id) of row r = (b, j).
__device__ __forceinline__ void qg_chunk(const Args& a, int r, int b, int j, int c,
                                         uint32_t* s_cnt, uint64_t* s_red, double* s_sc,
                                         int* s_id) {
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  const int qr = b * a.k + j;
  const RowParams p = load_params(a, b, j);
  const float m = a.s.rs[r].m;
  const uint64_t sp = t < a.W ? a.s.qpart[(size_t)qr * a.s.wmax + t] : 0ull;
  float l[EPT];
  q_tokens(a, r, b, j, p, c, s_cnt, l);
  const uint64_t S = block_sum_u64<TPB>(sp, s_red);
  const double lse = log((double)S / XFIX);
  const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
  const uint64_t pkey = mix64(p.seed, p.position);
  const XQ q = q_of_row(a, qr);
  const int i0 = c * CHUNK + t * EPT;
  // the thread's 8 uniforms (two Philox blocks: i0 is a multiple of 8) and its table
  // membership bits (one 32-id word)
  float u[EPT];
  if (a.noise) {
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      u[e] = a.noise[(int64_t)r * a.noise_stride + (i0 + e < a.V ? i0 + e : 0)];
  } else {
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const uint4 wb = philox_block(pkey, (uint64_t)((i0 >> 2) + hb));
      u[4 * hb] = u01(wb.x); u[4 * hb + 1] = u01(wb.y);
      u[4 * hb + 2] = u01(wb.z); u[4 * hb + 3] = u01(wb.w);
    }
  }
  const uint32_t qword = q.dbits[(i0 < a.V ? i0 : 0) >> 5];
  const uint32_t qbits = qword >> (i0 & 31);
  // fp32 screen: an upper bound ub of every token's score (log(p - q) <= log p, so a
  // table token's p-score bounds its residual score) and, from the tokens outside the
  // table (whose score is the p-score), a lower bound lb of the wave's best. Only tokens
  // with ub >= the wave's largest lb can be the best; they alone are scored exactly in
  // fp64, with the same arithmetic and tie rule as every token was before. The margin
  // covers the fp32 rounding of l - m - lse and the proxy transform's error (at most
  // 2e-6; well below 1e-4 in all at these magnitudes).
  const float mf = m, lsef = (float)lse;
  float ub[EPT];
  float lbw = -INFINITY;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    ub[e] = -INFINITY;
    if (!(l[e] > -INFINITY)) continue;
    const float bf = no_lse ? l[e] : (l[e] - mf) - lsef;
    const float sf = bf + gumbel32(u[e]);
    const float mg = 1e-3f + 1e-5f * fabsf(sf);
    ub[e] = sf + mg;
    if (!((qbits >> e) & 1u)) lbw = fmaxf(lbw, sf - mg);
  }
  lbw = wave_max_f(lbw);
  double bsc = -INFINITY;
  int bid = -1;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (!(l[e] > -INFINITY) || !(ub[e] >= lbw)) continue;
    const int id = i0 + e;
    double base = no_lse ? (double)l[e] : ((double)l[e] - (double)m) - lse;
    if ((qbits >> e) & 1u) {
      const double qq = exp((double)xq_v(q, id, qword, q.wrank[id >> 5]) - (double)q.mq) / q.Z;
      if (qq != 0.0) {
        // residual score: log(p - q), excluded where p <= q
        const double rr = exp(base) - qq;
        if (!(rr > 0.0)) continue;
        base = log(rr);
      }
    }
    q_take(bsc, bid, base + gumbel64(u[e]), id);
  }
  q_wave_best(bsc, bid);
  if (lane == 0) {
    s_sc[w] = bsc;
    s_id[w] = bid;
  }
  __syncthreads();
  if (t == 0) {
#pragma unroll
    for (int k = 1; k < TPB / WAVE; ++k) q_take(bsc, bid, s_sc[k], s_id[k]);
    const size_t o = ((size_t)qr * a.s.wmax + c) * QNB;
    a.s.qhm[o] = (unsigned long long)__double_as_longlong(bsc);
    a.s.qhc[o] = (uint32_t)bid;
  }
}

// Grid (W, R), or with a.qskip (W, B): workgroup (c, b) takes chunk c of sequence b's
// first rejected draft row (the only residual draw read), found from the rows' accept
// outcomes in one wave load (k <= 64). Every workgroup, with a chunk to score or not,
// then counts itself in the sequence's arrival counter (after a device-scope fence that
// publishes its result); the last of the sequence's workgroups to arrive resets the
// counter and runs the sequence's pick (qg_pick), so no further launch waits for them.
template <bool COMBINE>
__global__ __launch_bounds__(TPB) void k_qgumbel(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  __shared__ uint64_t s_red[TPB / WAVE];
  __shared__ double s_sc[TPB / WAVE];
  __shared__ int s_id[TPB / WAVE];
  __shared__ RowOut s_out[MAXP];
  __shared__ int s_mine[MAXP];
  __shared__ double s_sig[MAXP];
  __shared__ int s_last;
  const int t = threadIdx.x, lane = t & (WAVE - 1);
  int r = 0, c, b, j = 0;
  bool work = true;  // (uniform over the workgroup)
  const bool pre = a.qskip && a.k < WAVE;  // the rows' outcomes kept from the routing load
  if (a.qskip) {
    b = blockIdx.y;
    c = blockIdx.x;
    const int k1 = a.k + 1;
    bool rej = false;
    int ph = -1;
    if (lane <= a.k) {
      const RowState& rq = a.s.rs[(int64_t)b * k1 + lane];
      const int st = rq.status, ac = rq.accept, tk = rq.token;
      if (lane < a.k) {
        rej = !(st == STRIM_OK && ac);
        ph = rq.phase;
      }
      if (pre && t < WAVE) {  // (wave 0; for the last arriver's pick)
        s_out[lane] = RowOut{st, ac, tk};
        if (lane < a.k) s_sig[lane] = rq.sum_kept;
      }
    }
    const uint64_t m_rej = __ballot(rej);
    if (m_rej == 0ull) {
      work = false;  // every draft accepted: no residual draw
    } else {
      j = (int)__ffsll((long long)m_rej) - 1;
      if (__builtin_amdgcn_readlane(ph, j) != PH_QRES) work = false;
      r = b * k1 + j;
    }
  } else {
    map_block(a, r, c);
    row_bj(a, r, b, j);
    if (uniform_copy(a.s.rs[r].phase) != PH_QRES) work = false;
  }
  if (work) qg_chunk(a, r, b, j, c, s_cnt, s_red, s_sc, s_id);
  // arrival: every workgroup of the sequence (W of them, or W (k + 1) without qskip)
  if (t == 0) {
    __threadfence();  // (this workgroup's result is visible before its count)
    const uint32_t expect = (uint32_t)(a.qskip ? a.W : a.W * (a.k + 1));
    const uint32_t old = atomicAdd(&a.s.qarr[b], 1u);
    const bool last = old + 1u == expect;
    if (last) a.s.qarr[b] = 0u;  // every workgroup has counted: ready for the next launch
    s_last = last ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();  // (the other workgroups' results are read after their counts)
  qg_pick<COMBINE, TPB / WAVE>(a, b, s_out, s_mine, s_sig, pre, pre && work ? j : -1);
}

hipError_t launch_qgumbel(const Args& a, bool combine, dim3 grid, hipStream_t st, hipEvent_t e0,
                          hipEvent_t e1) {
  return combine ? launch_args((const void*)k_qgumbel<true>, grid, dim3(TPB), a, st, e0, e1)
                 : launch_args((const void*)k_qgumbel<false>, grid, dim3(TPB), a, st, e0, e1);
}

}  // namespace strim
