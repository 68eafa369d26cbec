// sample_kernels.hip — k_final (the exact resolution of general-q verify rows), the
// validation output (k_probs), the verify combine and the general-q preparation
// (k_qprep).
#include "exact.hpp"

namespace strim {

// ---------------------------------------------------------------------------------
// k_final: the general-q verify rows k_finalize left in phase EXACT (a filter, or an icdf
// residual bin too wide for the grid-wide draw), on the exact streaming resolution with
// the draft distribution q; every other row is already decided.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(FIN_T) void k_final(Args a) {
  __shared__ uint64_t s_key[CAP];
  __shared__ uint32_t s_cnt[FIN_T * EPT];
  __shared__ double s_dred[FIN_T / WAVE];
  __shared__ uint64_t s_ured[FIN_T / WAVE];
  __shared__ int s_ired[FIN_T / WAVE];
  __shared__ uint64_t s_u2[2 * FIN_T / WAVE];
  __shared__ XState s_x;
  static_assert(CAP >= XB + XB / 2, "the exact path's keys and bin counts share s_key");

  const int r = blockIdx.x;
  int b, j;
  row_bj(a, r, b, j);
  RowState* rsp = &a.s.rs[r];
  if (rsp->phase != PH_EXACT) return;
  const RowParams p = load_params(a, b, j);
  // k_finalize has checked the row (status, draft, table) and left its maximum and first
  // argmax
  const float m = rsp->m;
  const int arg = rsp->token;
  const int draft = a.drafts[(int64_t)b * a.k + j];
  // ---- exact streaming resolution ---------------------------------------------------
  const XScratch xs = xscratch(s_key, (uint32_t*)(s_key + XB), s_cnt, s_u2, s_dred, s_ured, s_ired);
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
  xa.has_q = 1;
  // the draft distribution q of the row (k_qprep)
  const int qr = b * a.k + j;
  const QStat qs = a.s.qst[qr];
  xa.q.dbits = a.s.dbits;
  xa.q.vq = a.s.vq + (size_t)qr * (size_t)a.s.wmax * CHUNK;
  xa.q.mq = qs.mq;
  xa.q.Z = qs.Z;
  const XOut xo = exact_row<FIN_T, true>(xa, r, b, j, p, m, arg, draft, true, rsp->l_draft, xs,
                                   *(lds_t<XState>*)&s_x);
  if (threadIdx.x == 0) {
    rsp->status = xo.status;
    rsp->token = xo.token;
    rsp->accept = xo.accept;
    rsp->sum_kept = xo.sig;
    rsp->last_key = xo.last_key;
    rsp->phase = PH_DONE;
  }
}

// ---------------------------------------------------------------------------------
// k_probs: processed distribution (validation output)
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(TPB) void k_probs(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  int r, c;
  map_block(a, r, c);
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
  for (int e = 0; e < EPT; ++e) {
    const int i = i0 + e;
    if (i >= a.V) break;
    float pv = 0.0f;
    if (l[e] > -INFINITY) {
      // the kept set is a prefix of the (l desc, id asc) order, up to last_key
      const bool kept = rs.last_key != 0ull && ckey(l[e], i) <= rs.last_key;
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
  verify_combine_one(a, b, [&](int j) {
    const RowState& rs = a.s.rs[(int64_t)b * (a.k + 1) + j];
    return RowOut{rs.status, rs.accept, rs.token};
  });
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
// [0, V). Each draft row's k_finalize workgroup merges the row's slices. Blocks after them: one thread per table entry
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

}  // namespace strim
