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
  xa.q = q_of_row(a, qr);
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


}  // namespace strim
