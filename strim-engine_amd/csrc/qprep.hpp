// qprep.hpp — the general-q verify inputs, one block function for NT-thread workgroups:
// run by k_qprep (sample_kernels.hip) as a launch of its own, or by k_stream as extra
// workgroups of its own launch (rows past R of its grid): the two are independent and
// k_finalize reads both, so one launch saves a dependent launch and overlaps them.
#pragma once

#include "select.hpp"

namespace strim {

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

// NT-thread workgroups. Blocks [0, B*k*QSPLIT): slice sp of draft row qr (blk = qr *
// QSPLIT + sp, 1/QSPLIT of the table each): the slice maximum of v = draft_logit / T
// (fp32 division, as the target's temperature), the slice's sum of exp(v - max) in fp64
// and the table index of the row's draft token if the slice holds it (the draft
// distribution of SpecSampling's general-q extension; its readers take v at a member id
// from the draft logits through the id's table index); row 0's slices also check that
// the table is strictly ascending inside [0, V). Each draft row's k_finalize workgroup
// merges the row's slices. Blocks after them: one thread per table entry builds the
// membership bitmap and the rank words: the first entry of each 32-id word writes the
// word's bits and its table index, and the same index with no bits into the empty words
// before it (the last entry also Vd into those after it), so every word is written once.
template <int NT>
__device__ __forceinline__ void qprep_block(const Args& a, int blk) {
  __shared__ float s_m[NT / WAVE];
  __shared__ double s_d[NT / WAVE];
  __shared__ int s_bad[NT / WAVE];
  const int t = threadIdx.x;
  const int nq = a.B * a.k, Vd = a.Vd;
  if (blk < nq * QSPLIT) {
    // slice sp of draft row qr: table entries [lo, hi)
    const int qr = blk / QSPLIT, sp = blk - qr * QSPLIT;
    const int span = (Vd + QSPLIT - 1) / QSPLIT;
    const int lo = min(Vd, sp * span), hi = min(Vd, lo + span);
    const int b = qr / a.k, j = qr % a.k;
    const int d = a.drafts[(int64_t)b * a.k + j];
    const float T = a.p[b].temperature;
    const size_t base = (size_t)qr * (size_t)Vd;
    auto ld = [&](int i) -> float {
      return a.dtype == STRIM_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)a.dlog)[base + i])
                                         : ((const float*)a.dlog)[base + i];
    };
    // batches of QB entries per thread, every load of a batch issued before any wait.
    // One pass: the table check (row 0), the draft's table index and the maximum of
    // v = logit / T.
    constexpr int QB = 4;
    const bool live = T > 0.0f;
    float mx = -INFINITY;
    int bad = 0, td = -1;
    for (int i0 = lo + t; i0 < hi; i0 += QB * NT) {
      float v[QB];
      int id[QB], idn[QB];
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        const int i = i0 + q * NT < hi ? i0 + q * NT : lo;
        v[q] = ld(i);
        id[q] = a.dtable[i];
        idn[q] = a.dtable[i + 1 < Vd ? i + 1 : i];
      }
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        const int i = i0 + q * NT;
        if (i >= hi) continue;
        if (id[q] < 0 || id[q] >= a.V || (i + 1 < Vd && !(id[q] < idn[q]))) bad = 1;
        if (id[q] == d) td = i;
        if (live) mx = fmaxf(mx, v[q] / T);
      }
    }
    if (qr == 0) bad = block_or<NT>(bad, s_bad);
    td = -block_min<NT>(-td, s_bad);  // at most one entry holds the draft
    QPart q{-INFINITY, td, 0.0, bad, 0};
    if (live) {
      mx = wave_max_f(mx);
      if ((t & (WAVE - 1)) == 0) s_m[t / WAVE] = mx;
      __syncthreads();
      mx = s_m[0];
#pragma unroll
      for (int w = 1; w < NT / WAVE; ++w) mx = fmaxf(mx, s_m[w]);
      double z = 0.0;
      for (int i0 = lo + t; i0 < hi; i0 += QB * NT) {
        float v[QB];
#pragma unroll
        for (int w = 0; w < QB; ++w) v[w] = ld(i0 + w * NT < hi ? i0 + w * NT : lo);
#pragma unroll
        for (int w = 0; w < QB; ++w)
          if (i0 + w * NT < hi) z += exp((double)(v[w] / T) - (double)mx);
      }
      z = block_sum_f64<NT>(z, s_d);
      q.m = mx;
      q.z = z;
    }
    if (t == 0) a.s.qpp[blk] = q;
    return;
  }
  const int i = (blk - nq * QSPLIT) * NT + t;
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
  a.s.wrank[w] = (uint32_t)i;
  for (int z = max(pw + 1, 0); z < w; ++z) {
    a.s.dbits[z] = 0u;
    a.s.wrank[z] = (uint32_t)i;
  }
  if (i == Vd - 1)
    for (int z = w + 1; z < words; ++z) {
      a.s.dbits[z] = 0u;
      a.s.wrank[z] = (uint32_t)Vd;
    }
}

}  // namespace strim
