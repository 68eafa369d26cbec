// sample_kernels.hip — the four passes of one token-selection call on gfx950.
//
//   k_stats   (rows x chunks) processed logits -> chunk max / argmax / allowed count;
//             the row's last workgroup merges them (row max m, greedy result, status).
//   k_hist    (rows x chunks) histogram of d = m - l over NBINS bins: counts and
//             fixed-point masses exp(-d) * 2^40, merged with integer atomics (exact,
//             order-independent). The last workgroup turns the histogram into bin-level
//             bounds for min-p / top-k / top-p / the icdf draw, and picks the bins whose
//             tokens must be resolved exactly.
//   k_collect (rows x chunks) appends the tokens of those bins to the row's candidate
//             buffer and keeps, per chunk, the two best surely-kept tokens by the fp32
//             Gumbel proxy (used when the kept set is too large to collect).
//   k_final   (one 1024-thread workgroup per row) sorts the candidates in LDS by
//             (l desc, id asc) and resolves every decision in fp64, then draws.
// No pass waits on another workgroup: the merges use the last-arriving workgroup.
#include "kernels.hpp"

namespace strim {

// ---------------------------------------------------------------------------------
// k_stats
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(TPB) void k_stats(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  __shared__ float s_v[TPB / WAVE];
  __shared__ int s_i[TPB / WAVE];
  __shared__ int s_n[TPB / WAVE];
  __shared__ int s_f[TPB / WAVE];
  __shared__ int s_last;

  int r, c;
  map_block(a, blockIdx.x, r, c);
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  const int c0 = c * CHUNK;
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;

  if (p.valid && p.pen) build_counts(a, b, j, c0, s_cnt);
  float l[EPT];
  bool nf = false;
  process_tokens(a, r, c0, p, s_cnt, l, nf);

  float mv = -INFINITY;
  int mi = -1, n = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e)
    if (l[e] > -INFINITY) {
      ++n;
      argmax_merge(mv, mi, l[e], c0 + t * EPT + e);
    }
  // verify: the draft token's processed logit
  if (a.verify && j < a.k) {
    const int d = a.drafts[(int64_t)b * a.k + j];
    const int o = d - (c0 + t * EPT);
    if (o >= 0 && o < EPT) {
      float ld = -INFINITY;
#pragma unroll
      for (int e = 0; e < EPT; ++e)
        if (e == o) ld = l[e];
      a.s.rs[r].l_draft = ld;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float v2 = __shfl_xor(mv, o, WAVE);
    int i2 = __shfl_xor(mi, o, WAVE);
    argmax_merge(mv, mi, v2, i2);
  }
  n = wave_sum(n);
  int f = __any(nf) ? 1 : 0;
  if (lane == 0) {
    s_v[w] = mv;
    s_i[w] = mi;
    s_n[w] = n;
    s_f[w] = f;
  }
  // zero this chunk's slice of the row histogram for k_hist
  {
    const int slice = (NBINS + a.W - 1) / a.W;
    const int lo = c * slice, hi = min(NBINS, lo + slice);
    for (int i = lo + t; i < hi; i += TPB) {
      a.s.hcnt[(int64_t)r * NBINS + i] = 0u;
      a.s.hmass[(int64_t)r * NBINS + i] = 0ull;
    }
  }
  __syncthreads();
  if (t == 0) {
    float bv = s_v[0];
    int bi = s_i[0], bn = s_n[0], bf = s_f[0];
    for (int i = 1; i < TPB / WAVE; ++i) {
      argmax_merge(bv, bi, s_v[i], s_i[i]);
      bn += s_n[i];
      bf |= s_f[i];
    }
    a.s.cstat[(int64_t)r * a.s.wmax + c] = ChunkStat{bv, bi, bn, bf};
    __threadfence();
    unsigned prev = atomicAdd(&a.s.cnt_stats[r], 1u);
    s_last = (prev == (unsigned)(a.W - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // ---- last workgroup of row r: merge the chunk statistics -----------------------
  float bv = -INFINITY;
  int bi = -1, bn = 0, bf = 0;
  for (int cc = t; cc < a.W; cc += TPB) {
    ChunkStat cs = a.s.cstat[(int64_t)r * a.s.wmax + cc];
    argmax_merge(bv, bi, cs.m, cs.arg);
    bn += cs.n;
    bf |= cs.flags;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float v2 = __shfl_xor(bv, o, WAVE);
    int i2 = __shfl_xor(bi, o, WAVE);
    argmax_merge(bv, bi, v2, i2);
    bn += __shfl_xor(bn, o, WAVE);
    bf |= __shfl_xor(bf, o, WAVE);
  }
  __syncthreads();
  if (lane == 0) {
    s_v[w] = bv;
    s_i[w] = bi;
    s_n[w] = bn;
    s_f[w] = bf;
  }
  __syncthreads();
  if (t == 0) {
    for (int i = 1; i < TPB / WAVE; ++i) {
      argmax_merge(s_v[0], s_i[0], s_v[i], s_i[i]);
      s_n[0] += s_n[i];
      s_f[0] |= s_f[i];
    }
    int status = STRIM_OK;
    int draft = -1;
    if (a.verify && j < a.k) {
      draft = a.drafts[(int64_t)b * a.k + j];
      if (draft < 0 || draft >= a.V) status = STRIM_EINVAL;
    }
    if (!p.valid) status = STRIM_EINVAL;
    else if (s_f[0]) status = STRIM_ENONFINITE;
    else if (s_n[0] == 0) status = STRIM_EEMPTY;
    RowState& rs = a.s.rs[r];
    rs.m = s_v[0];
    rs.status = status;
    rs.n_allowed = s_n[0];
    rs.argmax = s_i[0];
    rs.greedy = p.greedy ? 1 : 0;
    rs.mode = MODE_NONE;
    rs.draft = draft;
    rs.token = -1;
    rs.accept = 0;
    rs.sum_kept = 0.0;
    rs.last_key = 0ull;
    if (!a.verify) {
      if (status != STRIM_OK) {
        a.out_ids[r] = -1;
        if (a.out_status) a.out_status[r] = status;
      } else if (p.greedy) {
        a.out_ids[r] = s_i[0];
        if (a.out_status) a.out_status[r] = STRIM_OK;
      }
    }
    if (p.greedy) rs.token = s_i[0];
    a.s.cnt_stats[r] = 0u;
  }
}

// ---------------------------------------------------------------------------------
// k_hist
// ---------------------------------------------------------------------------------
__device__ __forceinline__ bool in_ranges(const RowState& rs, int bin) {
  return (bin >= rs.rng[0][0] && bin <= rs.rng[0][1]) ||
         (bin >= rs.rng[1][0] && bin <= rs.rng[1][1]) ||
         (bin >= rs.rng[2][0] && bin <= rs.rng[2][1]);
}

// First bin b in [lo, hi] with pred(b) true, for a monotone predicate; hi + 1 if none.
template <typename F>
__device__ __forceinline__ int first_true(int lo, int hi, F pred) {
  int L = lo, H = hi + 1;
  while (L < H) {
    int mid = (L + H) >> 1;
    if (pred(mid)) H = mid;
    else L = mid + 1;
  }
  return L;
}

__device__ __forceinline__ float row_uniform(const Args& a, int r, const RowParams& p,
                                             int64_t idx) {
  if (a.noise) return a.noise[(int64_t)r * a.noise_stride + idx];
  return philox_uniform(mix64(p.seed, p.position), (uint64_t)idx);
}

__global__ __launch_bounds__(TPB) void k_hist(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  __shared__ uint32_t s_hc[NBINS];
  __shared__ unsigned long long s_hm[NBINS];
  __shared__ uint64_t s_red[TPB / WAVE];
  __shared__ int s_last;

  int r, c;
  map_block(a, blockIdx.x, r, c);
  const RowState* rsp = &a.s.rs[r];
  if (rsp->status != STRIM_OK || rsp->greedy) return;  // uniform over the row
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  const int c0 = c * CHUNK;
  const int t = threadIdx.x;
  const float m = rsp->m;

  for (int i = t; i < NBINS; i += TPB) {
    s_hc[i] = 0u;
    s_hm[i] = 0ull;
  }
  if (p.pen) build_counts(a, b, j, c0, s_cnt);
  else __syncthreads();
  float l[EPT];
  bool nf = false;
  process_tokens(a, r, c0, p, s_cnt, l, nf);
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (!(l[e] > -INFINITY)) continue;
    const float d = m - l[e];
    const int bin = dbin(d);
    const unsigned long long fix = __float2ull_rn(expf(-d) * FIX_SCALE_F);
    atomicAdd(&s_hc[bin], 1u);
    if (fix) atomicAdd(&s_hm[bin], fix);
  }
  __syncthreads();
  for (int i = t; i < NBINS; i += TPB) {
    const uint32_t cn = s_hc[i];
    if (cn) {
      atomicAdd(&a.s.hcnt[(int64_t)r * NBINS + i], cn);
      const unsigned long long ms = s_hm[i];
      if (ms) atomicAdd(&a.s.hmass[(int64_t)r * NBINS + i], ms);
    }
  }
  __threadfence();
  __syncthreads();
  if (t == 0) {
    unsigned prev = atomicAdd(&a.s.cnt_hist[r], 1u);
    s_last = (prev == (unsigned)(a.W - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // ---- last workgroup: inclusive cumulative counts C[b] and masses M[b] -----------
  constexpr int BPT = NBINS / TPB;  // bins per thread
  uint32_t lc[BPT];
  unsigned long long lm[BPT];
  uint32_t sc = 0;
  unsigned long long sm = 0;
#pragma unroll
  for (int q = 0; q < BPT; ++q) {
    const int bi = t * BPT + q;
    lc[q] = __hip_atomic_load(&a.s.hcnt[(int64_t)r * NBINS + bi], __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    lm[q] = __hip_atomic_load(&a.s.hmass[(int64_t)r * NBINS + bi], __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    sc += lc[q];
    sm += lm[q];
  }
  uint64_t tot_m;
  const uint64_t base_m = block_excl_scan_u64<TPB>((uint64_t)sm, s_red, &tot_m);
  uint64_t tot_c64;
  const uint64_t base_c64 = block_excl_scan_u64<TPB>((uint64_t)sc, s_red, &tot_c64);
  {
    uint32_t cc = (uint32_t)base_c64;
    unsigned long long mm = base_m;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      cc += lc[q];
      mm += lm[q];
      s_hc[t * BPT + q] = cc;  // inclusive cumulative count
      s_hm[t * BPT + q] = mm;  // inclusive cumulative mass
    }
  }
  __syncthreads();
  if (t != 0) return;

  RowState& rs = a.s.rs[r];
  const int V = a.V;
  const uint32_t N = s_hc[NBINS - 1];
  const double inv = 1.0 / FIX_SCALE;
  const double EPS = 1e-5;
  const double SLACK = ((double)N + 2.0) * 2.0 * inv;
  auto Mb = [&](int bb) -> double { return bb < 0 ? 0.0 : (double)s_hm[bb] * inv; };
  auto Cb = [&](int bb) -> uint32_t { return bb < 0 ? 0u : s_hc[bb]; };

  // pre-kept bounds (min-p and top-k): bins < s1 surely pass, bins > e1 surely fail
  int s1 = NBINS, e1 = NBINS - 1;
  if (p.min_p > 0.0f) {
    const double thr = -log((double)p.min_p);
    const int bt = thr < 63.0 ? (int)(thr * (double)BIN_SCALE) : NBINS - 1;
    s1 = min(s1, max(0, bt - 1));
    e1 = min(e1, min(NBINS - 1, bt + 1));
  }
  const bool topk = p.top_k > 0 && p.top_k < V;
  if (topk && N > (uint32_t)p.top_k) {
    const uint32_t K = (uint32_t)p.top_k;
    const int bk = first_true(0, NBINS - 1, [&](int bb) { return s_hc[bb] >= K; });
    s1 = min(s1, bk);
    e1 = min(e1, bk);
  }
  // top-p bounds
  int s = s1, e = e1;
  const bool topp = p.top_p < 1.0f;
  if (topp) {
    const double P = (double)p.top_p;
    const double sig_hi = Mb(e1) * (1.0 + EPS) + SLACK;
    const double sig_lo = Mb(s1 - 1) * (1.0 - EPS) - SLACK;
    const int lim = min(e1, s1 - 1);
    int ep = e1;
    if (lim >= 0) {
      const int f = first_true(0, lim, [&](int bb) { return Mb(bb) * (1.0 - EPS) - SLACK > P * sig_hi; });
      if (f <= lim) ep = f;
    }
    // bins < sp surely kept: M[b](1+eps)+slack <= P * sig_lo
    const int sp = first_true(0, NBINS - 1, [&](int bb) { return Mb(bb) * (1.0 + EPS) + SLACK > P * sig_lo; });
    e = min(e1, ep);
    s = min(s1, sp);
  }
  if (s > e + 1) s = e + 1;
  const bool icdf = a.noise_mode == STRIM_NOISE_ICDF;
  const bool by_rank = (p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp;
  int mode;
  int rng[3][2] = {{1, 0}, {1, 0}, {1, 0}};
  if (Cb(e1) <= (uint32_t)CAP) {
    mode = MODE_A;  // every possibly pre-kept token is collected: all decisions exact
    rng[0][0] = 0;
    rng[0][1] = e1;
    s = 0;
  } else if (by_rank) {
    mode = MODE_NONE;  // rank-indexed noise needs the whole kept set in order
  } else {
    mode = MODE_B;
    rng[0][0] = s;
    rng[0][1] = e;
    if (s1 <= e1) {
      rng[1][0] = s1;
      rng[1][1] = e1;
    }
    if (icdf) {
      const double u = (double)row_uniform(a, r, p, 0);
      double wd = 0.0;
      if (a.verify && rs.draft >= 0 && rs.l_draft > -INFINITY)
        wd = exp((double)rs.l_draft - (double)m);
      const double klo = Mb(s - 1) * (1.0 - EPS) - SLACK;
      const double khi = Mb(e) * (1.0 + EPS) + SLACK;
      const double tlo = u * (klo - wd) - SLACK;
      const double thi = u * khi + wd + SLACK;
      const int dlo = first_true(0, NBINS - 1, [&](int bb) { return Mb(bb) * (1.0 + EPS) + SLACK > tlo; });
      int dhi = first_true(0, NBINS - 1, [&](int bb) { return Mb(bb) * (1.0 - EPS) - SLACK > thi; });
      dhi = min(dhi, e);
      rng[2][0] = dlo;
      rng[2][1] = dhi;
    }
    uint32_t total = 0;
    // union size of the (possibly overlapping) ranges, bin by bin (<= NBINS steps)
    int lo = NBINS, hi = -1;
    for (int q = 0; q < 3; ++q)
      if (rng[q][0] <= rng[q][1]) {
        lo = min(lo, rng[q][0]);
        hi = max(hi, rng[q][1]);
      }
    for (int bb = lo; bb <= hi; ++bb) {
      bool in = false;
      for (int q = 0; q < 3; ++q) in |= (bb >= rng[q][0] && bb <= rng[q][1]);
      if (in) total += Cb(bb) - Cb(bb - 1);
    }
    if (total > (uint32_t)CAP) mode = MODE_NONE;
  }
  if (mode == MODE_NONE) {
    rs.status = STRIM_ECAPACITY;
    if (!a.verify) {
      a.out_ids[r] = -1;
      if (a.out_status) a.out_status[r] = STRIM_ECAPACITY;
    }
  }
  rs.mode = mode;
  rs.s = s;
  rs.e = e;
  rs.s1 = s1;
  for (int q = 0; q < 3; ++q) {
    rs.rng[q][0] = rng[q][0];
    rs.rng[q][1] = rng[q][1];
  }
  a.s.ncand[r] = 0u;
  a.s.cnt_hist[r] = 0u;
}

// ---------------------------------------------------------------------------------
// k_collect
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void top2_merge(float& s0, float& l0, int& i0, float& s1, float& l1,
                                           int& i1, float t0, float tl0, int ti0, float t1,
                                           float tl1, int ti1) {
  // merge (t0, t1) into the sorted pair (s0 >= s1); ids break ties (smaller first)
  auto better = [](float a, int ia, float b, int ib) {
    return ib < 0 || (ia >= 0 && (a > b || (a == b && ia < ib)));
  };
  float cs[4] = {s0, s1, t0, t1}, cl[4] = {l0, l1, tl0, tl1};
  int ci[4] = {i0, i1, ti0, ti1};
  int bi = 0;
  for (int q = 1; q < 4; ++q)
    if (better(cs[q], ci[q], cs[bi], ci[bi])) bi = q;
  int si = -1;
  for (int q = 0; q < 4; ++q)
    if (q != bi && (si < 0 || better(cs[q], ci[q], cs[si], ci[si]))) si = q;
  s0 = cs[bi]; l0 = cl[bi]; i0 = ci[bi];
  s1 = cs[si]; l1 = cl[si]; i1 = ci[si];
}

__global__ __launch_bounds__(TPB) void k_collect(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  __shared__ float s_s0[TPB / WAVE], s_l0[TPB / WAVE], s_s1[TPB / WAVE], s_l1[TPB / WAVE];
  __shared__ int s_i0[TPB / WAVE], s_i1[TPB / WAVE];

  int r, c;
  map_block(a, blockIdx.x, r, c);
  const RowState rs = a.s.rs[r];
  if (rs.status != STRIM_OK || rs.greedy || rs.mode == MODE_NONE) return;
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  const int c0 = c * CHUNK;
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;

  if (p.pen) build_counts(a, b, j, c0, s_cnt);
  float l[EPT];
  bool nf = false;
  process_tokens(a, r, c0, p, s_cnt, l, nf);

  const bool want_top = rs.mode == MODE_B && a.noise_mode == STRIM_NOISE_GUMBEL;
  const uint64_t key = mix64(p.seed, p.position);
  int mycnt = 0;
  uint32_t sel = 0u;
  float s0 = -INFINITY, s1 = -INFINITY, l0 = 0.f, l1 = 0.f;
  int i0 = -1, i1 = -1;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (!(l[e] > -INFINITY)) continue;
    const int bin = dbin(rs.m - l[e]);
    if (in_ranges(rs, bin)) {
      sel |= 1u << e;
      ++mycnt;
    } else if (want_top && bin < rs.s) {
      const int id = c0 + t * EPT + e;
      const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + id]
                              : philox_uniform(key, (uint64_t)id);
      const float sc = l[e] + gumbel32(u);
      top2_merge(s0, l0, i0, s1, l1, i1, sc, l[e], id, -INFINITY, 0.f, -1);
    }
  }
  // wave-aggregated append to the row's candidate buffer
  const int incl = wave_incl_scan(mycnt);
  const int tot = __shfl(incl, WAVE - 1, WAVE);
  if (tot > 0) {
    unsigned base = 0;
    if (lane == WAVE - 1) base = atomicAdd(&a.s.ncand[r], (unsigned)tot);
    base = __shfl(base, WAVE - 1, WAVE);
    unsigned pos = base + (unsigned)(incl - mycnt);
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if ((sel >> e) & 1u) {
        if (pos < (unsigned)CAP)
          a.s.cand[(int64_t)r * CAP + pos] = Cand{l[e], c0 + t * EPT + e};
        ++pos;
      }
  }
  if (want_top) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float ts0 = __shfl_xor(s0, o, WAVE), tl0 = __shfl_xor(l0, o, WAVE);
      float ts1 = __shfl_xor(s1, o, WAVE), tl1 = __shfl_xor(l1, o, WAVE);
      int ti0 = __shfl_xor(i0, o, WAVE), ti1 = __shfl_xor(i1, o, WAVE);
      top2_merge(s0, l0, i0, s1, l1, i1, ts0, tl0, ti0, ts1, tl1, ti1);
    }
    if (lane == 0) {
      s_s0[w] = s0; s_l0[w] = l0; s_i0[w] = i0;
      s_s1[w] = s1; s_l1[w] = l1; s_i1[w] = i1;
    }
    __syncthreads();
    if (t == 0) {
      for (int q = 1; q < TPB / WAVE; ++q)
        top2_merge(s0, l0, i0, s1, l1, i1, s_s0[q], s_l0[q], s_i0[q], s_s1[q], s_l1[q], s_i1[q]);
      a.s.ctop[(int64_t)r * a.s.wmax + c] = ChunkTop{l0, i0, l1, i1};
    }
  }
}

// ---------------------------------------------------------------------------------
// k_final
// ---------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  uint32_t lo = __shfl_xor((uint32_t)v, o, WAVE);
  uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, WAVE);
  return ((uint64_t)hi << 32) | lo;
}

// Bitonic sort of FIN_Q * FIN_T keys held striped in registers (element e = q*FIN_T + t).
// Only the first n2 (a power of two >= 64) elements take part; the rest are padding.
__device__ void bitonic_sort(uint64_t (&k)[FIN_Q], int n2, uint64_t* s_key) {
  const int t = threadIdx.x;
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= FIN_T) {
        const int qs = stride / FIN_T;
#pragma unroll
        for (int q = 0; q < FIN_Q; ++q) {
          const int e = q * FIN_T + t;
          const int pq = q ^ qs;
          if (pq > q) {
            const bool asc = (e & size) == 0;
            uint64_t x = k[q], y = k[pq];
            bool sw = asc ? (x > y) : (x < y);
            if (sw) { k[q] = y; k[pq] = x; }
          }
        }
      } else if (stride >= WAVE) {
#pragma unroll
        for (int q = 0; q < FIN_Q; ++q) s_key[q * FIN_T + t] = k[q];
        __syncthreads();
#pragma unroll
        for (int q = 0; q < FIN_Q; ++q) {
          const int e = q * FIN_T + t;
          const int pe = e ^ stride;
          const uint64_t o = s_key[pe];
          const bool asc = (e & size) == 0;
          const bool lower = e < pe;
          k[q] = (lower == asc) ? (k[q] < o ? k[q] : o) : (k[q] > o ? k[q] : o);
        }
        __syncthreads();
      } else {
#pragma unroll
        for (int q = 0; q < FIN_Q; ++q) {
          const int e = q * FIN_T + t;
          const uint64_t o = shfl_xor_u64(k[q], stride);
          const bool asc = (e & size) == 0;
          const bool lower = (e & stride) == 0;
          k[q] = (lower == asc) ? (k[q] < o ? k[q] : o) : (k[q] > o ? k[q] : o);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) s_key[q * FIN_T + t] = k[q];
  __syncthreads();
}

// Block argmax over (score desc, tie key asc). Returns the winner's id in *out_id.
__device__ void block_argmax_score(double sc, uint64_t tk, int id, double* s_sc, uint64_t* s_tk,
                                   int* s_id, int* out_id, double* out_sc, double* out_second) {
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
  // track best and second best score values for the margin
  double sec = -INFINITY;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    double sc2 = __shfl_xor(sc, o, WAVE);
    uint64_t tk2 = shfl_xor_u64(tk, o);
    int id2 = __shfl_xor(id, o, WAVE);
    double sec2 = __shfl_xor(sec, o, WAVE);
    bool take = id2 >= 0 && (id < 0 || sc2 > sc || (sc2 == sc && tk2 < tk));
    double lose = take ? sc : sc2;
    sec = fmax(fmax(sec, sec2), (id >= 0 && id2 >= 0) ? lose : -INFINITY);
    if (take) { sc = sc2; tk = tk2; id = id2; }
  }
  if (lane == 0) { s_sc[w] = sc; s_tk[w] = tk; s_id[w] = id; s_sc[FIN_T / WAVE + w] = sec; }
  __syncthreads();
  if (t == 0) {
    double bs = s_sc[0], bsec = s_sc[FIN_T / WAVE];
    uint64_t btk = s_tk[0];
    int bid = s_id[0];
    for (int q = 1; q < FIN_T / WAVE; ++q) {
      bsec = fmax(bsec, s_sc[FIN_T / WAVE + q]);
      if (s_id[q] < 0) continue;
      bool take = bid < 0 || s_sc[q] > bs || (s_sc[q] == bs && s_tk[q] < btk);
      if (bid >= 0) bsec = fmax(bsec, take ? bs : s_sc[q]);
      if (take) { bs = s_sc[q]; btk = s_tk[q]; bid = s_id[q]; }
    }
    *out_id = bid;
    *out_sc = bs;
    *out_second = bsec;
  }
  __syncthreads();
}

__global__ __launch_bounds__(FIN_T) void k_final(Args a) {
  __shared__ uint64_t s_key[CAP];
  __shared__ double s_P1[NBINS + 1];
  __shared__ double s_P2[NBINS + 1];
  __shared__ uint32_t s_PC[NBINS + 1];
  __shared__ double s_dred[2 * FIN_T / WAVE];
  __shared__ uint64_t s_ured[FIN_T / WAVE];
  __shared__ int s_ired[FIN_T / WAVE];
  __shared__ int s_int[4];
  __shared__ float s_kth;

  const int r = blockIdx.x;
  const RowState rs = a.s.rs[r];
  if (rs.status != STRIM_OK || rs.greedy) return;
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  const int t = threadIdx.x;
  const uint32_t nc = a.s.ncand[r];
  const int V = a.V;
  const bool verify_draft_row = a.verify && j < a.k;

  auto fail = [&](int st) {
    if (t == 0) {
      a.s.rs[r].status = st;
      if (!a.verify) {
        a.out_ids[r] = -1;
        if (a.out_status) a.out_status[r] = st;
      }
    }
  };
  if (nc > (uint32_t)CAP) {
    fail(STRIM_ECAPACITY);
    return;
  }
  const int n = (int)nc;

  // 1. candidates -> sorted keys (l desc, id asc)
  uint64_t kk[FIN_Q];
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    const int idx = q * FIN_T + t;
    if (idx < n) {
      const Cand cd = a.s.cand[(int64_t)r * CAP + idx];
      kk[q] = ckey(cd.l, cd.id);
    } else {
      kk[q] = ~0ull;
    }
  }
  int n2 = 64;
  while (n2 < n) n2 <<= 1;
  bitonic_sort(kk, n2, s_key);

  // 2. per-bin prefixes over NON-collected bins (histogram masses)
  {
    constexpr int BPT = NBINS / FIN_T;
    double m1[BPT], m2[BPT];
    uint32_t cn[BPT];
    double t1 = 0.0, t2 = 0.0;
    uint64_t tc = 0;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      const int bb = t * BPT + q;
      const bool col = in_ranges(rs, bb);
      const uint32_t hc = a.s.hcnt[(int64_t)r * NBINS + bb];
      const double hm = (double)a.s.hmass[(int64_t)r * NBINS + bb] * (1.0 / FIX_SCALE);
      cn[q] = col ? 0u : hc;
      m1[q] = (!col && bb < rs.s1) ? hm : 0.0;
      m2[q] = (!col && bb < rs.s) ? hm : 0.0;
      t1 += m1[q];
      t2 += m2[q];
      tc += cn[q];
    }
    double tot1, tot2;
    uint64_t totc;
    double b1 = block_excl_scan_f64<FIN_T>(t1, s_dred, &tot1);
    double b2 = block_excl_scan_f64<FIN_T>(t2, s_dred, &tot2);
    uint64_t bc = block_excl_scan_u64<FIN_T>(tc, s_ured, &totc);
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      const int bb = t * BPT + q;
      s_P1[bb] = b1;
      s_P2[bb] = b2;
      s_PC[bb] = (uint32_t)bc;
      b1 += m1[q];
      b2 += m2[q];
      bc += cn[q];
    }
    if (t == 0) {
      s_P1[NBINS] = tot1;
      s_P2[NBINS] = tot2;
      s_PC[NBINS] = (uint32_t)totc;
    }
  }
  if (t == 0) s_kth = -INFINITY;
  __syncthreads();

  // 3. decode this thread's blocked positions [t*Q, t*Q+Q)
  const float m = rs.m;
  float lv[FIN_Q];
  int idv[FIN_Q], binv[FIN_Q];
  double wv[FIN_Q];
  uint64_t keyv[FIN_Q];
  bool pre[FIN_Q];
  const bool minp = p.min_p > 0.0f;
  const double lmp = minp ? log((double)p.min_p) : 0.0;
  const bool topk = p.top_k > 0 && p.top_k < V;
  const bool keep_ties = (p.flags & STRIM_FLAG_TOPK_KEEP_TIES) != 0;
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    const int pos = t * FIN_Q + q;
    const uint64_t key = s_key[pos];
    keyv[q] = key;
    lv[q] = fkey_desc_inv((uint32_t)(key >> 32));
    idv[q] = (int)(uint32_t)key;
    binv[q] = pos < n ? dbin(m - lv[q]) : NBINS - 1;
    wv[q] = pos < n ? exp((double)lv[q] - (double)m) : 0.0;
    if (pos < n && topk && keep_ties && s_PC[binv[q]] + (uint32_t)pos == (uint32_t)(p.top_k - 1))
      s_kth = lv[q];
  }
  __syncthreads();
  const float kth = s_kth;
  int first_bad = n;
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    const int pos = t * FIN_Q + q;
    bool ok = pos < n;
    if (ok && minp) ok = ((double)lv[q] - (double)m) >= lmp;
    if (ok && topk) {
      const uint32_t rank = s_PC[binv[q]] + (uint32_t)pos;
      ok = keep_ties ? (lv[q] >= kth) : (rank < (uint32_t)p.top_k);
    }
    pre[q] = ok;
    if (!ok && pos < first_bad) first_bad = pos;
  }
  // n_pre = first position failing the pre-filters (prefix property)
  first_bad = wave_min_i(first_bad);
  if ((t & (WAVE - 1)) == 0) s_ired[t / WAVE] = first_bad;
  __syncthreads();
  if (t == 0) {
    int v = n;
    for (int q = 0; q < FIN_T / WAVE; ++q) v = min(v, s_ired[q]);
    s_int[0] = v;
  }
  __syncthreads();
  const int n_pre = s_int[0];

  // 4. top-p over the pre-kept set
  double loc = 0.0;
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) loc += (t * FIN_Q + q < n_pre) ? wv[q] : 0.0;
  double tot_pre;
  double ex = block_excl_scan_f64<FIN_T>(loc, s_dred, &tot_pre);
  const double sig_pre = s_P1[NBINS] + tot_pre;
  int n_keep = n_pre;
  if (p.top_p < 1.0f) {
    const double P = (double)p.top_p;
    int fd = n;
    double run = ex;
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q) {
      const int pos = t * FIN_Q + q;
      if (pos < n_pre) {
        const double before = s_P1[binv[q]] + run;
        if (before / sig_pre - P > 0.0 && pos < fd) fd = pos;
        run += wv[q];
      }
    }
    fd = wave_min_i(fd);
    __syncthreads();
    if ((t & (WAVE - 1)) == 0) s_ired[t / WAVE] = fd;
    __syncthreads();
    if (t == 0) {
      int v = n_pre;
      for (int q = 0; q < FIN_T / WAVE; ++q) v = min(v, s_ired[q]);
      s_int[1] = v;
    }
    __syncthreads();
    n_keep = s_int[1];
  }
  // 5. kept mass and the kept prefix
  loc = 0.0;
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) loc += (t * FIN_Q + q < n_keep) ? wv[q] : 0.0;
  double tot_keep;
  const double exk = block_excl_scan_f64<FIN_T>(loc, s_dred, &tot_keep);
  const double sig_k = s_P2[NBINS] + tot_keep;
  const uint64_t last_key = n_keep > 0 ? s_key[n_keep - 1] : 0ull;

  // draft (verify rows): kept? and its mass
  double w_d = 0.0;
  uint64_t key_d = ~0ull;
  if (verify_draft_row && rs.l_draft > -INFINITY) {
    const int bd = dbin(m - rs.l_draft);
    key_d = ckey(rs.l_draft, rs.draft);
    const bool kept_d = in_ranges(rs, bd) ? (key_d <= last_key && last_key != 0ull) : (bd < rs.s);
    if (kept_d) w_d = exp((double)rs.l_draft - (double)m);
  }
  const bool one_hot = verify_draft_row;  // general-q residuals are not built yet
  const int excl_id = one_hot ? rs.draft : -1;

  // 6. draw
  int token = -1;
  if (a.noise_mode == STRIM_NOISE_ICDF) {
    const float u = row_uniform(a, r, p, 0);
    const double sig_r = sig_k - (one_hot ? w_d : 0.0);
    const double tgt = (double)u * sig_r;
    int best = n;
    double run = exk;
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q) {
      const int pos = t * FIN_Q + q;
      if (pos < n_keep) {
        double before = s_P2[binv[q]] + run;
        if (one_hot && key_d < keyv[q]) before -= w_d;
        const double wq = (idv[q] == excl_id) ? 0.0 : wv[q];
        if (before + wq > tgt && wq > 0.0 && pos < best) best = pos;
        run += wv[q];
      }
    }
    best = wave_min_i(best);
    __syncthreads();
    if ((t & (WAVE - 1)) == 0) s_ired[t / WAVE] = best;
    __syncthreads();
    if (t == 0) {
      int v = n;
      for (int q = 0; q < FIN_T / WAVE; ++q) v = min(v, s_ired[q]);
      s_int[2] = v;
    }
    __syncthreads();
    int bp = s_int[2];
    if (bp >= n_keep) {
      // rounding pushed the target past the last collected kept token
      if (rs.mode == MODE_A && n_keep > 0) bp = n_keep - 1;
      else bp = -1;
    }
    if (bp < 0) {
      fail(STRIM_ECAPACITY);
      return;
    }
    token = (int)(uint32_t)s_key[bp];
  } else {
    const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
    const bool topp = p.top_p < 1.0f;
    const bool by_rank = (p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp;
    const bool cand_sorted = no_lse ? topp : (topk || topp);
    const double lse = log(sig_k);
    const uint64_t pkey = mix64(p.seed, p.position);
    double bsc = -INFINITY;
    uint64_t btk = ~0ull;
    int bid = -1;
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q) {
      const int pos = t * FIN_Q + q;
      if (pos >= n_keep || idv[q] == excl_id) continue;
      const uint32_t rank = s_PC[binv[q]] + (uint32_t)pos;
      const int64_t nidx = by_rank ? (int64_t)rank : (int64_t)idv[q];
      const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + nidx]
                              : philox_uniform(pkey, (uint64_t)nidx);
      const double base = no_lse ? (double)lv[q] : ((double)lv[q] - (double)m) - lse;
      const double sc = base + gumbel64(u);
      const uint64_t tk = cand_sorted ? keyv[q] : (uint64_t)idv[q];
      if (bid < 0 || sc > bsc || (sc == bsc && tk < btk)) { bsc = sc; btk = tk; bid = idv[q]; }
    }
    if (rs.mode == MODE_B) {
      for (int cc = t; cc < a.W; cc += FIN_T) {
        const ChunkTop ct = a.s.ctop[(int64_t)r * a.s.wmax + cc];
        for (int h = 0; h < 2; ++h) {
          const int id = h == 0 ? ct.id0 : ct.id1;
          const float l = h == 0 ? ct.l0 : ct.l1;
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
    double bsc_out, second;
    block_argmax_score(bsc, btk, bid, s_dred, s_ured, s_ired, &s_int[3], &bsc_out, &second);
    token = s_int[3];
    if (token < 0) token = n_keep > 0 ? (int)(uint32_t)s_key[0] : -1;  // all scores -inf
    if (token < 0) {
      fail(STRIM_ECAPACITY);
      return;
    }
  }

  // 7. accept test (verify draft rows) and outputs
  if (t == 0) {
    RowState& o = a.s.rs[r];
    o.sum_kept = sig_k;
    o.last_key = last_key;
    o.token = token;
    if (verify_draft_row) {
      const double q_d = 1.0;
      const double p_d = w_d / sig_k;
      const double ratio = q_d > 0.0 ? p_d / q_d : (p_d > 0.0 ? INFINITY : 0.0);
      const float ua = row_uniform(a, r, p, a.noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V : 1);
      o.accept = ((double)ua < ratio) ? 1 : 0;
    }
    if (!a.verify) {
      a.out_ids[r] = token;
      if (a.out_status) a.out_status[r] = STRIM_OK;
    }
  }
}

// ---------------------------------------------------------------------------------
// k_probs: processed distribution (validation output)
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(TPB) void k_probs(Args a) {
  __shared__ uint32_t s_cnt[CHUNK];
  int r, c;
  map_block(a, blockIdx.x, r, c);
  const RowState rs = a.s.rs[r];
  int b, j;
  row_bj(a, r, b, j);
  const RowParams p = load_params(a, b, j);
  const int c0 = c * CHUNK;
  const int t = threadIdx.x;
  float* out = a.out_probs + (int64_t)r * a.V;
  const int i0 = c0 + t * EPT;
  if (rs.status != STRIM_OK || rs.greedy) {
    for (int e = 0; e < EPT; ++e)
      if (i0 + e < a.V)
        out[i0 + e] = (rs.status == STRIM_OK && i0 + e == rs.argmax) ? 1.0f : 0.0f;
    return;
  }
  if (p.pen) build_counts(a, b, j, c0, s_cnt);
  float l[EPT];
  bool nf = false;
  process_tokens(a, r, c0, p, s_cnt, l, nf);
  for (int e = 0; e < EPT; ++e) {
    const int i = i0 + e;
    if (i >= a.V) break;
    float pv = 0.0f;
    if (l[e] > -INFINITY) {
      const int bin = dbin(rs.m - l[e]);
      const bool kept = in_ranges(rs, bin) ? (rs.last_key != 0ull && ckey(l[e], i) <= rs.last_key)
                                           : (bin < rs.s);
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
  for (int j = 0; j <= k; ++j) {
    const RowState& rs = a.s.rs[(int64_t)b * (k + 1) + j];
    if (rs.status != STRIM_OK) {
      if (status == STRIM_OK) status = rs.status;
      if (a.out_row_accept && j < k) a.out_row_accept[(int64_t)b * k + j] = 0;
      if (a.out_row_token) a.out_row_token[(int64_t)b * (k + 1) + j] = -1;
      continue;
    }
    int acc = 0;
    if (j < k) acc = rs.greedy ? (rs.argmax == rs.draft) : rs.accept;
    const int tok = rs.greedy ? rs.argmax : rs.token;
    if (a.out_row_accept && j < k) a.out_row_accept[(int64_t)b * k + j] = acc;
    if (a.out_row_token) a.out_row_token[(int64_t)b * (k + 1) + j] = tok;
    if (alive) {
      if (j < k && acc) ++n;
      else {
        alive = false;
        token = tok;
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

}  // namespace strim
