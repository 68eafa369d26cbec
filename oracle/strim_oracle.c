/*
 * strim_oracle.c — CPU restatement of strim's token-selection path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product never does. Built with -ffp-contract=off so every fp32 step is one IEEE
 * rounding, exactly as the semantics below are written. See strim_oracle.h for the
 * full definition of each stage and the reference lines it follows.
 *
 * Parity pins (tests/test_oracle.py):
 *   so_mix            SplitMix64 published outputs (seed 0); SpecSampling.swift:29-34
 *   so_philox4x32_10  Random123 known-answer vectors (Salmon et al., SC'11)
 *   filter            SpecSamplingTests.filteredMatchesReference (ln[8,4,2,1,1]),
 *                     brute force on tiny V (enumerated orders), closed forms
 *   draws             SpecSamplingTests.temperatureZeroPathEqualsArgmax,
 *                     verifyAcceptCountSemantics, exact icdf quantile grids and
 *                     chi-square marginals
 *   penalties, min-p  brute-force restatement in numpy (float32 rounding steps)
 */
#include "strim_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Mutation switch of the known-answer tests' discrimination check: the tests build
 * variants of this file with SO_MUTANT set to one of the values below (a plausible
 * indexing mistake each) and assert that the injected-uniform known-answer tests FAIL on
 * every variant. The normal build leaves it 0. */
#ifndef SO_MUTANT
#define SO_MUTANT 0
#endif
#define SO_MUT_NOISE_INDEX 1  /* Gumbel noise by sorted position instead of token id, and
                                 by token id instead of rank under NOISE_BY_RANK         */
#define SO_MUT_ACCEPT_INDEX 2 /* accept uniform from element 0 instead of V (Gumbel)     */
#define SO_MUT_ICDF_SWAP 3    /* icdf draw and accept elements exchanged                 */

/* ------------------------------------------------------------------------------ */
/* Random numbers                                                                  */
/* ------------------------------------------------------------------------------ */

/* SpecSampling.mix (Sources/StrimCore/SpecSampling.swift:29-34): the SplitMix64
 * finaliser applied to seed + golden-gamma * (position + 1), wrapping u64 arithmetic. */
uint64_t so_mix(uint64_t seed, uint64_t position) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (position + 1u);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As Easy as
 * 1, 2, 3", SC'11): 10 rounds of two 32x32->64 multiplies, key bumped by the Weyl
 * constants between rounds. */
void so_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
    uint32_t n1 = (uint32_t)p1;
    uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    uint32_t n3 = (uint32_t)p0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* Uniform element `index` of the [V+1] noise vector of one output position: the
 * position key is SpecSampling.mix(seed, position) (SpecSampling.swift:38); Philox
 * counter = index / 4, lane = index % 4; u = (word >> 8) * 2^-24, in [0, 1). */
float so_uniform(uint64_t seed, uint64_t position, uint64_t index) {
  uint64_t kk = so_mix(seed, position);
  uint32_t key[2] = {(uint32_t)kk, (uint32_t)(kk >> 32)};
  uint64_t blk = index >> 2;
  uint32_t ctr[4] = {(uint32_t)blk, (uint32_t)(blk >> 32), 0u, 0u};
  uint32_t out[4];
  so_philox4x32_10(ctr, key, out);
  return (float)(out[index & 3u] >> 8) * 5.9604644775390625e-08f;
}

void so_uniforms(uint64_t seed, uint64_t position, int64_t n, float* out) {
  uint64_t kk = so_mix(seed, position);
  uint32_t key[2] = {(uint32_t)kk, (uint32_t)(kk >> 32)};
  for (int64_t b = 0; b * 4 < n; ++b) {
    uint32_t ctr[4] = {(uint32_t)b, (uint32_t)((uint64_t)b >> 32), 0u, 0u};
    uint32_t w[4];
    so_philox4x32_10(ctr, key, w);
    for (int j = 0; j < 4 && b * 4 + j < n; ++j)
      out[b * 4 + j] = (float)(w[j] >> 8) * 5.9604644775390625e-08f;
  }
}

/* Gumbel transform of SpecSampling.rowOutcome (SpecSampling.swift:79):
 * -log(-log(max(u, 1e-30))), the clamp in float32, the logs in fp64. */
double so_gumbel(float u) {
  float uu = u > 1e-30f ? u : 1e-30f;
  return -log(-log((double)uu));
}

/* ------------------------------------------------------------------------------ */
/* Row processing: penalties -> mask -> temperature                                */
/* ------------------------------------------------------------------------------ */

static int so_params_ok(const strim_sampling_params* p) {
  if (isnan(p->temperature) || isinf(p->temperature)) return 0;
  if (!(p->top_p > 0.0f && p->top_p <= 1.0f)) return 0;
  if (p->top_k < 0) return 0;
  if (!(p->min_p >= 0.0f && p->min_p <= 1.0f)) return 0;
  if (!(p->repetition_penalty > 0.0f) || isinf(p->repetition_penalty)) return 0;
  if (!isfinite(p->presence_penalty) || !isfinite(p->frequency_penalty)) return 0;
  return 1;
}

static inline int so_allowed(const uint32_t* mask, int32_t i) {
  return mask == NULL || ((mask[i >> 5] >> (i & 31)) & 1u);
}

int32_t so_process_row(const float* x, int32_t V, const uint32_t* mask, const int32_t* hist,
                       int32_t hlen, const int32_t* extra, int32_t nextra,
                       const strim_sampling_params* p, float* l_out) {
  if (!so_params_ok(p)) return STRIM_EINVAL;
  int32_t* cnt = NULL;
  if ((hist && hlen > 0) || (extra && nextra > 0)) {
    cnt = (int32_t*)calloc((size_t)V, sizeof(int32_t));
    for (int32_t j = 0; hist && j < hlen; ++j)
      if (hist[j] >= 0 && hist[j] < V) cnt[hist[j]]++;
    for (int32_t j = 0; extra && j < nextra; ++j)
      if (extra[j] >= 0 && extra[j] < V) cnt[extra[j]]++;
  }
  const int greedy = !(p->temperature > 0.0f);
  const float rep = p->repetition_penalty, pres = p->presence_penalty,
              freq = p->frequency_penalty, T = p->temperature;
  int nonfinite = 0;
  int32_t n_allowed = 0;
  for (int32_t i = 0; i < V; ++i) {
    float v = x[i];
    if (cnt && cnt[i] > 0) {
      v = v > 0.0f ? v / rep : v * rep;
      v = v - freq * (float)cnt[i];
      v = v - pres;
    }
    if (!so_allowed(mask, i)) { l_out[i] = -INFINITY; continue; }
    if (isnan(v) || v == INFINITY) nonfinite = 1;
    float l = greedy ? v : v / T;
    if (l == INFINITY) nonfinite = 1;
    l_out[i] = l;
    if (l > -INFINITY) n_allowed++;
  }
  free(cnt);
  if (nonfinite) return STRIM_ENONFINITE;
  if (n_allowed == 0) return STRIM_EEMPTY;
  return STRIM_OK;
}

/* ------------------------------------------------------------------------------ */
/* Ordering keys                                                                   */
/* ------------------------------------------------------------------------------ */

/* 32-bit key whose ascending order is the float's DEScending order (-0 == +0). */
static inline uint32_t so_fkey_desc(float f) {
  if (f == 0.0f) f = 0.0f;
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ~asc;
}
/* Ascending order of this 64-bit key = (l descending, id ascending). */
static inline uint64_t so_ckey(float l, int32_t id) {
  return ((uint64_t)so_fkey_desc(l) << 32) | (uint32_t)id;
}

static int so_cmp_u64(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return (x > y) - (x < y);
}

/* Place the n_sel smallest keys first (unordered), average O(n). */
static void so_select(uint64_t* a, int64_t n, int64_t n_sel) {
  int64_t lo = 0, hi = n - 1, k = n_sel - 1;
  while (hi > lo) {
    int64_t mid = lo + (hi - lo) / 2;
    uint64_t x = a[lo], y = a[mid], z = a[hi];
    uint64_t piv = (x < y) ? ((y < z) ? y : (x < z ? z : x)) : ((x < z) ? x : (y < z ? z : y));
    int64_t i = lo, j = hi;
    while (i <= j) {
      while (a[i] < piv) i++;
      while (a[j] > piv) j--;
      if (i <= j) { uint64_t t = a[i]; a[i] = a[j]; a[j] = t; i++; j--; }
    }
    if (k <= j) hi = j;
    else if (k >= i) lo = i;
    else break;
  }
}

/* ------------------------------------------------------------------------------ */
/* Filtered distribution                                                          */
/* ------------------------------------------------------------------------------ */

typedef struct {
  int32_t n;         /* kept count                                              */
  int32_t sorted;    /* ids in (l desc, id asc) order, else id order             */
  int32_t cand_sorted; /* reference candidate order is the sorted one          */
  int32_t topp;      /* top-p active                                             */
  float m;
  int32_t n_allowed;
  double sumw;       /* sum of w over kept                                       */
  double margin;
  int32_t* ids;      /* kept ids                                                 */
  double* w;         /* exp(l - m) per kept id                                   */
  uint64_t* keys;    /* scratch [V]                                              */
} so_dist;

static void so_dist_alloc(so_dist* d, int32_t V) {
  memset(d, 0, sizeof(*d));
  d->ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)V);
  d->w = (double*)malloc(sizeof(double) * (size_t)V);
  d->keys = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
}
static void so_dist_free(so_dist* d) {
  free(d->ids); free(d->w); free(d->keys);
}

static inline double so_minabs(double a, double b) { return a < b ? a : b; }

/* min-p -> top-k -> top-p over processed logits l (status already STRIM_OK).
 * SpecSampling.filtered (SpecSampling.swift:44-68) and Sampler.sample's filtering
 * (Sampler.swift:37-49); min-p is the extension defined in the header. need_sorted
 * forces the kept set into (l desc, id asc) order (icdf draws, rank noise). */
static void so_filter(const float* l, int32_t V, const strim_sampling_params* p, int need_sorted,
                      so_dist* d) {
  const int32_t K = p->top_k;
  const int topk = K > 0 && K < V;
  const int topp = p->top_p < 1.0f;
  const int keep_ties = (p->flags & STRIM_FLAG_TOPK_KEEP_TIES) != 0;
  const int sampler_order = (p->flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
  d->margin = INFINITY;
  d->topp = topp;
  /* reference candidate order: filtered() returns sorted ids when top-k or top-p is
   * active; Sampler's categorical runs over the id-ordered row unless top-p sorts it. */
  d->cand_sorted = sampler_order ? topp : (topk || topp);

  float m = -INFINITY;
  int32_t na = 0;
  for (int32_t i = 0; i < V; ++i)
    if (l[i] > -INFINITY) { na++; if (l[i] > m) m = l[i]; }
  d->m = m;
  d->n_allowed = na;

  /* min-p (extension): keep iff l - m >= log(min_p), in fp64. */
  const int minp = p->min_p > 0.0f;
  const double lmp = minp ? log((double)p->min_p) : 0.0;
  int64_t n = 0;
  for (int32_t i = 0; i < V; ++i) {
    if (!(l[i] > -INFINITY)) continue;
    if (minp) {
      double diff = (double)l[i] - (double)m - lmp;
      d->margin = so_minabs(d->margin, fabs(diff));
      if (diff < 0.0) continue;
    }
    d->keys[n++] = so_ckey(l[i], i);
  }
  /* keys[] is in id order here */
  int sorted = 0;
  if (topk && n > K) {
    so_select(d->keys, n, K);
    if (keep_ties) {
      /* K-th value: the largest key among the K selected */
      uint64_t kmax = 0;
      for (int64_t j = 0; j < K; ++j) if (d->keys[j] > kmax) kmax = d->keys[j];
      uint32_t kth = (uint32_t)(kmax >> 32);
      int64_t m2 = K;
      for (int64_t j = K; j < n; ++j)
        if ((uint32_t)(d->keys[j] >> 32) == kth) d->keys[m2++] = d->keys[j];
      n = m2;
    } else {
      n = K;
    }
    qsort(d->keys, (size_t)n, sizeof(uint64_t), so_cmp_u64);
    sorted = 1;
  } else if (topp || need_sorted || d->cand_sorted || SO_MUTANT == SO_MUT_NOISE_INDEX) {
    qsort(d->keys, (size_t)n, sizeof(uint64_t), so_cmp_u64);
    sorted = 1;
  }
  for (int64_t j = 0; j < n; ++j) {
    int32_t id = (int32_t)(uint32_t)d->keys[j];
    d->ids[j] = id;
    d->w[j] = exp((double)l[id] - (double)m);
  }
  /* top-p: drop iff the mass strictly before the token exceeds P * (kept mass). */
  if (topp) {
    double S = 0.0;
    for (int64_t j = 0; j < n; ++j) S += d->w[j];
    const double P = (double)p->top_p;
    double before = 0.0;
    int64_t cut = n;
    for (int64_t j = 0; j < n; ++j) {
      double r = before / S - P;
      if (r > 0.0) { cut = j; d->margin = so_minabs(d->margin, fabs(r)); break; }
      d->margin = so_minabs(d->margin, fabs(r));
      before += d->w[j];
    }
    n = cut;
  }
  double sw = 0.0;
  for (int64_t j = 0; j < n; ++j) sw += d->w[j];
  d->n = (int32_t)n;
  d->sorted = sorted;
  d->sumw = sw;
}

/* ------------------------------------------------------------------------------ */
/* Draws                                                                           */
/* ------------------------------------------------------------------------------ */

/* Noise source of one row: injected pointer (layout per mode) or Philox. */
typedef struct {
  const float* inj;   /* row base of injected noise or NULL */
  uint64_t seed, pos;
} so_noise;

static inline float so_u(const so_noise* nz, int64_t idx) {
  return nz->inj ? nz->inj[idx] : so_uniform(nz->seed, nz->pos, (uint64_t)idx);
}

/* icdf draw over weights r (aligned with d->ids, sorted order): first j with
 * inclusive cumulative > u * sum. Returns the index into d->ids. */
static int32_t so_icdf(const so_dist* d, const double* r, float u, double* margin) {
  double S = 0.0;
  for (int32_t j = 0; j < d->n; ++j) S += r[j];
  if (!(S > 0.0)) return 0;
  const double t = (double)u * S;
  double c = 0.0;
  for (int32_t j = 0; j < d->n; ++j) {
    double prev = c;
    c += r[j];
    if (c > t) {
      *margin = so_minabs(*margin, so_minabs(fabs(c - t), fabs(prev - t)) / S);
      return j;
    }
  }
  *margin = 0.0; /* only reachable through rounding at the very end */
  return d->n - 1;
}

/* Gumbel-max over kept entries with per-entry base score s[j] (-inf = excluded).
 * Noise index = token id, or sorted rank when by_rank. First max wins (MLX argMax). */
static int32_t so_gumbel_max(const so_dist* d, const double* s, const so_noise* nz, int by_rank,
                             double* margin) {
  int32_t best = -1;
  double b1 = -INFINITY, b2 = -INFINITY;
  for (int32_t j = 0; j < d->n; ++j) {
    if (s[j] == -INFINITY) continue;
    const int by_pos = SO_MUTANT == SO_MUT_NOISE_INDEX ? !by_rank : by_rank;
    double g = so_gumbel(so_u(nz, by_pos ? j : d->ids[j]));
    double sc = s[j] + g;
    if (best < 0 || sc > b1) { b2 = b1; b1 = sc; best = j; }
    else if (sc > b2) b2 = sc;
  }
  if (best < 0) return 0; /* every score -inf: argMax returns the first candidate */
  if (b2 > -INFINITY) *margin = so_minabs(*margin, b1 - b2);
  return best;
}

/* Reorder the kept set to id order (the reference's candidate order when no filter
 * sorted it). */
static int so_cmp_i32(const void* a, const void* b) {
  int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
  return (x > y) - (x < y);
}
static void so_to_id_order(so_dist* d, const float* l) {
  if (!d->sorted) return;
  qsort(d->ids, (size_t)d->n, sizeof(int32_t), so_cmp_i32);
  for (int32_t j = 0; j < d->n; ++j) d->w[j] = exp((double)l[d->ids[j]] - (double)d->m);
  d->sorted = 0;
}

/* Plain draw from the filtered distribution. Returns the token id. */
static int32_t so_draw(so_dist* d, const float* l, const strim_sampling_params* p, int noise_mode,
                       const so_noise* nz, int64_t accept_idx_unused, double* scratch) {
  (void)accept_idx_unused;
  if (noise_mode == STRIM_NOISE_ICDF) {
    int32_t j = so_icdf(d, d->w, so_u(nz, SO_MUTANT == SO_MUT_ICDF_SWAP ? 1 : 0), &d->margin);
    return d->ids[j];
  }
  const int no_lse = (p->flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
  const int by_rank = (p->flags & STRIM_FLAG_NOISE_BY_RANK) && d->topp;
  if (!d->cand_sorted && !by_rank && SO_MUTANT != SO_MUT_NOISE_INDEX) so_to_id_order(d, l);
  const double lse = log(d->sumw);
  for (int32_t j = 0; j < d->n; ++j) {
    double lj = (double)l[d->ids[j]];
    scratch[j] = no_lse ? lj : (lj - (double)d->m) - lse;
  }
  int32_t j = so_gumbel_max(d, scratch, nz, by_rank, &d->margin);
  return d->ids[j];
}

/* ------------------------------------------------------------------------------ */
/* Batched sampling                                                                */
/* ------------------------------------------------------------------------------ */

static int32_t so_argmax(const float* l, int32_t V) {
  int32_t best = -1;
  float bv = -INFINITY;
  for (int32_t i = 0; i < V; ++i)
    if (l[i] > -INFINITY && (best < 0 || l[i] > bv)) { bv = l[i]; best = i; }
  return best;
}

static void so_sample_row(const float* x, int32_t V, const strim_sampling_params* p,
                          const uint32_t* mask, const int32_t* hist, int32_t hlen,
                          int32_t noise_mode, const float* noise_row, float* lbuf,
                          so_dist* d, double* scratch, so_row_result* res, float* probs) {
  memset(res, 0, sizeof(*res));
  res->token = -1;
  res->margin = INFINITY;
  if (probs) for (int32_t i = 0; i < V; ++i) probs[i] = 0.0f;
  int32_t st = so_process_row(x, V, mask, hist, hlen, NULL, 0, p, lbuf);
  res->status = st;
  if (st != STRIM_OK) return;
  if (!(p->temperature > 0.0f)) { /* greedy: argMax of the masked row (EngineCore.swift:933) */
    res->token = so_argmax(lbuf, V);
    res->n_kept = 1;
    res->n_allowed = 0;
    for (int32_t i = 0; i < V; ++i) if (lbuf[i] > -INFINITY) res->n_allowed++;
    if (probs) probs[res->token] = 1.0f;
    return;
  }
  so_noise nz = {noise_row, p->seed, p->position};
  so_filter(lbuf, V, p, noise_mode == STRIM_NOISE_ICDF, d);
  if (probs)
    for (int32_t j = 0; j < d->n; ++j) probs[d->ids[j]] = (float)(d->w[j] / d->sumw);
  res->token = so_draw(d, lbuf, p, noise_mode, &nz, V, scratch);
  res->n_allowed = d->n_allowed;
  res->n_kept = d->n;
  res->m = d->m;
  res->sum_kept = d->sumw;
  res->margin = d->margin;
}

void so_sample_batch(const float* x, int32_t B, int32_t V, const strim_sampling_params* params,
                     const uint32_t* mask, int64_t mask_stride, const int32_t* history,
                     const int32_t* history_len, int32_t H, int32_t noise_mode,
                     const float* noise, so_row_result* out, float* out_probs, int32_t nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const int64_t nstride = noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V + 1 : 2;
#pragma omp parallel
  {
    float* lbuf = (float*)malloc(sizeof(float) * (size_t)V);
    double* scratch = (double*)malloc(sizeof(double) * (size_t)V);
    so_dist d;
    so_dist_alloc(&d, V);
#pragma omp for schedule(dynamic, 1)
    for (int32_t b = 0; b < B; ++b) {
      int32_t hl = history ? (history_len ? history_len[b] : H) : 0;
      if (hl > H) hl = H;
      so_sample_row(x + (int64_t)b * V, V, &params[b], mask ? mask + (int64_t)b * mask_stride : NULL,
                    history ? history + (int64_t)b * H : NULL, hl, noise_mode,
                    noise ? noise + (int64_t)b * nstride : NULL, lbuf, &d, scratch, &out[b],
                    out_probs ? out_probs + (int64_t)b * V : NULL);
    }
    so_dist_free(&d);
    free(lbuf);
    free(scratch);
  }
}

/* ------------------------------------------------------------------------------ */
/* Verify                                                                          */
/* ------------------------------------------------------------------------------ */

static int32_t so_table_find(const int32_t* t, int32_t n, int32_t id) {
  int32_t lo = 0, hi = n - 1;
  while (lo <= hi) {
    int32_t mid = lo + (hi - lo) / 2;
    if (t[mid] == id) return mid;
    if (t[mid] < id) lo = mid + 1; else hi = mid - 1;
  }
  return -1;
}

void so_verify_batch(const float* target, int32_t B, int32_t k, int32_t V,
                     const float* draft_logits, int32_t Vd, const int32_t* draft_to_full,
                     const int32_t* draft_tokens, const strim_sampling_params* params,
                     const uint32_t* mask, int64_t mask_stride, const int32_t* history,
                     const int32_t* history_len, int32_t H, int32_t noise_mode,
                     const float* noise, int32_t* out_accepted, int32_t* out_token,
                     int32_t* out_row_accept, int32_t* out_row_token, int32_t* out_status,
                     double* out_margin, float* out_probs, int32_t nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const int64_t nstride = noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V + 1 : 2;
#pragma omp parallel
  {
    float* lbuf = (float*)malloc(sizeof(float) * (size_t)V);
    double* scratch = (double*)malloc(sizeof(double) * (size_t)V);
    double* qfull = (double*)malloc(sizeof(double) * (size_t)V);
    double* qd = (double*)malloc(sizeof(double) * (size_t)(Vd > 0 ? Vd : 1));
    so_dist d;
    so_dist_alloc(&d, V);
#pragma omp for schedule(dynamic, 1)
    for (int32_t b = 0; b < B; ++b) {
      const strim_sampling_params* p = &params[b];
      int32_t hl = history ? (history_len ? history_len[b] : H) : 0;
      if (hl > H) hl = H;
      const int32_t* hist = history ? history + (int64_t)b * H : NULL;
      const int32_t* drafts = draft_tokens + (int64_t)b * k;
      const int greedy = !(p->temperature > 0.0f);
      int32_t status = STRIM_OK;
      int32_t n_acc = 0, alive = 1, token = -1;
      double margin = INFINITY;
      for (int32_t j = 0; j <= k; ++j) {
        const int64_t row = (int64_t)b * (k + 1) + j;
        const float* x = target + row * V;
        const uint32_t* mrow = mask ? mask + row * mask_stride : NULL;
        float* probs = out_probs ? out_probs + row * V : NULL;
        if (probs) for (int32_t i = 0; i < V; ++i) probs[i] = 0.0f;
        const int32_t dj = j < k ? drafts[j] : -1;
        /* a row error ends the sequence only when the accept chain reaches the row (the
         * reference consumes rows 0 .. n alone, SpecSampling.swift:101-105); a later
         * row reports it in its own outputs */
        int32_t st = (j < k && (dj < 0 || dj >= V)) ? STRIM_EINVAL
                                                    : so_process_row(x, V, mrow, hist, hl, drafts, j, p, lbuf);
        int32_t acc = 0, tok = -1;
        if (st == STRIM_OK && !greedy && j < k && draft_logits != NULL &&
            so_table_find(draft_to_full, Vd, dj) < 0)
          st = STRIM_EINVAL;
        if (st != STRIM_OK) {
          if (alive) { status = st; alive = 0; }
          if (out_row_accept && j < k) out_row_accept[(int64_t)b * k + j] = 0;
          if (out_row_token) out_row_token[(int64_t)b * (k + 1) + j] = -1;
          continue;
        }
        if (greedy) {
          /* SpecStream.swift:269-273: accept while argmax == draft */
          tok = so_argmax(lbuf, V);
          acc = j < k && tok == dj;
          if (probs) probs[tok] = 1.0f;
        } else {
          so_noise nz = {noise ? noise + row * nstride : NULL, p->seed, p->position + (uint64_t)j};
          /* verify is the SpecSampling path: the Sampler-only flags do not apply */
          strim_sampling_params pv = *p;
          pv.flags &= STRIM_FLAG_TOPK_KEEP_TIES;
          so_filter(lbuf, V, &pv, noise_mode == STRIM_NOISE_ICDF, &d);
          if (probs)
            for (int32_t t = 0; t < d.n; ++t) probs[d.ids[t]] = (float)(d.w[t] / d.sumw);
          if (j == k) {
            tok = so_draw(&d, lbuf, &pv, noise_mode, &nz, V, scratch);
          } else {
            /* draft distribution q (one-hot when draft_logits == NULL) */
            double q_d = 1.0;
            int general = draft_logits != NULL;
            if (general) {
              const float* dl = draft_logits + ((int64_t)b * k + j) * Vd;
              int32_t t = so_table_find(draft_to_full, Vd, dj); /* >= 0: checked above */
              float mq = -INFINITY;
              for (int32_t a = 0; a < Vd; ++a) {
                float v = dl[a] / p->temperature;
                qd[a] = v;
                if (v > mq) mq = v;
              }
              double Z = 0.0;
              for (int32_t a = 0; a < Vd; ++a) { qd[a] = exp(qd[a] - (double)mq); Z += qd[a]; }
              for (int32_t a = 0; a < Vd; ++a) qd[a] /= Z;
              q_d = qd[t];
            }
            /* p(d) under the filtered target */
            double p_d = 0.0;
            int32_t dpos = -1;
            for (int32_t t = 0; t < d.n; ++t)
              if (d.ids[t] == dj) { dpos = t; p_d = d.w[t] / d.sumw; break; }
            double ratio = q_d > 0.0 ? p_d / q_d : (p_d > 0.0 ? INFINITY : 0.0);
            /* accept uniform: element V of the Gumbel vector (SpecSampling.swift:83),
             * element 1 of the icdf pair */
            const int64_t acc_idx =
                noise_mode == STRIM_NOISE_GUMBEL ? (SO_MUTANT == SO_MUT_ACCEPT_INDEX ? 0 : V)
                                                 : (SO_MUTANT == SO_MUT_ICDF_SWAP ? 0 : 1);
            float ua = so_u(&nz, acc_idx);
            acc = (double)ua < ratio;
            if (isfinite(ratio)) margin = so_minabs(margin, fabs((double)ua - ratio));
            /* residual max(0, p - q) over the kept set */
            if (general) {
              for (int32_t i = 0; i < V; ++i) qfull[i] = 0.0;
              for (int32_t a = 0; a < Vd; ++a) qfull[draft_to_full[a]] = qd[a];
            }
            if (noise_mode == STRIM_NOISE_ICDF) {
              for (int32_t t = 0; t < d.n; ++t) {
                double pi = d.w[t] / d.sumw;
                double qi = general ? qfull[d.ids[t]] : (t == dpos ? 1.0 : 0.0);
                double r = pi - qi;
                scratch[t] = r > 0.0 ? r : 0.0;
              }
              int32_t sel =
                  so_icdf(&d, scratch, so_u(&nz, SO_MUTANT == SO_MUT_ICDF_SWAP ? 1 : 0), &d.margin);
              tok = d.ids[sel];
            } else {
              if (!d.cand_sorted) {
                so_to_id_order(&d, lbuf);
                dpos = -1;
                for (int32_t t = 0; t < d.n; ++t) if (d.ids[t] == dj) dpos = t;
              }
              const double lse = log(d.sumw);
              for (int32_t t = 0; t < d.n; ++t) {
                double logp = ((double)lbuf[d.ids[t]] - (double)d.m) - lse;
                double qi = general ? qfull[d.ids[t]] : (t == dpos ? 1.0 : 0.0);
                if (qi == 0.0) scratch[t] = logp;
                else {
                  double r = exp(logp) - qi;
                  scratch[t] = r > 0.0 ? log(r) : -INFINITY;
                }
              }
              int32_t sel = so_gumbel_max(&d, scratch, &nz, 0, &d.margin);
              tok = d.ids[sel];
            }
          }
          if (alive) margin = so_minabs(margin, d.margin);
        }
        if (out_row_accept && j < k) out_row_accept[(int64_t)b * k + j] = acc;
        if (out_row_token) out_row_token[(int64_t)b * (k + 1) + j] = tok;
        if (alive) {
          if (j < k && acc) n_acc++;
          else { alive = 0; token = tok; }
        }
      }
      if (status != STRIM_OK) { n_acc = 0; token = -1; }
      out_accepted[b] = n_acc;
      out_token[b] = token;
      if (out_status) out_status[b] = status;
      if (out_margin) out_margin[b] = margin;
    }
    so_dist_free(&d);
    free(lbuf); free(scratch); free(qfull); free(qd);
  }
}
