/*
 * strim_oracle.h — CPU restatement of strim's token-selection path.
 *
 * TEST INFRASTRUCTURE ONLY. It is the parity checker for the HIP library and the timed
 * CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product (strim-engine_amd/) never links, loads or calls it.
 *
 * Semantics (each function cites the reference lines it restates; the extensions with
 * no reference source are defined here in closed form):
 *   counts  c_i   = occurrences of token i in the row history (+ verify draft prefix)
 *   penalty x'_i  = c_i > 0 ? ((x_i > 0 ? x_i / rep : x_i * rep) - freq * c_i) - pres : x_i
 *                   (fp32, each operation rounded, no fused multiply-add)
 *   mask    x'_i  = -inf where the bit is clear          (TokenMask.swift:15-17)
 *   temp    l_i   = x'_i / T  (fp32 division)             (SpecSampling.swift:45, Sampler.swift:37)
 *   order         : l descending, then id ascending
 *   min-p         : keep iff (double)l_i - (double)m >= log(min_p), m = max allowed l
 *   top-k         : exactly K first in order (SpecSampling.swift:49-54) or, with
 *                   STRIM_FLAG_TOPK_KEEP_TIES, every l >= the K-th value (Sampler.swift:39-43)
 *   top-p         : masses w_i = exp((double)l_i - (double)m); drop iff the mass strictly
 *                   before i in order exceeds P * (mass of the kept set)
 *                   (SpecSampling.swift:62-66, Sampler.swift:44-49)
 *   draw GUMBEL   : argmax over kept of (logp_i + g_i), g = -log(-log(max(u,1e-30)))
 *                   (SpecSampling.swift:78-86); with SCORE_NO_LSE the score is l_i + g_i
 *                   and with NOISE_BY_RANK (top-p active) g is indexed by sorted rank
 *                   (Sampler.swift:44-53)
 *   draw ICDF     : first kept token in order whose inclusive cumulative mass
 *                   exceeds u * (kept mass) (extension)
 *   verify        : accept iff u_accept < p(d) / q(d); residual max(0, p - q); one-hot q
 *                   reduces to the reference rule (SpecSampling.swift:74-106)
 * All probability arithmetic is fp64. Every decision that depends on rounding reports
 * its fp64 margin; the row margin is the smallest of them.
 */
#ifndef STRIM_ORACLE_H
#define STRIM_ORACLE_H

#include <stdint.h>
#include "../include/strim_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Per-row outcome of so_sample_batch. */
typedef struct so_row_result {
  int32_t token;     /* sampled id, -1 on error                                   */
  int32_t status;    /* STRIM_OK or STRIM_E*                                      */
  int32_t n_allowed; /* allowed tokens (mask set and l > -inf)                    */
  int32_t n_kept;    /* size of the filtered support                              */
  float m;           /* max allowed processed logit                               */
  float pad;
  double sum_kept;   /* sum of exp(l - m) over the kept set                       */
  double margin;     /* smallest fp64 decision margin (+inf when exact)           */
} so_row_result;

uint64_t so_mix(uint64_t seed, uint64_t position);
void so_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float so_uniform(uint64_t seed, uint64_t position, uint64_t index);
void so_uniforms(uint64_t seed, uint64_t position, int64_t n, float* out);
double so_gumbel(float u);

/* Processed logits of one row (penalties, mask, temperature). Greedy rows (T <= 0)
 * return the penalised, masked logits without temperature. Returns a status. */
int32_t so_process_row(const float* x, int32_t V, const uint32_t* mask, const int32_t* hist,
                       int32_t hlen, const int32_t* extra, int32_t nextra,
                       const strim_sampling_params* p, float* l_out);

/* Batched sampling. x [B][V] float32 (bf16 inputs converted exactly by the caller).
 * mask [B][mask_stride] or NULL, history [B][H] + history_len [B] (or NULL = H),
 * noise per STRIM_NOISE_* (NULL = Philox). out_probs [B][V] or NULL.
 * nthreads <= 0 uses the OpenMP default. */
void so_sample_batch(const float* x, int32_t B, int32_t V, const strim_sampling_params* params,
                     const uint32_t* mask, int64_t mask_stride, const int32_t* history,
                     const int32_t* history_len, int32_t H, int32_t noise_mode,
                     const float* noise, so_row_result* out, float* out_probs, int32_t nthreads);

/* Batched verify; shapes as strim_verify (float32 inputs). draft_logits may be NULL. */
void so_verify_batch(const float* target, int32_t B, int32_t k, int32_t V,
                     const float* draft_logits, int32_t Vd, const int32_t* draft_to_full,
                     const int32_t* draft_tokens, const strim_sampling_params* params,
                     const uint32_t* mask, int64_t mask_stride, const int32_t* history,
                     const int32_t* history_len, int32_t H, int32_t noise_mode,
                     const float* noise, int32_t* out_accepted, int32_t* out_token,
                     int32_t* out_row_accept, int32_t* out_row_token, int32_t* out_status,
                     double* out_margin, float* out_probs, int32_t nthreads);

#ifdef __cplusplus
}
#endif
#endif
