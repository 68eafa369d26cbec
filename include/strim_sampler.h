/*
 * strim_sampler.h — C ABI of the MI355X (gfx950) token-selection path.
 *
 * This library replaces strim's per-step token selection: logit penalties, grammar
 * bitmask, temperature, min-p, top-k / top-p, categorical draw, and the MTP
 * speculative accept/reject verifier. Every entry point is plain C: device pointers,
 * sizes and a HIP stream passed as void*. No torch or C++ types cross the boundary.
 *
 * Reference interfaces replaced (paths relative to the strim-engine repository):
 *   strim_sample  <- Sampler.sample / Sampler.sampleFirst
 *                      (Sources/StrimEngine/Sampler.swift:29-54),
 *                    SpecSampling.sample (Sources/StrimCore/SpecSampling.swift:109-116),
 *                    the per-row pick loop of EngineCore.decodeBatch
 *                      (Sources/StrimEngine/EngineCore.swift:968-974,998-1002),
 *                    greedy argMax (EngineCore.swift:933,973).
 *   strim_verify  <- SpecSampling.verify / rowOutcome
 *                      (Sources/StrimCore/SpecSampling.swift:74-106) and the greedy
 *                    prefix-compare verify (Sources/StrimCore/SpecStream.swift:256-273).
 *   strim_mask_logits <- maskLogits (Sources/StrimCore/TokenMask.swift:15-17).
 *   strim_draft_argmax <- MTP.nextTokenIndex / nextToken draft map
 *                      (Sources/StrimCore/MTP.swift:104-111,120-125).
 *   strim_sampling_params <- GenParams (Sources/StrimEngine/EngineAPI.swift:47-67) and
 *                    SamplingConfig (Sources/StrimCore/SpecSampling.swift:7-15).
 *   strim_check_params <- request validation (Sources/StrimServer/ChatRequest.swift:148-161).
 *
 * Conventions
 *   - All array arguments are DEVICE pointers unless stated, owned by the caller. The
 *     per-row sampling params are HOST structs (the reference's GenParams are host
 *     values); they travel inside the kernel arguments, so a call copies nothing.
 *   - Calls are stream-ordered and asynchronous. A context (strim_ctx) owns scratch
 *     memory; calls that share one context must not overlap in time (use one context
 *     per stream), mirroring the reference's single engine thread
 *     (Sources/StrimEngine/Inbox.swift:42-46).
 *   - The synchronous return value reports host-checkable errors (sizes, pointers,
 *     dtype). Data-dependent errors are reported per row in out_status (device) and
 *     the row's output id is -1.
 *   - Token order used for every ordered decision: logit descending, then token id
 *     ascending.
 */
#ifndef STRIM_SAMPLER_H
#define STRIM_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------------- */
#define STRIM_OK 0
#define STRIM_EINVAL (-1)     /* bad params / sizes / pointers / draft id not in table */
#define STRIM_EEMPTY (-2)     /* the row allows no token (all-zero mask or all -inf)    */
#define STRIM_ENONFINITE (-3) /* NaN or +inf logit in an allowed position              */
#define STRIM_ECAPACITY (-4)  /* the call exceeds a fixed capacity: V above the
                                 context's max_vocab, or the no-allocation limits      */
#define STRIM_EHIP (-5)       /* HIP runtime error                                      */
#define STRIM_ENOMEM (-6)     /* device allocation failed                              */

/* ---- logits dtype --------------------------------------------------------------- */
#define STRIM_DTYPE_F32 0
#define STRIM_DTYPE_BF16 1

/* ---- noise modes -----------------------------------------------------------------
 * ICDF   : one draw uniform and one accept uniform per row. Injected layout [R][2]
 *          (draw, accept). Draw = first kept token (in token order) whose inclusive
 *          cumulative mass exceeds u * (kept mass).
 * GUMBEL : the reference scheme (SpecSampling.swift:24-27,78-85): uniforms [R][V+1];
 *          element i < V is Gumbel noise for token i (or for sorted rank i with
 *          STRIM_FLAG_NOISE_BY_RANK), element V is the accept uniform.
 * noise == NULL: uniforms come from Philox4x32-10 keyed by
 *          SplitMix64(seed, position) (SpecSampling.mix, SpecSampling.swift:29-34), counter
 *          = element index / 4. ICDF uses elements 0 (draw) and 1 (accept).
 * Injected uniforms must lie in [0, 1) (what the Philox stream produces: k 2^-24). The
 * library does not check them. Below 1e-30 they are taken as 1e-30; exactly 1 gives a
 * Gumbel score of +inf; above 1, or NaN, gives a NaN score, and such a token is never
 * drawn (its score loses every comparison), where a scalar loop over the tokens may
 * keep a NaN score it met first.                                                     */
#define STRIM_NOISE_ICDF 0
#define STRIM_NOISE_GUMBEL 1

/* ---- per-row flags ------------------------------------------------------------- */
#define STRIM_FLAG_TOPK_KEEP_TIES 1u /* keep every token tied with the k-th value
                                        (Sampler.swift:39-43); default keeps exactly k
                                        (SpecSampling.swift:49-54)                      */
#define STRIM_FLAG_NOISE_BY_RANK 2u  /* Gumbel noise indexed by sorted rank when top-p
                                        is active (Sampler.swift:44-51)                 */
#define STRIM_FLAG_SCORE_NO_LSE 4u   /* Gumbel score = logit + g (categorical, Sampler)
                                        instead of log-prob + g (SpecSampling)          */
#define STRIM_FLAG_SAMPLER_COMPAT 7u /* all three: the non-MTP Sampler.sample          */

/* One per row. With the extensions at their defaults (strim_default_params) a row
 * reproduces the reference exactly: they are no-ops. Chain order: penalties -> mask -> /T -> min-p -> top-k -> top-p
 * -> draw. 48 bytes, naturally aligned. */
typedef struct strim_sampling_params {
  float temperature;        /* <= 0: greedy argmax (GenParams.isGreedy, EngineAPI.swift:66) */
  int32_t top_k;            /* 0 = off; >= V = off                                          */
  float top_p;              /* (0,1]; drop a token iff the mass strictly before it > top_p  */
  float min_p;              /* [0,1]; 0 = off. Drop p < min_p * p_max (extension)           */
  float repetition_penalty; /* > 0; 1 = off. In-history logit l: l>0 ? l/r : l*r (ext.)     */
  float presence_penalty;   /* 0 = off. In-history: l -= presence (extension)               */
  float frequency_penalty;  /* 0 = off. In-history: l -= frequency * count (extension)      */
  uint32_t flags;           /* STRIM_FLAG_*                                                 */
  uint64_t seed;            /* Philox key base (Sampler.seed)                               */
  uint64_t position;        /* output position (SpecStream.sampleIndex)                      */
} strim_sampling_params;

typedef struct strim_ctx strim_ctx;

/* Fill *p with T=1, top_k=0, top_p=1 and every extension off (plain sampling of the
 * reference's SamplingConfig with its topK / topP defaults, SpecSampling.swift:12; the
 * engine's GenParams defaults to T=0, greedy, EngineAPI.swift:59). Host. */
void strim_default_params(strim_sampling_params* p);

/* Validate n HOST param structs the way the engine consumes GenParams: temperature
 * finite (T <= 0 is greedy, GenParams.isGreedy, EngineAPI.swift:66), top_p in (0,1],
 * top_k >= 0 (ChatRequest.swift:148-161), plus the extensions (min_p in [0,1],
 * repetition > 0, finite penalties, known flags). Returns STRIM_OK or STRIM_EINVAL. */
int strim_check_params(const strim_sampling_params* host_params, int32_t n);

/* Create a context on `device` for up to max_rows rows of up to max_vocab tokens per
 * call (max_vocab <= 2^20). Allocates scratch once (hipMalloc); no call below allocates.
 * Calls with more rows than max_rows are processed in groups; a call with V above
 * max_vocab returns STRIM_ECAPACITY. */
int strim_ctx_create(strim_ctx** out, int32_t device, int32_t max_rows, int32_t max_vocab);
int strim_ctx_destroy(strim_ctx* ctx);

/* Sample one token per row from logits [B][V] (row r at logits + r*row_stride elements).
 *   params      HOST [B], read during the call (validated like strim_check_params; an
 *               invalid row fails the call with STRIM_EINVAL before any launch)
 *   mask_words  device [B][mask_stride] uint32 or NULL. Token i allowed iff bit (i & 31)
 *               of word (i >> 5) is set — the byte layout of the reference's UInt64
 *               bitset (GrammarVocab.swift:77-86) on little-endian hosts.
 *   history     device [B][H] int32 token ids or NULL; history_len device [B] (<= H) or
 *               NULL (= H). Ids outside [0,V) are ignored. Feeds the penalties.
 *   noise       see STRIM_NOISE_*.
 *   out_ids     device [B]; -1 on a row error.
 *   out_status  device [B] or NULL; STRIM_OK or a negative STRIM_E* per row
 *               (EEMPTY, ENONFINITE).
 *   out_probs   device [B][V] float or NULL: the processed distribution (validation).
 * Replaces Sampler.sample / SpecSampling.sample (Sampler.swift:34-54,
 * SpecSampling.swift:109-116) and the batched pick loop (EngineCore.swift:998-1002). */
int strim_sample(strim_ctx* ctx, void* stream, const void* logits, int32_t dtype, int32_t B,
                 int32_t V, int64_t row_stride, const strim_sampling_params* params,
                 const uint32_t* mask_words, int64_t mask_stride, const int32_t* history,
                 const int32_t* history_len, int32_t H, int32_t noise_mode, const float* noise,
                 int32_t* out_ids, int32_t* out_status, float* out_probs);

/* strim_sample without a context, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It has no counterpart
 * in the reference. Arguments as strim_sample, without out_probs. Its scratch is a fixed
 * device array inside the library, one per GPU (held until the process ends), so the call
 * allocates nothing: V above STRIM_NOALLOC_MAX_VOCAB returns STRIM_ECAPACITY, and B rows
 * run in groups of STRIM_NOALLOC_MAX_ROWS. Every call on a GPU shares that GPU's array:
 * calls that overlap in time on one GPU (two streams, two threads) race, so issue them on
 * one stream. Runs on the current device. */
#define STRIM_NOALLOC_MAX_ROWS 32
#define STRIM_NOALLOC_MAX_VOCAB 262144
int strim_sample_noalloc(void* stream, const void* logits, int32_t dtype, int32_t B, int32_t V,
                         int64_t row_stride, const strim_sampling_params* params,
                         const uint32_t* mask_words, int64_t mask_stride,
                         const int32_t* history, const int32_t* history_len, int32_t H,
                         int32_t noise_mode, const float* noise, int32_t* out_ids,
                         int32_t* out_status);

/* Speculative verification of k drafts for B independent sequences.
 *   target_logits [B][k+1][V] (row j = target distribution after the pending token and
 *                 drafts[0..j)), dtype as strim_sample.
 *   draft_logits  [B][k][Vd] (same dtype) or NULL. NULL: the draft is one-hot (the
 *                 reference's argmax drafter, SpecSampling.swift:17-22). Otherwise the
 *                 draft distribution q = softmax(draft_logits / T) over the draft vocab,
 *                 mapped to full-vocab ids by draft_to_full.
 *   draft_to_full [Vd] strictly ascending ids in [0, V) (Weights.swift:196-209); used
 *                 only with draft_logits (then 0 < Vd <= V). A table that is not strictly
 *                 ascending, or a sampled row's draft that is not in it, gives that
 *                 sequence STRIM_EINVAL in out_status (accepted 0, token -1).
 *   draft_tokens  [B][k] full-vocab ids.
 *   params        HOST [B], as strim_sample.
 *   mask_words    [B][k+1][mask_stride] or NULL (VerifyConstraint, TokenMask.swift:7-12).
 *   history       as strim_sample; row j additionally counts drafts[0..j).
 *   noise         ICDF [B][k+1][2]; GUMBEL [B][k+1][V+1]; NULL = Philox at positions
 *                 params[b].position + j (SpecSampling.swift:98).
 *   out_accepted  [B] leading accepted drafts n; out_token [B] the token decided at row n
 *                 (residual at the first rejection, bonus sample after k accepts).
 *   out_row_accept [B][k] / out_row_token [B][k+1] or NULL: per-row outcomes
 *                 (SpecSampling.rowOutcome). out_status [B] or NULL. With general-q
 *                 drafts and Gumbel noise, out_row_token NULL lets the call draw the
 *                 residual of each sequence's first rejected row only (the rows the
 *                 result depends on); out_row_accept is filled for every row either way.
 * T <= 0 rows use the greedy rule: accept while argmax == draft (SpecStream.swift:269-273). */
int strim_verify(strim_ctx* ctx, void* stream, const void* target_logits, int32_t dtype,
                 int32_t B, int32_t k, int32_t V, const void* draft_logits, int32_t Vd,
                 const int32_t* draft_to_full, const int32_t* draft_tokens,
                 const strim_sampling_params* params, const uint32_t* mask_words,
                 int64_t mask_stride, const int32_t* history, const int32_t* history_len,
                 int32_t H, int32_t noise_mode, const float* noise, int32_t* out_accepted,
                 int32_t* out_token, int32_t* out_row_accept, int32_t* out_row_token,
                 int32_t* out_status);

/* out[r][i] = allowed(r,i) ? float(logits[r][i]) : -inf, float32 [R][V] (maskLogits,
 * TokenMask.swift:15-17). mask_words as strim_sample (NULL = all allowed). */
int strim_mask_logits(void* stream, const void* logits, int32_t dtype, int32_t R, int32_t V,
                      int64_t row_stride, const uint32_t* mask_words, int64_t mask_stride,
                      float* out);

/* Draft-side map: out[r] = draft_to_full[argmax_j draft_logits[r][j]] (first max), or
 * argmax itself when draft_to_full is NULL (MTP.swift:104-111,120-125). */
int strim_draft_argmax(void* stream, const void* draft_logits, int32_t dtype, int32_t R,
                       int32_t Vd, int64_t row_stride, const int32_t* draft_to_full,
                       int32_t* out);

/* Producer of the logits (the step before the path): the decode step's final RMSNorm
 * and dense lm_head linear (QwenModel.swift:202-212; store.rmsNorm and store.linear,
 * Weights.swift:244-255,270-273), written as the bf16 logits strim_sample and
 * strim_verify read. hidden: bf16 [B][hidden_stride]; norm_weight: bf16 [K], or NULL when
 * hidden is already normalised; xn: bf16 [B][K] workspace for the normalised rows (unused
 * when norm_weight is NULL); lm_head: bf16 [V][lm_head_stride]; out_logits: bf16
 * [B][out_stride]. xn[b][k] = bf16(w[k] * bf16(x[b][k] / sqrt(mean_k x^2 + eps))) (squares
 * summed in double), logits[b][v] = bf16(sum_k xn[b][k] lm_head[v][k]) accumulated in
 * float32 on MFMA. B in [1, 64]; K a positive multiple of 256; hidden, xn, lm_head and
 * their row strides 16-byte aligned. Sizes or alignment out of range: STRIM_EINVAL. */
int strim_head_logits(void* stream, const void* hidden, int64_t hidden_stride, int32_t B,
                      int32_t K, const void* norm_weight, float eps, void* xn,
                      const void* lm_head, int64_t lm_head_stride, int32_t V, void* out_logits,
                      int64_t out_stride);

/* Hidden -> greedy token: the producer above (same operands and checks) with the pick
 * fused into it, for rows the reference decides by argmax alone (T <= 0 with no
 * penalties, no mask and no filters: Sampler.sample / SpecSampling's T -> 0 case,
 * SpecSampling.swift:70-88). The GEMV's epilogue writes each 128-row vocabulary tile's
 * first maximum per batch row (as bf16 logits, as strim_sample reads them) and one small
 * launch merges them, so the logits are not read back; out_logits may be NULL (then they
 * are not written at all). out_ids [B] = the first maximum's id, out_status [B] (or NULL)
 * = STRIM_OK, STRIM_ENONFINITE (a NaN or +inf logit) or STRIM_EEMPTY (every logit -inf),
 * with out_ids -1 on an error row: strim_sample's result for such a row. The tile maxima
 * use ctx's scratch (B <= max_rows and V <= max_vocab, else STRIM_ECAPACITY); calls on
 * one ctx run in stream order. */
int strim_head_greedy(strim_ctx* ctx, void* stream, const void* hidden, int64_t hidden_stride,
                      int32_t B, int32_t K, const void* norm_weight, float eps, void* xn,
                      const void* lm_head, int64_t lm_head_stride, int32_t V, void* out_logits,
                      int64_t out_stride, int32_t* out_ids, int32_t* out_status);

/* ---- per-kernel timing -------------------------------------------------------------
 * Counterpart of the reference's fenced per-region GPU timer OpTimer
 * (Sources/StrimCore/OpTimer.swift:1-60). While profiling is on, every kernel a call
 * launches carries a pair of HIP events bound to its dispatch's own start and end
 * timestamps (hipExtLaunchKernel), so the elapsed time is the kernel's execution alone;
 * strim_profile_end synchronises, sums the elapsed time per kernel and turns profiling
 * off. Profiling allocates its events in strim_profile_begin, never in the calls it
 * times. Do not profile calls that are being captured into a graph. */
#define STRIM_KERNEL_COUNT 8 /* stream, finalize, gfinal, final, probs, verify_combine,
                                qprep (no launches: the draft distributions run in the
                                stream launch), qres (the launches of the residual draw
                                of unfiltered general-q rows, timed together) */
int strim_profile_begin(strim_ctx* ctx, int32_t max_launches);
int strim_profile_end(strim_ctx* ctx, double* total_ms /* [STRIM_KERNEL_COUNT] */,
                      int64_t* launches /* [STRIM_KERNEL_COUNT] */);
const char* strim_kernel_name(int32_t kernel);

/* Library version string (static storage). */
const char* strim_version(void);

#ifdef __cplusplus
}
#endif

#endif /* STRIM_SAMPLER_H */
