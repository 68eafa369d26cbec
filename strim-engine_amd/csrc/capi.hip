// capi.hip — the C ABI (include/strim_sampler.h): context, validation, launches.
//
// A call is a fixed sequence of stream-ordered launches over caller-owned device
// buffers; the context's scratch is allocated once at strim_ctx_create and every
// per-call counter is reset by the kernel that consumes it, so no call allocates,
// copies or memsets (the sequence can be captured in a HIP graph).
#include <math.h>
#include <string.h>

#include "kernels.hpp"

namespace strim {
__global__ void k_stats(Args a);
__global__ void k_hist(Args a);
__global__ void k_collect(Args a);
__global__ void k_final(Args a);
__global__ void k_probs(Args a);
__global__ void k_verify_combine(Args a);
__global__ void k_mask_logits(const void* logits, int dtype, int V, int64_t row_stride,
                              const uint32_t* mask, int64_t mask_stride, float* out);
__global__ void k_draft_argmax(const void* logits, int dtype, int Vd, int64_t row_stride,
                               const int32_t* table, int32_t* out);
}  // namespace strim

using namespace strim;

struct strim_ctx {
  int32_t device;
  int32_t max_rows;
  int32_t max_vocab;
  void* base;
  size_t bytes;
  Scratch s;
};

namespace {

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? STRIM_OK : STRIM_EHIP;
}

// Runs `fn` with ctx->device current, restoring the caller's device afterwards.
template <typename F>
int on_device(int32_t device, F fn) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return STRIM_EHIP;
  if (cur != device && hipSetDevice(device) != hipSuccess) return STRIM_EHIP;
  int rc = fn();
  if (cur != device) (void)hipSetDevice(cur);
  return rc;
}

bool dtype_ok(int32_t d) { return d == STRIM_DTYPE_F32 || d == STRIM_DTYPE_BF16; }

int32_t vec_ok(const void* p, int64_t row_stride, int32_t dtype) {
  const int64_t per16 = dtype == STRIM_DTYPE_BF16 ? 8 : 4;
  return ((uintptr_t)p % 16 == 0) && (row_stride % per16 == 0) ? 1 : 0;
}

// The launch sequence shared by strim_sample and strim_verify.
int run_chain(strim_ctx* ctx, hipStream_t st, Args& a, bool probs) {
  const int R = a.R, W = a.W;
  const dim3 grid_rc((unsigned)(R * W));
  hipLaunchKernelGGL(k_stats, grid_rc, dim3(TPB), 0, st, a);
  hipLaunchKernelGGL(k_hist, grid_rc, dim3(TPB), 0, st, a);
  hipLaunchKernelGGL(k_collect, grid_rc, dim3(TPB), 0, st, a);
  hipLaunchKernelGGL(k_final, dim3((unsigned)R), dim3(FIN_T), 0, st, a);
  if (probs) hipLaunchKernelGGL(k_probs, grid_rc, dim3(TPB), 0, st, a);
  (void)ctx;
  return launch_status();
}

}  // namespace

extern "C" {

const char* strim_version(void) { return "strim-select-mi355x 0.1 (gfx950)"; }

void strim_default_params(strim_sampling_params* p) {
  if (!p) return;
  memset(p, 0, sizeof(*p));
  p->temperature = 1.0f;
  p->top_k = 0;
  p->top_p = 1.0f;
  p->min_p = 0.0f;
  p->repetition_penalty = 1.0f;
  p->presence_penalty = 0.0f;
  p->frequency_penalty = 0.0f;
  p->flags = 0u;
  p->seed = 0u;
  p->position = 0u;
}

// ChatRequest.parse (Sources/StrimServer/ChatRequest.swift:150-160): temperature >= 0,
// top_p in (0,1], top_k >= 0; plus the extension ranges.
int strim_check_params(const strim_sampling_params* hp, int32_t n) {
  if (!hp || n < 0) return STRIM_EINVAL;
  for (int32_t i = 0; i < n; ++i) {
    const strim_sampling_params& p = hp[i];
    if (!(p.temperature >= 0.0f) || isinf(p.temperature)) return STRIM_EINVAL;
    if (!(p.top_p > 0.0f && p.top_p <= 1.0f)) return STRIM_EINVAL;
    if (p.top_k < 0) return STRIM_EINVAL;
    if (!(p.min_p >= 0.0f && p.min_p <= 1.0f)) return STRIM_EINVAL;
    if (!(p.repetition_penalty > 0.0f) || isinf(p.repetition_penalty)) return STRIM_EINVAL;
    if (!isfinite(p.presence_penalty) || !isfinite(p.frequency_penalty)) return STRIM_EINVAL;
    if (p.flags & ~STRIM_FLAG_SAMPLER_COMPAT) return STRIM_EINVAL;
  }
  return STRIM_OK;
}

int strim_ctx_create(strim_ctx** out, int32_t device, int32_t max_rows, int32_t max_vocab) {
  // the fixed-point histogram (2^40 per token) must fit in 64 bits: V < 2^24
  if (!out || max_rows <= 0 || max_vocab <= 0 || max_rows > (1 << 20) ||
      max_vocab >= (1 << 24))
    return STRIM_EINVAL;
  *out = nullptr;
  strim_ctx* ctx = new (std::nothrow) strim_ctx();
  if (!ctx) return STRIM_ENOMEM;
  ctx->device = device;
  ctx->max_rows = max_rows;
  ctx->max_vocab = max_vocab;
  const int32_t wmax = (max_vocab + CHUNK - 1) / CHUNK;
  const size_t R = (size_t)max_rows;
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    size_t o = off;
    off = align_up(off + bytes, 256);
    return o;
  };
  const size_t o_cstat = carve(R * wmax * sizeof(ChunkStat));
  const size_t o_rs = carve(R * sizeof(RowState));
  const size_t o_cs = carve(R * sizeof(uint32_t));
  const size_t o_ch = carve(R * sizeof(uint32_t));
  const size_t o_hc = carve(R * NBINS * sizeof(uint32_t));
  const size_t o_hm = carve(R * NBINS * sizeof(unsigned long long));
  const size_t o_cand = carve(R * CAP * sizeof(Cand));
  const size_t o_nc = carve(R * sizeof(uint32_t));
  const size_t o_ct = carve(R * wmax * sizeof(ChunkTop));
  ctx->bytes = off;
  int rc = on_device(device, [&]() -> int {
    if (hipMalloc(&ctx->base, ctx->bytes) != hipSuccess) return STRIM_ENOMEM;
    if (hipMemset(ctx->base, 0, ctx->bytes) != hipSuccess) return STRIM_EHIP;
    if (hipDeviceSynchronize() != hipSuccess) return STRIM_EHIP;
    return STRIM_OK;
  });
  if (rc != STRIM_OK) {
    if (ctx->base) (void)hipFree(ctx->base);
    delete ctx;
    return rc;
  }
  char* b = (char*)ctx->base;
  ctx->s.cstat = (ChunkStat*)(b + o_cstat);
  ctx->s.rs = (RowState*)(b + o_rs);
  ctx->s.cnt_stats = (uint32_t*)(b + o_cs);
  ctx->s.cnt_hist = (uint32_t*)(b + o_ch);
  ctx->s.hcnt = (uint32_t*)(b + o_hc);
  ctx->s.hmass = (unsigned long long*)(b + o_hm);
  ctx->s.cand = (Cand*)(b + o_cand);
  ctx->s.ncand = (uint32_t*)(b + o_nc);
  ctx->s.ctop = (ChunkTop*)(b + o_ct);
  ctx->s.wmax = wmax;
  *out = ctx;
  return STRIM_OK;
}

int strim_ctx_destroy(strim_ctx* ctx) {
  if (!ctx) return STRIM_EINVAL;
  int rc = on_device(ctx->device, [&]() -> int {
    if (ctx->base && hipFree(ctx->base) != hipSuccess) return STRIM_EHIP;
    return STRIM_OK;
  });
  delete ctx;
  return rc;
}

int strim_sample(strim_ctx* ctx, void* stream, const void* logits, int32_t dtype, int32_t B,
                 int32_t V, int64_t row_stride, const strim_sampling_params* params,
                 const uint32_t* mask_words, int64_t mask_stride, const int32_t* history,
                 const int32_t* history_len, int32_t H, int32_t noise_mode, const float* noise,
                 int32_t* out_ids, int32_t* out_status, float* out_probs) {
  if (!ctx || !logits || !params || !out_ids || !dtype_ok(dtype)) return STRIM_EINVAL;
  if (B <= 0 || B > ctx->max_rows || V <= 0 || V > ctx->max_vocab || row_stride < V)
    return STRIM_EINVAL;
  if (mask_words && mask_stride < ((int64_t)V + 31) / 32) return STRIM_EINVAL;
  if (H < 0 || (H > 0 && !history) || (history && H == 0)) return STRIM_EINVAL;
  if (noise_mode != STRIM_NOISE_ICDF && noise_mode != STRIM_NOISE_GUMBEL) return STRIM_EINVAL;
  Args a;
  memset(&a, 0, sizeof(a));
  a.logits = logits;
  a.row_stride = row_stride;
  a.dtype = dtype;
  a.vec_ok = vec_ok(logits, row_stride, dtype);
  a.R = B;
  a.V = V;
  a.W = (V + CHUNK - 1) / CHUNK;
  a.B = B;
  a.k = 0;
  a.verify = 0;
  a.xcd_map = (B % 8 == 0) ? 1 : 0;
  a.params = params;
  a.mask = mask_words;
  a.mask_stride = mask_stride;
  a.hist = history;
  a.hist_len = history ? history_len : nullptr;
  a.H = H;
  a.noise_mode = noise_mode;
  a.noise = noise;
  a.noise_stride = noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V + 1 : 2;
  a.s = ctx->s;
  a.out_ids = out_ids;
  a.out_status = out_status;
  a.out_probs = out_probs;
  return on_device(ctx->device, [&]() { return run_chain(ctx, (hipStream_t)stream, a, out_probs != nullptr); });
}

int strim_verify(strim_ctx* ctx, void* stream, const void* target_logits, int32_t dtype,
                 int32_t B, int32_t k, int32_t V, const void* draft_logits, int32_t Vd,
                 const int32_t* draft_to_full, const int32_t* draft_tokens,
                 const strim_sampling_params* params, const uint32_t* mask_words,
                 int64_t mask_stride, const int32_t* history, const int32_t* history_len,
                 int32_t H, int32_t noise_mode, const float* noise, int32_t* out_accepted,
                 int32_t* out_token, int32_t* out_row_accept, int32_t* out_row_token,
                 int32_t* out_status) {
  if (!ctx || !target_logits || !params || !out_accepted || !out_token || !dtype_ok(dtype))
    return STRIM_EINVAL;
  if (B <= 0 || k < 0 || k > 64 || V <= 0 || V > ctx->max_vocab) return STRIM_EINVAL;
  if ((int64_t)B * (k + 1) > ctx->max_rows) return STRIM_EINVAL;
  if (k > 0 && !draft_tokens) return STRIM_EINVAL;
  if (draft_logits) return STRIM_EINVAL;  // general-q drafts: not supported yet
  (void)Vd;
  (void)draft_to_full;
  if (mask_words && mask_stride < ((int64_t)V + 31) / 32) return STRIM_EINVAL;
  if (H < 0 || (H > 0 && !history) || (history && H == 0)) return STRIM_EINVAL;
  if (noise_mode != STRIM_NOISE_ICDF && noise_mode != STRIM_NOISE_GUMBEL) return STRIM_EINVAL;
  Args a;
  memset(&a, 0, sizeof(a));
  a.logits = target_logits;
  a.row_stride = V;
  a.dtype = dtype;
  a.vec_ok = vec_ok(target_logits, V, dtype);
  a.R = B * (k + 1);
  a.V = V;
  a.W = (V + CHUNK - 1) / CHUNK;
  a.B = B;
  a.k = k;
  a.verify = 1;
  a.xcd_map = (a.R % 8 == 0) ? 1 : 0;
  a.params = params;
  a.mask = mask_words;
  a.mask_stride = mask_stride;
  a.hist = history;
  a.hist_len = history ? history_len : nullptr;
  a.H = H;
  a.drafts = draft_tokens;
  a.noise_mode = noise_mode;
  a.noise = noise;
  a.noise_stride = noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V + 1 : 2;
  a.s = ctx->s;
  a.out_accepted = out_accepted;
  a.out_token = out_token;
  a.out_row_accept = out_row_accept;
  a.out_row_token = out_row_token;
  a.out_status = out_status;
  return on_device(ctx->device, [&]() -> int {
    hipStream_t st = (hipStream_t)stream;
    int rc = run_chain(ctx, st, a, false);
    if (rc != STRIM_OK) return rc;
    hipLaunchKernelGGL(k_verify_combine, dim3((unsigned)((B + 63) / 64)), dim3(64), 0, st, a);
    return launch_status();
  });
}

int strim_mask_logits(void* stream, const void* logits, int32_t dtype, int32_t R, int32_t V,
                      int64_t row_stride, const uint32_t* mask_words, int64_t mask_stride,
                      float* out) {
  if (!logits || !out || !dtype_ok(dtype) || R <= 0 || V <= 0 || row_stride < V)
    return STRIM_EINVAL;
  if (mask_words && mask_stride < ((int64_t)V + 31) / 32) return STRIM_EINVAL;
  const dim3 grid((unsigned)((V + 1023) / 1024), (unsigned)R);
  hipLaunchKernelGGL(k_mask_logits, grid, dim3(256), 0, (hipStream_t)stream, logits, dtype, V,
                     row_stride, mask_words, mask_stride, out);
  return launch_status();
}

int strim_draft_argmax(void* stream, const void* draft_logits, int32_t dtype, int32_t R,
                       int32_t Vd, int64_t row_stride, const int32_t* draft_to_full,
                       int32_t* out) {
  if (!draft_logits || !out || !dtype_ok(dtype) || R <= 0 || Vd <= 0 || row_stride < Vd)
    return STRIM_EINVAL;
  hipLaunchKernelGGL(k_draft_argmax, dim3((unsigned)R), dim3(256), 0, (hipStream_t)stream,
                     draft_logits, dtype, Vd, row_stride, draft_to_full, out);
  return launch_status();
}

}  // extern "C"
