// capi.hip — the C ABI (include/strim_sampler.h): context, validation, launches.
//
// A call is a fixed sequence of stream-ordered launches over caller-owned device
// buffers; the context's scratch is allocated once at strim_ctx_create and every
// per-call counter is reset by the kernel that consumes it, so no call allocates,
// copies or memsets (the sequence can be captured in a HIP graph).
#include <math.h>
#include <string.h>

#include <mutex>

#include "stream.hpp"

namespace strim {
hipError_t launch_finalize(const Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1);
hipError_t launch_gfinal(const Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1);
hipError_t launch_head(const void* hidden, int64_t hidden_stride, int B, int K,
                       const void* norm_w, float eps, void* xn, const void* W, int64_t w_stride,
                       int V, void* out, int64_t out_stride, bool vo, hipStream_t st,
                       uint2* tbest, int32_t* out_ids, int32_t* out_status);
__global__ void k_final(Args a);
__global__ void k_probs(Args a);
__global__ void k_verify_combine(Args a);
__global__ void k_qhist(Args a);
__global__ void k_qpick(Args a);
__global__ void k_qcollect(Args a);
__global__ void k_qfinal(Args a);
hipError_t launch_qgumbel(const Args& a, bool combine, dim3 grid, hipStream_t st, hipEvent_t e0,
                          hipEvent_t e1);
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
  // per-kernel event profiling (off unless strim_profile_begin)
  int32_t prof_on = 0;
  int32_t prof_cap = 0;
  int32_t prof_n = 0;
  hipEvent_t* prof_ev = nullptr;  // [cap][2]
  int32_t* prof_kind = nullptr;   // [cap]
};

namespace {

constexpr size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Byte offsets of the scratch buffers of R rows of up to max_vocab tokens, each 256-byte
// aligned. The general-q verify buffers (dbits .. qarr) are sized only when `verify`.
struct ScratchLayout {
  size_t cstat, slot, part, rs, cand, nc, dbits, wrank, qpart, qhc, qhm, qst, qpp, qarr, lat,
      bytes;
};
constexpr ScratchLayout scratch_layout(size_t R, size_t max_vocab, bool verify) {
  const size_t wmax = (max_vocab + CHUNK - 1) / CHUNK;
  const size_t words = (max_vocab + 31) / 32;
  const size_t RQ = verify ? (R < (size_t)MAXP ? R : (size_t)MAXP) : 0;  // per group
  const size_t RV = verify ? R : 0;
  ScratchLayout L{};
  size_t off = 0;
  L.cstat = off; off = align_up(off + R * wmax * sizeof(ChunkStat), 256);
  L.slot = off; off = align_up(off + R * wmax * SLOT * sizeof(Cand), 256);
  L.part = off; off = align_up(off + R * wmax * sizeof(ChunkPart), 256);
  L.rs = off; off = align_up(off + R * sizeof(RowState), 256);
  L.cand = off; off = align_up(off + R * CAP * sizeof(Cand), 256);
  L.nc = off; off = align_up(off + R * sizeof(uint32_t), 256);
  L.dbits = off; off = align_up(off + (verify ? words : 0) * sizeof(uint32_t), 256);
  L.wrank = off; off = align_up(off + (verify ? words : 0) * sizeof(uint32_t), 256);
  L.qpart = off; off = align_up(off + RQ * wmax * sizeof(unsigned long long), 256);
  L.qhc = off; off = align_up(off + RQ * wmax * QNB * sizeof(uint32_t), 256);
  L.qhm = off; off = align_up(off + RQ * wmax * QNB * sizeof(unsigned long long), 256);
  L.qst = off; off = align_up(off + RV * sizeof(QStat), 256);
  L.qpp = off; off = align_up(off + RQ * QSPLIT * sizeof(QPart), 256);
  L.qarr = off; off = align_up(off + RQ * sizeof(uint32_t), 256);
  L.lat = off; off = align_up(off + R * wmax * NBW * sizeof(unsigned long long), 256);
  L.bytes = off;
  return L;
}

// The scratch pointers of a layout placed at device address `base` (the general-q
// buffers are null when the layout has none).
Scratch scratch_at(char* base, const ScratchLayout& L, size_t max_vocab, bool verify) {
  Scratch s{};
  s.cstat = (ChunkStat*)(base + L.cstat);
  s.slot = (Cand*)(base + L.slot);
  s.part = (ChunkPart*)(base + L.part);
  s.rs = (RowState*)(base + L.rs);
  s.cand = (Cand*)(base + L.cand);
  s.ncand = (uint32_t*)(base + L.nc);
  s.lat = (unsigned long long*)(base + L.lat);
  if (verify) {
    s.dbits = (uint32_t*)(base + L.dbits);
    s.wrank = (uint32_t*)(base + L.wrank);
    s.qpart = (unsigned long long*)(base + L.qpart);
    s.qhc = (uint32_t*)(base + L.qhc);
    s.qhm = (unsigned long long*)(base + L.qhm);
    s.qst = (QStat*)(base + L.qst);
    s.qpp = (QPart*)(base + L.qpp);
    s.qarr = (uint32_t*)(base + L.qarr);
  }
  s.wmax = (int32_t)((max_vocab + CHUNK - 1) / CHUNK);
  return s;
}

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
size_t dtype_size(int32_t d) { return d == STRIM_DTYPE_BF16 ? 2 : 4; }

int32_t vec_ok(const void* p, int64_t row_stride, int32_t dtype) {
  const int64_t per16 = dtype == STRIM_DTYPE_BF16 ? 8 : 4;
  return ((uintptr_t)p % 16 == 0) && (row_stride % per16 == 0) ? 1 : 0;
}

enum KernelId {
  KID_STREAM = 0, KID_FINALIZE, KID_GFINAL, KID_FINAL, KID_PROBS, KID_COMBINE, KID_QPREP,
  KID_QRES
};
const char* const kKernelNames[STRIM_KERNEL_COUNT] = {
    "k_stream", "k_finalize", "k_gfinal", "k_final", "k_probs", "k_verify_combine", "k_qprep",
    "k_qres"};

// Runs `launch(e0, e1)`: with profiling on, e0/e1 are the next event pair, which the
// launch binds to its dispatch's timestamps; otherwise both are null.
template <typename F>
void timed(strim_ctx* ctx, int kind, F launch) {
  if (ctx && ctx->prof_on && ctx->prof_n < ctx->prof_cap) {
    const int i = ctx->prof_n++;
    ctx->prof_kind[i] = kind;
    launch(ctx->prof_ev[2 * i], ctx->prof_ev[2 * i + 1]);
  } else {
    launch(nullptr, nullptr);
  }
}

// Launches the k_stream variant for the call: dtype, alignment, whether any row has
// penalties, whether a mask is given (unaligned calls take the penalties object, whose
// unaligned variant checks penalties and mask per row).
// Segments per thread of the k_stream launch: one (512-thread workgroups) while the
// launch is small and its time is latency, four (128 threads) once the rows alone fill
// the chip and instructions per token decide. (Eight segments in one-wave workgroups
// measured slower at B=64: 11.1 against 9.9 us.)
constexpr int LARGE_ROWS = 32;
int stream_threads(int rows) { return rows >= LARGE_ROWS ? stpb<4>() : stpb<1>(); }

hipError_t launch_stream(const Args& a, dim3 grid, hipStream_t st, bool any_pen, hipEvent_t e0,
                         hipEvent_t e1) {
  // history counts: none, 16-bit when no count can reach 65,536 (the history length plus
  // the draft prefix bound every count), else 32-bit; unaligned calls take the 32-bit
  // object, whose unaligned variant checks penalties and mask per row
  const int pen = a.vec_ok == 0 ? 1 : !any_pen ? 0 : (int64_t)a.H + a.k < 65536 ? 2 : 1;
  const bool big = a.R >= LARGE_ROWS;
#define STRIM_GROUP(DT, PEN, SSEG) launch_stream_group<DT, PEN, SSEG>(a, grid, st, e0, e1)
#define STRIM_SEGS(DT, PEN) (big ? STRIM_GROUP(DT, PEN, 4) : STRIM_GROUP(DT, PEN, 1))
#define STRIM_PENS(DT) \
  (pen == 2 ? STRIM_SEGS(DT, 2) : pen == 1 ? STRIM_SEGS(DT, 1) : STRIM_SEGS(DT, 0))
  return a.dtype == STRIM_DTYPE_BF16 ? STRIM_PENS(STRIM_DTYPE_BF16) : STRIM_PENS(STRIM_DTYPE_F32);
#undef STRIM_PENS
#undef STRIM_SEGS
#undef STRIM_GROUP
}

bool nofilter(const strim_sampling_params& p, int32_t V) {
  return !(p.top_k > 0 && p.top_k < V) && !(p.min_p > 0.0f) && !(p.top_p < 1.0f);
}

// The launch sequence of one row group: k_stream, then k_finalize for the greedy, fast
// and unfiltered Gumbel rows (and the marking of general-q draft rows) and k_gfinal for
// the general rows, each launched only when some row of the group needs it; general-q
// verify groups add the residual draw and k_final.
int run_group(strim_ctx* ctx, hipStream_t st, Args& a, int nb, bool probs,
              bool* combined = nullptr) {
  if (combined) *combined = false;
  bool need_fin = false, need_gfin = false, any_pen = false;
  const bool gq = a.verify && a.dlog != nullptr && a.k > 0;  // general-q draft rows
  for (int i = 0; i < nb; ++i) {
    const strim_sampling_params& q = a.p[i];
    if ((q.repetition_penalty != 1.0f || q.presence_penalty != 0.0f ||
         q.frequency_penalty != 0.0f) && (a.hist != nullptr || a.verify))
      any_pen = true;
    // the sample row, or a verify sequence's bonus row (and its draft rows without
    // general-q drafts)
    if (gfinal_row(q, a.V, a.noise_mode, false)) need_gfin = true;
    else need_fin = true;
  }
  if (gq) need_fin = true;
  // k_final decides the general-q draft rows left to the exact resolution: the filtered
  // ones, and (icdf draws) those whose residual bin overflows
  bool need_final = gq && a.noise_mode == STRIM_NOISE_ICDF;
  if (gq)
    for (int i = 0; i < nb; ++i) {
      const strim_sampling_params& q = a.p[i];
      if ((q.top_k > 0 && q.top_k < a.V) || q.top_p < 1.0f || q.min_p > 0.0f) need_final = true;
    }
  // rows per XCD when every chunk reads a history and no general row's cost depends on
  // its mask density (measured: -25 % of k_stream's HBM bytes at cfg2 at equal time;
  // general rows of unequal density 0.75 us slower when each XCD holds whole rows)
  a.xmap = any_pen && !need_gfin && !gq ? 1 : 0;
  a.gen = 0;
  for (int i = 0; i < nb; ++i)
    if (row_class(a.p[i], a.V) == CLS_GENERAL) a.gen = 1;
  const dim3 grid_rc((unsigned)a.W, (unsigned)a.R);
  // (general-q verify: the draft distributions' workgroups in extra grid rows)
  const dim3 grid_st((unsigned)a.W, (unsigned)(a.R + (a.nqprep + a.W - 1) / a.W));
  hipError_t e = hipSuccess;
  auto keep = [&e](hipError_t x) { if (e == hipSuccess) e = x; };
  timed(ctx, KID_STREAM,
        [&](hipEvent_t e0, hipEvent_t e1) { keep(launch_stream(a, grid_st, st, any_pen, e0, e1)); });
  if (need_fin)
    timed(ctx, KID_FINALIZE, [&](hipEvent_t e0, hipEvent_t e1) {
      keep(launch_finalize(a, st, e0, e1));
    });
  if (need_gfin)
    timed(ctx, KID_GFINAL, [&](hipEvent_t e0, hipEvent_t e1) {
      keep(launch_gfinal(a, st, e0, e1));
    });
  if (a.verify && a.dlog != nullptr) {
    // the residual draw of unfiltered general-q rows (rows in other phases return)
    const dim3 grid_r((unsigned)a.R);
    timed(ctx, KID_QRES, [&](hipEvent_t e0, hipEvent_t e1) {
      if (a.noise_mode == STRIM_NOISE_ICDF) {
        keep(launch_args((const void*)k_qhist, grid_rc, dim3(TPB), a, st, e0, nullptr));
        keep(launch_args((const void*)k_qpick, grid_r, dim3(QNB), a, st, nullptr, nullptr));
        keep(launch_args((const void*)k_qcollect, grid_rc, dim3(TPB), a, st, nullptr, nullptr));
        keep(launch_args((const void*)k_qfinal, grid_r, dim3(FIN_T), a, st, nullptr, e1));
      } else {
        const dim3 grid_q = a.qskip ? dim3((unsigned)a.W, (unsigned)a.B) : grid_rc;
        // the last workgroup of each sequence picks its rows; with nothing after it, it
        // also runs the verify combine
        const bool comb = combined != nullptr && !need_final && !probs;
        keep(launch_qgumbel(a, comb, grid_q, st, e0, e1));
        if (comb) *combined = true;
      }
    });
  }
  if (need_final)
    timed(ctx, KID_FINAL, [&](hipEvent_t e0, hipEvent_t e1) {
      keep(launch_args((const void*)k_final, dim3((unsigned)a.R), dim3(FIN_T), a, st, e0, e1));
    });
  if (probs)
    timed(ctx, KID_PROBS, [&](hipEvent_t e0, hipEvent_t e1) {
      keep(launch_args((const void*)k_probs, grid_rc, dim3(TPB), a, st, e0, e1));
    });
  if (e != hipSuccess) return STRIM_EHIP;
  return launch_status();
}

void profile_free(strim_ctx* ctx) {
  if (ctx->prof_ev) {
    for (int i = 0; i < 2 * ctx->prof_cap; ++i) (void)hipEventDestroy(ctx->prof_ev[i]);
    delete[] ctx->prof_ev;
    delete[] ctx->prof_kind;
  }
  ctx->prof_ev = nullptr;
  ctx->prof_kind = nullptr;
  ctx->prof_cap = ctx->prof_n = ctx->prof_on = 0;
}


// Host-checkable arguments of a sample call (everything but the capacity).
int check_sample_args(const void* logits, int32_t dtype, int32_t B, int32_t V, int64_t row_stride,
                      const strim_sampling_params* params, const uint32_t* mask_words,
                      int64_t mask_stride, const int32_t* history, int32_t H, int32_t noise_mode,
                      const int32_t* out_ids) {
  if (!logits || !params || !out_ids || !dtype_ok(dtype)) return STRIM_EINVAL;
  if (B <= 0 || V <= 0 || row_stride < V) return STRIM_EINVAL;
  if (mask_words && mask_stride < ((int64_t)V + 31) / 32) return STRIM_EINVAL;
  if (H < 0 || (H > 0 && !history) || (history && H == 0)) return STRIM_EINVAL;
  if (noise_mode != STRIM_NOISE_ICDF && noise_mode != STRIM_NOISE_GUMBEL) return STRIM_EINVAL;
  if (strim_check_params(params, B) != STRIM_OK) return STRIM_EINVAL;
  return STRIM_OK;
}

// The launch groups of one sample call over scratch `sc` sized for gmax rows (ctx only
// times the launches and may be null).
int sample_groups(strim_ctx* ctx, const Scratch& sc, int gmax, void* stream, const void* logits,
                  int32_t dtype, int32_t B, int32_t V, int64_t row_stride,
                  const strim_sampling_params* params, const uint32_t* mask_words,
                  int64_t mask_stride, const int32_t* history, const int32_t* history_len,
                  int32_t H, int32_t noise_mode, const float* noise, int32_t* out_ids,
                  int32_t* out_status, float* out_probs) {
  const int64_t nstride = noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V + 1 : 2;
  for (int32_t g0 = 0; g0 < B; g0 += gmax) {
    const int nb = (B - g0) < gmax ? (B - g0) : gmax;
    Args a;
    memset(&a, 0, sizeof(a));
    a.logits = (const char*)logits + (size_t)g0 * row_stride * dtype_size(dtype);
    a.row_stride = row_stride;
    a.dtype = dtype;
    a.vec_ok = vec_ok(a.logits, row_stride, dtype);
    a.R = nb;
    a.V = V;
    a.W = (V + CHUNK - 1) / CHUNK;
    a.B = nb;
    a.k = 0;
    a.verify = 0;
    a.mask = mask_words ? mask_words + (size_t)g0 * mask_stride : nullptr;
    a.mask_stride = mask_stride;
    a.hist = history ? history + (size_t)g0 * H : nullptr;
    a.hist_len = (history && history_len) ? history_len + g0 : nullptr;
    a.H = H;
    a.noise_mode = noise_mode;
    a.noise = noise ? noise + (size_t)g0 * nstride : nullptr;
    a.noise_stride = nstride;
    a.s = sc;
    a.out_ids = out_ids + g0;
    a.out_status = out_status ? out_status + g0 : nullptr;
    a.out_probs = out_probs ? out_probs + (size_t)g0 * V : nullptr;
    for (int i = 0; i < nb; ++i) {
      a.p[i] = params[g0 + i];
      a.lmp[i] = params[g0 + i].min_p > 0.0f ? log((double)params[g0 + i].min_p) : -INFINITY;
    }
    const int rc = run_group(ctx, (hipStream_t)stream, a, nb, out_probs != nullptr);
    if (rc != STRIM_OK) return rc;
  }
  return STRIM_OK;
}

constexpr ScratchLayout kNoallocLayout =
    scratch_layout((size_t)STRIM_NOALLOC_MAX_ROWS, (size_t)STRIM_NOALLOC_MAX_VOCAB, false);
static_assert(kNoallocLayout.bytes <= (size_t)16 << 20, "no-allocation scratch stays modest");

}  // namespace

// ---- the no-allocation entry point's scratch -------------------------------------------
// strim_sample_noalloc draws its scratch from this file-scope device array: one copy per
// GPU, at its own address, held until the process ends, zero at load. Its host-side name
// is not a device address: host code uses only the pointer noalloc_base returns.
static __device__ __align__(256) unsigned char noalloc_scratch[kNoallocLayout.bytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
char* g_noalloc_ptr[kMaxDevices] = {};

// The device address of `device`'s noalloc_scratch, looked up once per device with that
// device current (the caller's current device).
int noalloc_base(int device, char** out) {
  if (device < 0 || device >= kMaxDevices) return STRIM_EINVAL;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_ptr[device]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch)) != hipSuccess || !p)
      return STRIM_EHIP;
    g_noalloc_ptr[device] = (char*)p;
  }
  *out = g_noalloc_ptr[device];
  return STRIM_OK;
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

// GenParams as the engine consumes it: a finite temperature, T <= 0 greedy
// (GenParams.isGreedy, Sources/StrimEngine/EngineAPI.swift:66); top_p in (0,1] and
// top_k >= 0 (ChatRequest.swift:150-160); plus the extension ranges.
int strim_check_params(const strim_sampling_params* hp, int32_t n) {
  if (!hp || n < 0) return STRIM_EINVAL;
  for (int32_t i = 0; i < n; ++i) {
    const strim_sampling_params& p = hp[i];
    if (isnan(p.temperature) || isinf(p.temperature)) return STRIM_EINVAL;
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
  // V <= 2^20 keeps a row within 256 chunks, the bound of the finalize's per-chunk
  // LDS tables, and keeps a row's fixed-point mass sums (2^40 per unit of exp(l - m) in
  // k_gfinal, 2^43 in the exact resolution and the residual draw: at most V * 2^43)
  // inside 64 bits
  if (!out || max_rows <= 0 || max_vocab <= 0 || max_rows > (1 << 20) ||
      max_vocab > (1 << 20))
    return STRIM_EINVAL;
  *out = nullptr;
  strim_ctx* ctx = new (std::nothrow) strim_ctx();
  if (!ctx) return STRIM_ENOMEM;
  ctx->device = device;
  ctx->max_rows = max_rows;
  ctx->max_vocab = max_vocab;
  const ScratchLayout L = scratch_layout((size_t)max_rows, (size_t)max_vocab, true);
  ctx->bytes = L.bytes;
  int rc = on_device(device, [&]() -> int {
    if (hipMalloc(&ctx->base, ctx->bytes) != hipSuccess) return STRIM_ENOMEM;
    if (hipMemset(ctx->base, 0, ctx->bytes) != hipSuccess) return STRIM_EHIP;
    if (hipDeviceSynchronize() != hipSuccess) return STRIM_EHIP;
    return STRIM_OK;
  });
  if (rc != STRIM_OK) {
    if (ctx->base) (void)on_device(device, [&]() -> int { return (int)hipFree(ctx->base); });
    delete ctx;
    return rc;
  }
  ctx->s = scratch_at((char*)ctx->base, L, (size_t)max_vocab, true);
  *out = ctx;
  return STRIM_OK;
}

int strim_ctx_destroy(strim_ctx* ctx) {
  if (!ctx) return STRIM_EINVAL;
  int rc = on_device(ctx->device, [&]() -> int {
    profile_free(ctx);
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
  if (!ctx) return STRIM_EINVAL;
  const int rc = check_sample_args(logits, dtype, B, V, row_stride, params, mask_words,
                                   mask_stride, history, H, noise_mode, out_ids);
  if (rc != STRIM_OK) return rc;
  if (V > ctx->max_vocab) return STRIM_ECAPACITY;
  const int gmax = ctx->max_rows < MAXP ? ctx->max_rows : MAXP;
  return on_device(ctx->device, [&]() -> int {
    return sample_groups(ctx, ctx->s, gmax, stream, logits, dtype, B, V, row_stride, params,
                         mask_words, mask_stride, history, history_len, H, noise_mode, noise,
                         out_ids, out_status, out_probs);
  });
}

int strim_sample_noalloc(void* stream, const void* logits, int32_t dtype, int32_t B, int32_t V,
                         int64_t row_stride, const strim_sampling_params* params,
                         const uint32_t* mask_words, int64_t mask_stride,
                         const int32_t* history, const int32_t* history_len, int32_t H,
                         int32_t noise_mode, const float* noise, int32_t* out_ids,
                         int32_t* out_status) {
  const int rc = check_sample_args(logits, dtype, B, V, row_stride, params, mask_words,
                                   mask_stride, history, H, noise_mode, out_ids);
  if (rc != STRIM_OK) return rc;
  if (V > STRIM_NOALLOC_MAX_VOCAB) return STRIM_ECAPACITY;
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess) return STRIM_EHIP;
  char* base = nullptr;
  const int brc = noalloc_base(device, &base);
  if (brc != STRIM_OK) return brc;
  const Scratch sc = scratch_at(base, kNoallocLayout, (size_t)STRIM_NOALLOC_MAX_VOCAB, false);
  return sample_groups(nullptr, sc, STRIM_NOALLOC_MAX_ROWS, stream, logits, dtype, B, V,
                       row_stride, params, mask_words, mask_stride, history, history_len, H,
                       noise_mode, noise, out_ids, out_status, nullptr);
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
  if (B <= 0 || k < 0 || k > 64 || V <= 0) return STRIM_EINVAL;
  if (k + 1 > ctx->max_rows) return STRIM_EINVAL;
  if (k > 0 && !draft_tokens) return STRIM_EINVAL;
  if (draft_logits && (!draft_to_full || Vd <= 0 || Vd > V)) return STRIM_EINVAL;
  if (mask_words && mask_stride < ((int64_t)V + 31) / 32) return STRIM_EINVAL;
  if (H < 0 || (H > 0 && !history) || (history && H == 0)) return STRIM_EINVAL;
  if (noise_mode != STRIM_NOISE_ICDF && noise_mode != STRIM_NOISE_GUMBEL) return STRIM_EINVAL;
  if (strim_check_params(params, B) != STRIM_OK) return STRIM_EINVAL;
  if (V > ctx->max_vocab) return STRIM_ECAPACITY;
  const int64_t nstride = noise_mode == STRIM_NOISE_GUMBEL ? (int64_t)V + 1 : 2;
  int gmax = ctx->max_rows / (k + 1);
  if (gmax > MAXP) gmax = MAXP;
  // general-q: at most MAXP draft rows per group (their per-row scratch)
  if (draft_logits && k > 0 && gmax * k > MAXP) gmax = MAXP / k > 0 ? MAXP / k : 1;
  return on_device(ctx->device, [&]() -> int {
    hipStream_t st = (hipStream_t)stream;
    for (int32_t g0 = 0; g0 < B; g0 += gmax) {
      const int nb = (B - g0) < gmax ? (B - g0) : gmax;
      const int rows = nb * (k + 1);
      Args a;
      memset(&a, 0, sizeof(a));
      a.logits = (const char*)target_logits + (size_t)g0 * (k + 1) * V * dtype_size(dtype);
      a.row_stride = V;
      a.dtype = dtype;
      a.vec_ok = vec_ok(a.logits, V, dtype);
      a.R = rows;
      a.V = V;
      a.W = (V + CHUNK - 1) / CHUNK;
      a.B = nb;
      a.k = k;
      a.verify = 1;
      a.mask = mask_words ? mask_words + (size_t)g0 * (k + 1) * mask_stride : nullptr;
      a.mask_stride = mask_stride;
      a.hist = history ? history + (size_t)g0 * H : nullptr;
      a.hist_len = (history && history_len) ? history_len + g0 : nullptr;
      a.H = H;
      a.drafts = draft_tokens ? draft_tokens + (size_t)g0 * k : nullptr;
      if (draft_logits && k > 0) {
        a.dlog = (const char*)draft_logits + (size_t)g0 * k * Vd * dtype_size(dtype);
        a.dtable = draft_to_full;
        a.Vd = Vd;
        // without per-row tokens only the first rejection's residual is needed
        a.qskip = noise_mode == STRIM_NOISE_GUMBEL && out_row_token == nullptr ? 1 : 0;
      }
      a.noise_mode = noise_mode;
      a.noise = noise ? noise + (size_t)g0 * (k + 1) * nstride : nullptr;
      a.noise_stride = nstride;
      a.s = ctx->s;
      a.out_accepted = out_accepted + g0;
      a.out_token = out_token + g0;
      a.out_row_accept = out_row_accept ? out_row_accept + (size_t)g0 * k : nullptr;
      a.out_row_token = out_row_token ? out_row_token + (size_t)g0 * (k + 1) : nullptr;
      a.out_status = out_status ? out_status + g0 : nullptr;
      for (int i = 0; i < nb; ++i) {
        a.p[i] = params[g0 + i];
        a.lmp[i] = params[g0 + i].min_p > 0.0f ? log((double)params[g0 + i].min_p) : -INFINITY;
      }
      hipError_t e = hipSuccess;
      if (a.dlog) {
        // draft distributions (QSPLIT workgroups per draft row; each draft row's
        // k_finalize workgroup merges its slices) and, with the first group, the
        // draft-vocab bitmap (one thread per table entry), as extra workgroups of the
        // k_stream launch (measured: a launch of their own before k_stream cost 9.7 us
        // per step; on a second stream beside k_stream, joined by an event, 4.6 us more)
        const int nt = stream_threads(rows);
        const int nwb = g0 == 0 ? (int)((Vd + nt - 1) / nt) : 0;
        a.nqprep = nb * k * QSPLIT + nwb;
      }
      bool combined = false;
      int rc = run_group(ctx, st, a, nb, false, &combined);
      if (rc != STRIM_OK) return rc;
      if (!combined)
        timed(ctx, KID_COMBINE, [&](hipEvent_t e0, hipEvent_t e1) {
          e = launch_args((const void*)k_verify_combine, dim3((unsigned)((nb + 63) / 64)),
                          dim3(64), a, st, e0, e1);
        });
      rc = e != hipSuccess ? STRIM_EHIP : launch_status();
      if (rc != STRIM_OK) return rc;
    }
    return STRIM_OK;
  });
}

const char* strim_kernel_name(int32_t kernel) {
  return (kernel >= 0 && kernel < STRIM_KERNEL_COUNT) ? kKernelNames[kernel] : "";
}

int strim_profile_begin(strim_ctx* ctx, int32_t max_launches) {
  if (!ctx || max_launches <= 0 || max_launches > (1 << 22)) return STRIM_EINVAL;
  return on_device(ctx->device, [&]() -> int {
    profile_free(ctx);
    ctx->prof_ev = new (std::nothrow) hipEvent_t[2 * (size_t)max_launches];
    ctx->prof_kind = new (std::nothrow) int32_t[max_launches];
    if (!ctx->prof_ev || !ctx->prof_kind) {
      delete[] ctx->prof_ev;
      delete[] ctx->prof_kind;
      ctx->prof_ev = nullptr;
      ctx->prof_kind = nullptr;
      return STRIM_ENOMEM;
    }
    for (int i = 0; i < 2 * max_launches; ++i) {
      if (hipEventCreate(&ctx->prof_ev[i]) != hipSuccess) {
        for (int q = 0; q < i; ++q) (void)hipEventDestroy(ctx->prof_ev[q]);
        delete[] ctx->prof_ev;
        delete[] ctx->prof_kind;
        ctx->prof_ev = nullptr;
        ctx->prof_kind = nullptr;
        return STRIM_EHIP;
      }
    }
    ctx->prof_cap = max_launches;
    ctx->prof_n = 0;
    ctx->prof_on = 1;
    return STRIM_OK;
  });
}

int strim_profile_end(strim_ctx* ctx, double* total_ms, int64_t* launches) {
  if (!ctx || !total_ms || !launches || !ctx->prof_on) return STRIM_EINVAL;
  return on_device(ctx->device, [&]() -> int {
    for (int k = 0; k < STRIM_KERNEL_COUNT; ++k) {
      total_ms[k] = 0.0;
      launches[k] = 0;
    }
    int rc = STRIM_OK;
    for (int i = 0; i < ctx->prof_n; ++i) {
      float ms = 0.0f;
      if (hipEventSynchronize(ctx->prof_ev[2 * i + 1]) != hipSuccess ||
          hipEventElapsedTime(&ms, ctx->prof_ev[2 * i], ctx->prof_ev[2 * i + 1]) != hipSuccess) {
        rc = STRIM_EHIP;
        break;
      }
      total_ms[ctx->prof_kind[i]] += (double)ms;
      launches[ctx->prof_kind[i]] += 1;
    }
    profile_free(ctx);
    return rc;
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

namespace {
// the producer's operand checks (out_logits NULL is allowed where the caller says so)
bool head_args_ok(const void* hidden, int64_t hidden_stride, int32_t B, int32_t K,
                  const void* norm_weight, float eps, const void* xn, const void* lm_head,
                  int64_t lm_head_stride, int32_t V, const void* out_logits, int64_t out_stride) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (!hidden || !lm_head || B < 1 || B > 64 || K <= 0 || K % 256 != 0 || V <= 0 ||
      hidden_stride < K || lm_head_stride < K || (out_logits && out_stride < V) ||
      !(eps >= 0.0f) || !al16(hidden) || hidden_stride % 8 != 0 || !al16(lm_head) ||
      lm_head_stride % 8 != 0)
    return false;
  if (norm_weight && (!xn || !al16(xn) || !al16(norm_weight))) return false;
  return true;
}
}  // namespace

int strim_head_logits(void* stream, const void* hidden, int64_t hidden_stride, int32_t B,
                      int32_t K, const void* norm_weight, float eps, void* xn,
                      const void* lm_head, int64_t lm_head_stride, int32_t V, void* out_logits,
                      int64_t out_stride) {
  if (!out_logits || !head_args_ok(hidden, hidden_stride, B, K, norm_weight, eps, xn, lm_head,
                                   lm_head_stride, V, out_logits, out_stride))
    return STRIM_EINVAL;
  const bool vo = ((uintptr_t)out_logits & 7u) == 0 && out_stride % 4 == 0;
  const hipError_t e = launch_head(hidden, hidden_stride, B, K, norm_weight, eps, xn, lm_head,
                                   lm_head_stride, V, out_logits, out_stride, vo,
                                   (hipStream_t)stream, nullptr, nullptr, nullptr);
  return e == hipSuccess ? STRIM_OK : STRIM_EHIP;
}

int strim_head_greedy(strim_ctx* ctx, void* stream, const void* hidden, int64_t hidden_stride,
                      int32_t B, int32_t K, const void* norm_weight, float eps, void* xn,
                      const void* lm_head, int64_t lm_head_stride, int32_t V, void* out_logits,
                      int64_t out_stride, int32_t* out_ids, int32_t* out_status) {
  if (!ctx || !out_ids ||
      !head_args_ok(hidden, hidden_stride, B, K, norm_weight, eps, xn, lm_head, lm_head_stride,
                    V, out_logits, out_stride))
    return STRIM_EINVAL;
  if (B > ctx->max_rows || V > ctx->max_vocab) return STRIM_ECAPACITY;
  // the tile maxima [B][ceil(V / 128)] go to the context's candidate slots (stream-ordered
  // with every other call on the context; they need B * V / 16 bytes, the slots hold
  // max_rows * max_vocab bytes)
  static_assert(sizeof(Cand) * SLOT >= (CHUNK / 128) * sizeof(uint2), "tile maxima fit the slots");
  uint2* tbest = (uint2*)ctx->s.slot;
  const bool vo = out_logits && ((uintptr_t)out_logits & 7u) == 0 && out_stride % 4 == 0;
  const hipError_t e = launch_head(hidden, hidden_stride, B, K, norm_weight, eps, xn, lm_head,
                                   lm_head_stride, V, out_logits, out_stride, vo,
                                   (hipStream_t)stream, tbest, out_ids, out_status);
  return e == hipSuccess ? STRIM_OK : STRIM_EHIP;
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
