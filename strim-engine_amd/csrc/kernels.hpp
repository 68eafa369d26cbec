// kernels.hpp — argument block, scratch layout and per-row processing shared by the
// gfx950 kernels.
//
// A sampling call runs two kernels over R rows of V logits:
//   k_stream   (rows x chunks)  the single streaming pass: processed logits, chunk
//                               statistics and the chunk's candidates;
//   k_finalize (one workgroup per row) decides greedy, fast and unfiltered Gumbel rows,
//   k_gfinal   (one workgroup per row) the general rows (each runs only when some row of
//                               the call needs it).
// A general-q verify adds k_qprep before them and the residual draw (qres_kernels.hip)
// after them, and k_final when a draft row can need the exact resolution. Rows whose candidates overflow are decided
// by the exact streaming resolution (exact.hpp) inside the deciding workgroup.
// Workgroups never wait for or fence against each other: every partial result is a
// plain store into a per-(row, chunk) slot that the next kernel reads.
#pragma once

#include "common.hpp"

namespace strim {

constexpr int MAXP = 64;         // parameter rows carried inline per launch group
constexpr int QNB = 256;         // QRES coarse bins of d = m - l, 1/4 nat wide
constexpr int QPT = 1024;        // threads of a k_qprep workgroup
// k_stream runs one chunk per workgroup with 8 SSEG tokens per thread: SSEG = 1 (512
// threads, 8 waves) for small batches, whose time is latency, and SSEG = 4 (128 threads,
// 2 waves) for large ones, whose time is instructions per token. Each wave writes its
// fast-row candidates to its own region of the chunk's SLOT entries.
constexpr int SMAXW = 8;         // most waves of a k_stream workgroup
constexpr int SLOT = 512;        // fast-path candidate entries per chunk
constexpr int FTPB = 256;        // threads of a k_finalize workgroup (one row)
constexpr int FCAND = 8192;      // candidates per row k_finalize gathers
constexpr int FCAP = 8192;       // candidate keys k_finalize holds in LDS
constexpr int FCAP_FAST = 4096;  // of which fast rows use at most this many
// General rows bin their tokens on an absolute lattice of l = v / T: bin A(l) =
// floor(l * LBS), so every chunk of a row bins the same way and the chunks' histograms
// add up to the row's. A chunk keeps the NBW bins below its top bin A(m_c) (its window,
// 12 nats), counts and masses per bin, and writes its window tokens in bin order, as
// many whole bins as fit LCAP entries of its slot region.
constexpr int LBS = 16;          // lattice bins per nat (a power of two: l * LBS is exact)
constexpr int NBW = 192;         // window bins of a chunk (and of a row, below its top)
constexpr int LCAP = 256;        // candidates a general row's chunk writes in bin order
constexpr int LWMAX = 40;        // chunks of a row k_gfinal's lattice path serves
                                 // (V <= 163,840; wider rows take the exact resolution)
constexpr int LCSH = 51;         // a lattice word: count << LCSH | mass (2^37 per unit of
                                 // exp(l - A / LBS), A the bin's lattice index)
constexpr uint64_t LMMASK = (1ull << LCSH) - 1ull;
constexpr int KLOC = 256;        // largest top-k served by local candidates
constexpr float MINP_FAST = 3.3546262e-4f;  // e^-8: min-p at or above bounds candidates

enum RowClass : int32_t { CLS_GREEDY = 0, CLS_FAST = 1, CLS_GENERAL = 2, CLS_INVALID = 3 };

// Set by k_finalize and k_gfinal: DONE rows are decided; EXACT rows (filtered general-q
// verify rows) go to k_final's exact streaming resolution, whose workgroups are four
// times wider than k_finalize's; QRES rows (unfiltered general-q verify rows) are decided
// by the grid-wide residual draw (qres_kernels.hip), which demotes an icdf row to EXACT
// when its bucket overflows.
enum RowPhase : int32_t { PH_DONE = 1, PH_EXACT = 2, PH_QRES = 3 };

// Written by k_stream without a closing barrier: m, n, flags, g and ncand by the first
// wave, arg by the wave holding the first maximum.
struct ChunkStat {
  float m;         // chunk max of processed logits (-inf if none allowed)
  int32_t n;       // allowed tokens (fast and greedy rows: 1 if any)
  int32_t flags;   // bit0: non-finite logit
  float g;         // fast top-k rows: at least k of the chunk's tokens have v >= g (v is
                   // the value before temperature), -inf when not certified
  double S;        // sum exp(l - m) over the chunk (general rows)
  int32_t arg;     // first id reaching m
  uint32_t ncand;  // fast rows: candidates in the chunk's slot region (> SLOT: overflow);
                   // general rows: window bins whose tokens are all written (nfull)
  float g2;        // (unused)
  uint32_t ncand2; // general rows: window bins with lattice words written (nb: the last
                   // non-empty bin + 1); LNONE when the lattice cannot hold the row
  uint32_t pad_;
};
constexpr uint32_t LNONE = 0xFFFFFFFFu;
static_assert(sizeof(ChunkStat) == 48, "ChunkStat layout");

// Unfiltered Gumbel rows: the chunk's two best tokens by the fp32 Gumbel proxy l + g.
struct ChunkPart {
  float l0, l1;
  int32_t id0, id1;
};

// A candidate: fast rows store the value before temperature, general rows after it.
struct Cand {
  float l;
  int32_t id;
};

struct RowState {
  float l_draft;   // verify: processed logit of the row's draft (-inf if masked)
  int32_t status;
  int32_t token;
  int32_t accept;
  double sum_kept;
  float m;
  int32_t phase;      // RowPhase: which kernel still has to decide the row
  uint64_t last_key;  // last kept token's order key (the kept set is the prefix of the
                      // (l desc, id asc) order up to it; 0 = none)
  // QRES rows: plain mass S, residual mass, draw target T (fixed point), the chosen
  // coarse bin and the residual mass before it
  uint64_t qS, qR, qT, qbelow;
  int32_t qbin, pad_;
};

// Draft distribution of one general-q verify row: q = softmax(draft logits / T).
struct QStat {
  float mq;     // max of draft_logit / T (fp32 division)
  int32_t td;   // table index of the row's draft token, -1 if absent
  double Z;     // sum of exp(v - mq), fp64
};

// k_qprep's partial result over one of the QSPLIT slices of a draft row's table.
constexpr int QSPLIT = 16;
struct QPart {
  float m;      // slice maximum of v (-inf if empty)
  int32_t td;   // table index of the draft in the slice, -1 if absent
  double z;     // sum over the slice of exp(v - m), fp64
  int32_t bad;  // the slice breaks the table's order or range (row 0 only)
  int32_t pad_;
};

// Device scratch owned by a context (allocated once in strim_ctx_create).
struct Scratch {
  ChunkStat* cstat;               // [rows][wmax]
  Cand* slot;                     // [rows][wmax][SLOT] the chunks' candidates: (v before
                                  // temperature, id) for fast rows, (l, id) for general
                                  // rows
  ChunkPart* part;                // [rows][wmax]
  RowState* rs;                   // [rows]
  Cand* cand;                     // [rows][CAP] QRES rows: the tokens of the draw's bin
  uint32_t* ncand;                // [rows] their count
  uint32_t* dbits;                // [ceil(V/32)] general-q verify: draft-vocab membership
  uint32_t* wrank;                // [ceil(V/32)] table entries below id 32 w: a member id's
                                  // table index is wrank[id / 32] + the member bits below it
  unsigned long long* qpart;      // [MAXP][wmax] QRES rows: plain mass per chunk
  uint32_t* qhc;                  // [MAXP][wmax][QNB] QRES rows: residual counts per bin
  unsigned long long* qhm;        // [MAXP][wmax][QNB] QRES rows: residual masses per bin
  QStat* qst;                     // [rows] per draft row (b * k + j)
  QPart* qpp;                     // [MAXP][QSPLIT] k_qprep slices, merged by k_finalize
  uint32_t* qarr;                 // [MAXP] per sequence: k_qgumbel workgroups arrived (zero
                                  // between launches: the last arriver resets it)
  unsigned long long* lat;        // [rows][wmax][NBW] general rows: per window bin of the
                                  // chunk, its inclusive count prefix << LCSH | its mass
                                  // (2^37 per unit of exp(l - A / LBS), A the bin's index)
  int32_t wmax;
};

// One launch argument block (passed by value to every kernel of a call).
struct Args {
  const void* logits;
  int64_t row_stride;
  int32_t dtype;
  int32_t vec_ok;
  int32_t R, V, W;   // rows in this group, vocab, chunks per row
  int32_t B, k;      // batch rows in this group and draft length (k = 0: sample)
  int32_t verify;
  int32_t xmap;           // k_stream and the residual-draw kernels: rows kept per XCD
  int32_t gen;            // some row of the launch is general (row_class): the host picks
                          // the k_stream variant with the general rows' code
  int32_t qskip;          // general-q verify without per-row tokens: k_finalize takes the
                          // accept test, the residual draw serves first rejections only
  int32_t nqprep;         // general-q verify: k_qprep blocks carried by the k_stream launch
                          // (its grid rows past R)
  const uint32_t* mask;
  int64_t mask_stride;
  const int32_t* hist;
  const int32_t* hist_len;
  int32_t H;
  const int32_t* drafts;  // [B][k] (group-relative)
  const void* dlog;       // general-q verify: draft logits [B][k][Vd] (dtype), or NULL
  const int32_t* dtable;  // [Vd] strictly ascending full-vocab ids
  int32_t Vd;
  int32_t noise_mode;
  const float* noise;
  int64_t noise_stride;
  Scratch s;
  int32_t* out_ids;
  int32_t* out_status;
  float* out_probs;
  int32_t* out_accepted;
  int32_t* out_token;
  int32_t* out_row_accept;
  int32_t* out_row_token;
  strim_sampling_params p[MAXP];  // per batch row of the group
  double lmp[MAXP];               // log(min_p) per batch row (host libm), -inf when off
};
// The block is passed by value: it must fit the 4 KB kernel-argument segment.
static_assert(sizeof(Args) <= 4096, "Args exceeds the 4 KB kernel-argument limit");

// Launches kernel `fn(Args)` on st. Given a start/stop event pair, the events take the
// dispatch's own begin and end timestamps (hipExtLaunchKernel), so their elapsed time is
// the kernel's execution alone, without the queue's gap before it; a sequence of
// launches passes the start event to its first and the stop event to its last.
inline hipError_t launch_args(const void* fn, dim3 grid, dim3 block, const Args& a,
                              hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  void* args[] = {const_cast<Args*>(&a)};
  if (e0 || e1) return hipExtLaunchKernel(fn, grid, block, args, 0, st, e0, e1, 0);
  return hipLaunchKernel(fn, grid, block, args, 0, st);
}

struct RowParams {
  double lmp;  // log(min_p), -inf when min-p is off
  float T, rep, pres, freq, min_p, top_p;
  int32_t top_k;
  uint32_t flags;
  uint64_t seed, position;
  bool greedy, pen;
  int32_t cls;
};

// Smallest v (the value before temperature) whose l = RN(v / T) can pass min-p against
// a maximum mt after temperature: v >= (mt + log(min_p)) T, less a rounding margin of a
// few ulps.
__device__ __forceinline__ float minp_vlo(float mt, const RowParams& p) {
  const double tl = ((double)mt + p.lmp) * (double)p.T;
  return (float)(tl - fabs(tl) * 4e-7 - 1e-37);
}

// Classification shared by host and device: which path resolves the row.
__host__ __device__ inline int32_t row_class(const strim_sampling_params& p, int32_t V) {
  if (!(p.temperature > 0.0f)) return CLS_GREEDY;
  const bool topk = p.top_k > 0 && p.top_k < V;
  if (topk && p.top_k <= KLOC) return CLS_FAST;
  if (p.min_p >= MINP_FAST) return CLS_FAST;
  return CLS_GENERAL;
}

// Rows k_gfinal decides (gfinal_kernels.hip): the general rows, except the unfiltered
// Gumbel rows (k_finalize's two-best path) and the draft rows of a general-q verify
// (k_finalize marks them for the residual draw and k_final).
__host__ __device__ inline bool gfinal_row(const strim_sampling_params& p, int32_t V,
                                           int32_t noise_mode, bool general_q_draft_row) {
  if (row_class(p, V) != CLS_GENERAL || general_q_draft_row) return false;
  const bool nofilter = !(p.top_k > 0 && p.top_k < V) && !(p.min_p > 0.0f) && !(p.top_p < 1.0f);
  return !(noise_mode == STRIM_NOISE_GUMBEL && nofilter);
}

// A row's outcome as the verify combine reads it.
struct RowOut {
  int32_t status, accept, token;
};
// SpecSampling.verify's accept chain over sequence b's k + 1 rows (one thread): the
// leading accepted drafts, the token at the first rejection (or the bonus row's), and the
// per-row outputs; row(j) gives row j's outcome.
template <typename F>
__device__ __forceinline__ void verify_combine_one(const Args& a, int b, F row) {
  const int k = a.k;
  int status = STRIM_OK, n = 0, token = -1;
  bool alive = true;
  // SpecSampling.verify consumes only the rows its accept chain reaches, 0 .. n
  // (SpecSampling.swift:101-105): a row error counts for the sequence only when the chain
  // reaches that row; later rows report theirs in the per-row outputs alone. The rows are
  // taken four at a time, their outcomes read together (places past k repeat row k).
  for (int j0 = 0; j0 <= k; j0 += 4) {
    RowOut o[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = row(min(j0 + u, k));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u;
      if (j > k) break;
      const RowOut rs = o[u];
      if (rs.status != STRIM_OK) {
        if (alive) {
          status = rs.status;
          alive = false;
        }
        if (a.out_row_accept && j < k) a.out_row_accept[(int64_t)b * k + j] = 0;
        if (a.out_row_token) a.out_row_token[(int64_t)b * (k + 1) + j] = -1;
        continue;
      }
      const int acc = j < k ? rs.accept : 0;
      if (a.out_row_accept && j < k) a.out_row_accept[(int64_t)b * k + j] = acc;
      if (a.out_row_token) a.out_row_token[(int64_t)b * (k + 1) + j] = rs.token;
      if (alive) {
        if (j < k && acc) ++n;
        else {
          alive = false;
          token = rs.token;
        }
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

__device__ __forceinline__ void row_bj(const Args& a, int r, int& b, int& j) {
  if (a.verify) {
    b = r / (a.k + 1);
    j = r - b * (a.k + 1);
  } else {
    b = r;
    j = 0;
  }
}

// Workgroup -> (row, chunk) on a (W chunks, R rows) grid. The dispatcher hands the
// workgroups of a launch to the 8 XCDs round robin in linear order, and each XCD has an
// L2 of its own. With a.xmap the map gives XCD x one contiguous run of the row-major
// (row, chunk) order, so the chunks of a row share one L2 and what every chunk of a row
// reads (its history ids) comes from HBM once per row instead of once per XCD; without
// it the chunks of a row spread over every XCD, which balances rows of unequal cost (a
// dense-mask general row) better. Both are bijections for every grid, whatever the
// dispatch order.
constexpr uint32_t NXCD = 8;
template <typename A>
__device__ __forceinline__ void map_block(const A& a, int& r, int& c) {
  if (!a.xmap) {
    r = blockIdx.y;
    c = blockIdx.x;
    return;
  }
  const uint32_t W = (uint32_t)a.W;
  const uint32_t n = W * (uint32_t)a.R;
  const uint32_t L = blockIdx.x + blockIdx.y * W;
  const uint32_t x = L % NXCD, q = n / NXCD, rem = n % NXCD;
  const uint32_t m = x * q + (x < rem ? x : rem) + L / NXCD;
  r = (int)(m / W);
  c = (int)(m - (uint32_t)r * W);
}

__device__ __forceinline__ RowParams load_params(const Args& a, int b, int j) {
  const strim_sampling_params& sp = a.p[b];
  RowParams p;
  p.T = sp.temperature;
  p.rep = sp.repetition_penalty;
  p.pres = sp.presence_penalty;
  p.freq = sp.frequency_penalty;
  p.min_p = sp.min_p;
  p.lmp = a.lmp[b];
  p.top_p = sp.top_p;
  p.top_k = sp.top_k;
  p.flags = a.verify ? (sp.flags & STRIM_FLAG_TOPK_KEEP_TIES) : sp.flags;
  p.seed = sp.seed;
  p.position = sp.position + (uint64_t)j;
  p.greedy = !(p.T > 0.0f);
  // (bitwise, not short-circuit: no branch on the parameters here)
  const bool active = (p.rep != 1.0f) | (p.pres != 0.0f) | (p.freq != 0.0f);
  p.pen = active & ((a.hist != nullptr) | ((a.verify != 0) & (j > 0)));
  p.cls = row_class(sp, a.V);
  return p;
}

// Raw logits of this thread's EPT tokens (issued before anything waits on memory).
template <typename A>
__device__ __forceinline__ void load_tokens(const A& a, int r, int i0, float (&x)[EPT]) {
  const int64_t base = (int64_t)r * a.row_stride;
  if (a.dtype == STRIM_DTYPE_BF16) {
    const uint16_t* xb = (const uint16_t*)a.logits + base;
    if (a.vec_ok && i0 + EPT <= a.V) {
      const uint4 v = *(const uint4*)(xb + i0);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[2 * e] = __uint_as_float(w[e] << 16);
        x[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) x[e] = (i0 + e < a.V) ? bf16_to_f32(xb[i0 + e]) : 0.0f;
    }
  } else {
    const float* xf = (const float*)a.logits + base;
    if (a.vec_ok && i0 + EPT <= a.V) {
      const float4 v0 = *(const float4*)(xf + i0);
      const float4 v1 = *(const float4*)(xf + i0 + 4);
      x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w;
      x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) x[e] = (i0 + e < a.V) ? xf[i0 + e] : 0.0f;
    }
  }
}

// History counts of the span [c0, c0 + SPAN) in LDS (plus the verify draft prefix).
// Called by every thread of an NT-thread workgroup when p.pen.
template <int NT, int SPAN, typename A>
__device__ __forceinline__ void build_counts_span(const A& a, int b, int j, int c0,
                                                  uint32_t* s_cnt) {
  for (int i = threadIdx.x; i < SPAN; i += NT) s_cnt[i] = 0u;
  __syncthreads();
  if (a.hist) {
    int hl = a.hist_len ? a.hist_len[b] : a.H;
    hl = hl < 0 ? 0 : (hl > a.H ? a.H : hl);
    const int32_t* h = a.hist + (int64_t)b * a.H;
    for (int i = threadIdx.x; i < hl; i += NT) {
      const int id = h[i];
      const unsigned o = (unsigned)(id - c0);
      if (o < (unsigned)SPAN && id < a.V) atomicAdd(&s_cnt[o], 1u);
    }
  }
  if (a.verify && (int)threadIdx.x < j) {
    const int id = a.drafts[(int64_t)b * a.k + threadIdx.x];
    const unsigned o = (unsigned)(id - c0);
    if (o < (unsigned)SPAN && id < a.V) atomicAdd(&s_cnt[o], 1u);
  }
  __syncthreads();
}
__device__ __forceinline__ void build_counts(const Args& a, int b, int j, int c0,
                                             uint32_t* s_cnt) {
  build_counts_span<TPB, CHUNK>(a, b, j, c0, s_cnt);
}

// Penalties -> mask -> temperature on raw values x. Masked / out-of-range tokens get
// -inf. Greedy rows skip the temperature. Each step is one IEEE float32 operation (the
// library is built with -ffp-contract=off). `cnt` points at this thread's EPT history
// counts.
template <typename A>
__device__ __forceinline__ void process_tokens(const A& a, int r, int i0, const RowParams& p,
                                               const uint32_t* cnt, const float (&x)[EPT],
                                               float (&l)[EPT], bool& nonfinite) {
  uint32_t bits = 0xFFu;
  if (a.mask && i0 < a.V) {
    const uint32_t wd = a.mask[(int64_t)r * a.mask_stride + (i0 >> 5)];
    bits = (wd >> (i0 & 31)) & 0xFFu;
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    float v = x[e];
    if (p.pen) {
      const uint32_t c = cnt[e];
      if (c > 0u) {
        v = v > 0.0f ? v / p.rep : v * p.rep;
        v = v - p.freq * (float)c;
        v = v - p.pres;
      }
    }
    const bool ok = (i0 + e < a.V) && ((bits >> e) & 1u);
    if (!ok) {
      l[e] = -INFINITY;
      continue;
    }
    if (isnan(v) || v == INFINITY) nonfinite = true;
    const float lv = p.greedy ? v : v / p.T;
    if (lv == INFINITY) nonfinite = true;
    l[e] = lv;
  }
}

// Allow-bits of the 8 tokens [i0, i0 + 8) (i0 a multiple of 8): one byte of the packed
// row, because bit (i & 31) of word (i >> 5) on a little-endian device is bit (i & 7) of
// byte (i >> 3).
template <typename A>
__device__ __forceinline__ uint32_t load_mask8(const A& a, int r, int i0) {
  if (!a.mask || i0 >= a.V) return 0xFFu;
  return ((const uint8_t*)(a.mask + (int64_t)r * a.mask_stride))[i0 >> 3];
}

// process_tokens on preloaded allow-bits (see load_mask8).
template <typename A>
__device__ __forceinline__ void process_seg(const A& a, int i0, const RowParams& p, uint32_t bits,
                                            const uint32_t* cnt, const float (&x)[EPT],
                                            float (&l)[EPT], bool& nonfinite) {
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    float v = x[e];
    if (p.pen) {
      const uint32_t c = cnt[e];
      if (c > 0u) {
        v = v > 0.0f ? v / p.rep : v * p.rep;
        v = v - p.freq * (float)c;
        v = v - p.pres;
      }
    }
    const bool ok = (i0 + e < a.V) && ((bits >> e) & 1u);
    if (!ok) {
      l[e] = -INFINITY;
      continue;
    }
    if (isnan(v) || v == INFINITY) nonfinite = true;
    const float lv = p.greedy ? v : v / p.T;
    if (lv == INFINITY) nonfinite = true;
    l[e] = lv;
  }
}

// History counts of a span in LDS in two steps, so the history loads can be issued
// before the caller's logits loads and their latency overlaps them: hist_load requests
// this thread's first HPT history ids (16 bytes at a time when aligned); hist_count
// clears the table for [c0, c0 + SPAN), counts every history id inside it (plus the
// verify draft prefix) and ends with a barrier.
template <int NT>
constexpr int hpt() { return 4096 / NT; }  // history ids each thread preloads
template <int NT, typename A>
__device__ __forceinline__ void hist_load(const A& a, int b, int (&ids)[hpt<NT>()]) {
  constexpr int HPT = hpt<NT>();
  const int t = threadIdx.x;
  const int32_t* h = a.hist ? a.hist + (int64_t)b * a.H : nullptr;
  // loads from clamped indices with no branch between them (see load_chunk)
  if (h && ((uintptr_t)h & 15u) == 0 && (a.H & 3) == 0) {
    // (positions past the history length are ignored by hist_count, so the loaded
    // values are not touched here and no instruction waits for them yet)
#pragma unroll
    for (int q = 0; q < HPT / 4; ++q) {
      const int i = 4 * (q * NT + t);
      const int4 v = *(const int4*)(h + (i < a.H ? i : 0));
      ids[4 * q] = v.x; ids[4 * q + 1] = v.y; ids[4 * q + 2] = v.z; ids[4 * q + 3] = v.w;
    }
  } else if (h) {
#pragma unroll
    for (int q = 0; q < HPT; ++q) {
      const int i = 4 * ((q >> 2) * NT + t) + (q & 3);
      ids[q] = h[i < a.H ? i : 0];
    }
  } else {
#pragma unroll
    for (int q = 0; q < HPT; ++q) ids[q] = -1;
  }
}
// The row's history length. Read after the caller's other loads are issued: the
// compiler moves the uniform value to a scalar register at once, which waits for it.
template <typename A>
__device__ __forceinline__ int hist_len(const A& a, int b) {
  if (!a.hist) return 0;
  if (!a.hist_len) return a.H;
  const int raw = a.hist_len[b];
  return raw < 0 ? 0 : (raw > a.H ? a.H : raw);
}
// NARROW: 16-bit counts, two to a word (token o in the low half of word o / 2 when o is
// even), for callers that know no count reaches 65,536 (history length plus draft prefix
// below it); otherwise one 32-bit count per token.
template <int NT, int SPAN, typename A, bool NARROW = false>
__device__ __forceinline__ void hist_count(const A& a, int b, int j, int c0,
                                           const int (&ids)[hpt<NT>()], int hl, uint32_t* s_cnt) {
  constexpr int HPT = hpt<NT>();
  const int t = threadIdx.x;
  auto add = [&](uint32_t o) {
    if constexpr (NARROW) atomicAdd(&s_cnt[o >> 1], 1u << ((o & 1u) << 4));
    else atomicAdd(&s_cnt[o], 1u);
  };
  uint4* s4 = (uint4*)s_cnt;
  for (int i = t; i < (NARROW ? SPAN / 8 : SPAN / 4); i += NT) s4[i] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();
  const uint32_t uc0 = (uint32_t)c0;
  // ids inside [c0, c0 + lim) count: lim stops at the row end, and a negative id wraps
  // to a large offset
  const int rem = a.V - c0;
  const uint32_t lim = rem <= 0 ? 0u : (uint32_t)(rem < SPAN ? rem : SPAN);
#pragma unroll
  for (int q = 0; q < HPT; ++q) {
    // a group of four ids per thread lies wholly past the history length for the whole
    // workgroup (hl is the row's): skipped by a scalar branch
    if (4 * (q >> 2) * NT >= hl) continue;
    const int i = 4 * ((q >> 2) * NT + t) + (q & 3);
    const uint32_t o = (uint32_t)ids[q] - uc0;
    if (i < hl && o < lim) add(o);
  }
  if (hl > HPT * NT) {
    const int32_t* h = a.hist + (int64_t)b * a.H;
    for (int i = HPT * NT + t; i < hl; i += NT) {
      const int id = h[i];
      const uint32_t o = (uint32_t)id - uc0;
      if (o < (uint32_t)SPAN && id >= 0 && id < a.V) add(o);
    }
  }
  if (a.verify && t < j) {
    const int id = a.drafts[(int64_t)b * a.k + t];
    const uint32_t o = (uint32_t)id - uc0;
    if (o < (uint32_t)SPAN && id >= 0 && id < a.V) add(o);
  }
  __syncthreads();
}

// x[e] for a lane-varying e, by a three-level merge under bit masks of e. Integer
// merges, not selects: a select between two elements of one array may be folded into
// an indexed load, which would move the whole array to scratch memory.
__device__ __forceinline__ uint32_t merge_bits(uint32_t lo, uint32_t hi, uint32_t m) {
  return lo ^ ((lo ^ hi) & m);
}
__device__ __forceinline__ float pick8(const float (&x)[EPT], int e) {
  const uint32_t m0 = 0u - ((uint32_t)e & 1u), m1 = 0u - (((uint32_t)e >> 1) & 1u);
  const uint32_t m2 = 0u - (((uint32_t)e >> 2) & 1u);
  uint32_t a[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    a[q] = merge_bits(__float_as_uint(x[2 * q]), __float_as_uint(x[2 * q + 1]), m0);
  return __uint_as_float(merge_bits(merge_bits(a[0], a[1], m1), merge_bits(a[2], a[3], m1), m2));
}

// Uniform element `idx` of row r's noise vector: injected, or Philox at the row's
// (seed, position) key.
template <typename A>
__device__ __forceinline__ float row_uniform(const A& a, int r, const RowParams& p,
                                             int64_t idx) {
  if (a.noise) return a.noise[(int64_t)r * a.noise_stride + idx];
  return philox_uniform(mix64(p.seed, p.position), (uint64_t)idx);
}

}  // namespace strim
