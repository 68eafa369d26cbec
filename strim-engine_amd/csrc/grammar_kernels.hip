// grammar_kernels.hip — on-device grammar masks (include/strim_grammar.h).
//
// The reference walks a byte trie of the vocabulary through the grammar DFA on the host,
// once per new state, and uploads a bool row per use (GrammarVocab.swift:75-102,
// RequestConstraint.swift:16-43). Here a mask row is one launch: every thread takes one
// token and steps the DFA by the token's bytes (a token is allowed iff no step reaches the
// dead state, which is what the trie walk decides for every token below a live trie
// path); a wave ballot packs 64 decisions into the two u32 words that k_stream reads.
// Produced blocks of a cached state are kept in HBM, so a state seen before costs a copy.
//
// HBM layout of a strim_grammar:
//   head   [count] uint4      the first 16 bytes of each token, zero padded
//   meta   [count] uint2      {offset of the token's bytes, length | eligible << 31}
//   bytes  [total] u8         every token's bytes (read past the first 16)
//   eosw   [words] u32        end-of-turn ids as mask words
//   next   [n_states][256] i32, flags [n_states] u8   the DFA
//   cache  [cache_states][words] u32, ready [cache_states][nblk] u32
#include <stdlib.h>
#include <string.h>

#include "common.hpp"
#include "../../include/strim_grammar.h"

namespace strim {

constexpr int GM_T = 256;              // threads of a k_gmask workgroup
constexpr int GM_Q = 1;                // tokens per thread (walked in lockstep)
constexpr int GM_TOK = GM_T * GM_Q;    // tokens per workgroup
constexpr int GM_W = GM_TOK / 32;      // mask words per workgroup
constexpr int GM_HEAD = 16;            // bytes held in a token's head

struct GView {
  const uint4* head;
  const uint2* meta;
  const uint8_t* bytes;
  const uint32_t* eosw;
  const int32_t* next;
  const uint8_t* flags;
  uint32_t* cache;
  uint32_t* ready;
  int32_t count, width, words, nblk, cache_states, n_states;
};

// The state after a token's bytes from live state s (-1 = dead). The first 16 bytes come
// from the head in registers; longer tokens continue from the byte array.
__device__ __forceinline__ int walk_token(const GView& g, int s, uint4 h, uint32_t off,
                                          uint32_t len) {
  const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
  int st = s;
#pragma unroll
  for (int i = 0; i < GM_HEAD; ++i) {
    if ((uint32_t)i < len && st >= 0) {
      const uint32_t b = (hw[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      st = g.next[(int64_t)st * 256 + b];
    }
  }
  for (uint32_t i = GM_HEAD; i < len && st >= 0; ++i)
    st = g.next[(int64_t)st * 256 + g.bytes[off + i]];
  return st;
}

constexpr int GM_LDS_STATES = 16;      // DFAs up to this many states walk from LDS

// Steps every token of the thread from st[q] through table `tab` (LDS or global).
template <typename Tab>
__device__ __forceinline__ void walk_all(Tab tab, const GView& g, const uint4* h,
                                         const uint2* m, const uint32_t* len, int* st) {
#pragma unroll
  for (int i = 0; i < GM_HEAD; ++i) {
#pragma unroll
    for (int q = 0; q < GM_Q; ++q) {
      if ((uint32_t)i < len[q] && st[q] >= 0) {
        const uint32_t hw = i < 4 ? h[q].x : i < 8 ? h[q].y : i < 12 ? h[q].z : h[q].w;
        const uint32_t b = (hw >> (8 * (i & 3))) & 0xFFu;
        st[q] = tab[st[q] * 256 + (int)b];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < GM_Q; ++q)
    for (uint32_t i = GM_HEAD; i < len[q] && st[q] >= 0; ++i)
      st[q] = tab[st[q] * 256 + (int)g.bytes[m[q].x + i]];
}

// Grid (nblk, n): workgroup (blk, r) produces mask words blk * GM_W .. of row r. Thread t
// walks tokens blk * GM_TOK + q * 256 + t (q < GM_Q) in lockstep, one table lookup of each
// in flight at a time; wave w's ballot for q gives words blk * GM_W + q * 8 + 2 w + {0, 1}.
// (One token per thread measured fastest to produce: 8.0 us for a 151,936-token row of a
// JSON-string state against 9.8 and 14.3 with two and four, before LDS staging; the walk
// is a chain of dependent table lookups, and more waves hide more of it than lockstep
// walks do. Staging a small DFA in LDS took 8 such rows from 18.6 to 12.4 us.)
// A cached block is used only when an earlier launch produced it (ready holds the
// producing launch's sequence number, never 0): the kernel boundary has made its words
// visible, so plain loads and stores suffice. Blocks produced in this launch are produced
// again by any other row that needs them (the same words, written twice).
__global__ __launch_bounds__(GM_T) void k_gmask(GView g, const int32_t* keys, uint32_t* out,
                                                int64_t out_stride, uint32_t seq) {
  __shared__ int s_tab[GM_LDS_STATES * 256];
  const int blk = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  const int lane = t & (WAVE - 1), w = t / WAVE;
  const int key = keys[r];
  uint32_t* orow = out + (int64_t)r * out_stride;
  const bool grammar = key >= 0 && key < g.n_states;
  const bool cached = grammar && key < g.cache_states;
  if (cached) {
    const uint32_t rd = g.ready[(int64_t)key * g.nblk + blk];
    if (rd != 0u && rd != seq) {
      if (t < GM_W) {
        const int wi = blk * GM_W + t;
        if (wi < g.words) orow[wi] = g.cache[(int64_t)key * g.words + wi];
      }
      return;
    }
  }
  bool ok[GM_Q];
  if (key == -1 || key < -1 || !grammar) {
#pragma unroll
    for (int q = 0; q < GM_Q; ++q) {
      const int id = blk * GM_TOK + q * GM_T + t;
      ok[q] = key == -1 ? id < g.width : (key < -1 && id == -2 - key && id < g.width);
    }
  } else {
    const uint32_t f = g.flags[key];
    const bool con = (f & STRIM_DFA_CONSUMING) != 0;
    uint4 h[GM_Q];
    uint2 m[GM_Q];
    int st[GM_Q];
    uint32_t len[GM_Q];
#pragma unroll
    for (int q = 0; q < GM_Q; ++q) {
      const int id = blk * GM_TOK + q * GM_T + t;
      const bool in = id < g.count && id < g.width;
      const int ii = in ? id : 0;  // clamped: every load issued before any wait
      h[q] = g.head[ii];
      m[q] = g.meta[ii];
      len[q] = m[q].y & 0x7FFFFFFFu;
      // a token takes part when it exists, is eligible and the state consumes
      st[q] = in && con && (m[q].y >> 31) ? key : -1;
    }
    // a DFA of at most GM_LDS_STATES states is staged in LDS: the walk's chain of
    // dependent lookups then costs LDS latency per byte instead of a cache hit's
    if (g.n_states <= GM_LDS_STATES) {
      const int4* src = (const int4*)g.next;
      const int n4 = g.n_states * 64;
      for (int e = t; e < n4; e += GM_T) ((int4*)s_tab)[e] = src[e];
      __syncthreads();
      walk_all(s_tab, g, h, m, len, st);
    } else {
      walk_all(g.next, g, h, m, len, st);
    }
#pragma unroll
    for (int q = 0; q < GM_Q; ++q) ok[q] = st[q] >= 0;
  }
  const bool acc = grammar && (g.flags[key] & STRIM_DFA_ACCEPTING);
#pragma unroll
  for (int q = 0; q < GM_Q; ++q) {
    const uint64_t bal = __ballot(ok[q]);
    const int wi = blk * GM_W + q * (GM_T / 32) + 2 * w + (lane & 1);
    if (lane < 2 && wi < g.words) {
      uint32_t word = lane == 0 ? (uint32_t)bal : (uint32_t)(bal >> 32);
      if (acc) word |= g.eosw[wi];
      orow[wi] = word;
      if (cached) g.cache[(int64_t)key * g.words + wi] = word;
    }
  }
  if (cached && t == 0) g.ready[(int64_t)key * g.nblk + blk] = seq;
}

// One thread per request: the keys of its k + 1 verify rows.
__global__ void k_gadvance(GView g, const int32_t* state, int B, const int32_t* tokens, int k,
                           int32_t* keys_out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  int s = state[b];
  int32_t* o = keys_out + (int64_t)b * (k + 1);
  o[0] = s;
  for (int i = 0; i < k; ++i) {
    if (s >= 0 && s < g.n_states) {
      const int d = tokens[(int64_t)b * k + i];
      if (d >= 0 && d < g.count) {
        const uint2 m = g.meta[d];
        s = walk_token(g, s, g.head[d], m.x, m.y & 0x7FFFFFFFu);  // dead: -1 = free
      }
    }
    o[i + 1] = s;
  }
}

// ---- per-request constraint state (RequestConstraint.key / step) --------------------
__device__ __forceinline__ int rq_key(const strim_request_state& s) {
  if (s.in_think)
    return (s.budget >= 0 && s.close_id >= 0 && s.count >= s.budget) ? -2 - s.close_id : -1;
  return s.g >= 0 ? s.g : -1;
}
__device__ __forceinline__ strim_request_state rq_step(const GView& g, strim_request_state s,
                                                        int t) {
  if (s.in_think) {
    if (t == s.close_id) s.in_think = 0;
    else s.count += 1;
  } else if (s.g >= 0 && s.g < g.n_states && t >= 0 && t < g.count) {
    const uint2 m = g.meta[t];
    s.g = walk_token(g, s.g, g.head[t], m.x, m.y & 0x7FFFFFFFu);  // dead: -1
  }
  return s;
}
// the step left a live grammar state for dead (RequestConstraint.swift:107,142)
__device__ __forceinline__ bool rq_died(const strim_request_state& prev,
                                        const strim_request_state& next) {
  return !prev.in_think && prev.g >= 0 && next.g < 0;
}

// One thread per request: the key of its next row and of its k verify rows.
__global__ void k_rkeys(GView g, const strim_request_state* states, int B,
                        const int32_t* drafts, int k, int32_t* keys_out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  strim_request_state s = states[b];
  int32_t* o = keys_out + (int64_t)b * (k + 1);
  o[0] = rq_key(s);
  bool live = true;
  for (int i = 0; i < k; ++i) {
    if (live) {
      const strim_request_state prev = s;
      s = rq_step(g, s, drafts[(int64_t)b * k + i]);
      if (rq_died(prev, s)) live = false;
    }
    o[i + 1] = live ? rq_key(s) : -1;
  }
}

// One thread per request: its state after drafts[0 .. accepted) and last.
__global__ void k_radvance(GView g, strim_request_state* states, int B, const int32_t* drafts,
                           int k, const int32_t* accepted, const int32_t* last) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  strim_request_state s = states[b];
  const int t_last = last[b];
  if (t_last >= 0) {
    int n = accepted ? accepted[b] : 0;
    n = n < 0 ? 0 : (n > k ? k : n);
    for (int i = 0; i <= n; ++i) {
      const int t = i < n ? drafts[(int64_t)b * k + i] : t_last;
      const strim_request_state nx = rq_step(g, s, t);
      const bool died = rq_died(s, nx);
      s = nx;
      if (died) s.violated = 1;
    }
  }
  states[b] = s;
}

__global__ void k_gclear(uint32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace strim

using namespace strim;

struct strim_grammar {
  int32_t device = 0;
  int32_t count = 0, width = 0, words = 0, nblk = 0, cache_states = 0, n_states = 0;
  void* base = nullptr;  // vocabulary, end-of-turn words, cache, ready flags
  int32_t* next = nullptr;
  uint8_t* flags = nullptr;
  uint4* head = nullptr;
  uint2* meta = nullptr;
  uint8_t* bytes = nullptr;
  uint32_t* eosw = nullptr;
  uint32_t* cache = nullptr;
  uint32_t* ready = nullptr;
  uint32_t seq = 0;  // launches of k_gmask, skipping 0
};

namespace {

template <typename F>
int g_on_device(int32_t device, F fn) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return STRIM_EHIP;
  if (cur != device && hipSetDevice(device) != hipSuccess) return STRIM_EHIP;
  const int rc = fn();
  if (cur != device) (void)hipSetDevice(cur);
  return rc;
}

size_t g_align(size_t x) { return (x + 255) / 256 * 256; }

GView view(const strim_grammar* g) {
  return GView{g->head, g->meta, g->bytes, g->eosw, g->next, g->flags, g->cache, g->ready,
               g->count, g->width, g->words, g->nblk, g->cache_states, g->n_states};
}

int g_status() { return hipGetLastError() == hipSuccess ? STRIM_OK : STRIM_EHIP; }

}  // namespace

extern "C" {

int strim_grammar_create(strim_grammar** out, int32_t device, int32_t count,
                         const uint32_t* offsets, const uint8_t* bytes, const uint8_t* skip,
                         int32_t width, const int32_t* eos, int32_t n_eos,
                         int32_t cache_states) {
  if (!out) return STRIM_EINVAL;
  *out = nullptr;
  if (count <= 0 || !offsets || width <= 0 || n_eos < 0 || (n_eos > 0 && !eos) ||
      cache_states < 0 || offsets[0] != 0u)
    return STRIM_EINVAL;
  for (int32_t i = 0; i < count; ++i)
    if (offsets[i + 1] < offsets[i]) return STRIM_EINVAL;
  const uint32_t total = offsets[count];
  if (total > 0 && !bytes) return STRIM_EINVAL;
  for (int32_t e = 0; e < n_eos; ++e)
    if (eos[e] < 0) return STRIM_EINVAL;
  const int32_t words = (width + 31) / 32;
  const int32_t nblk = (width + GM_TOK - 1) / GM_TOK;
  // host staging of the device layout
  uint4* h_head = (uint4*)calloc((size_t)count, sizeof(uint4));
  uint2* h_meta = (uint2*)calloc((size_t)count, sizeof(uint2));
  uint32_t* h_eosw = (uint32_t*)calloc((size_t)words, sizeof(uint32_t));
  if (!h_head || !h_meta || !h_eosw) {
    free(h_head); free(h_meta); free(h_eosw);
    return STRIM_ENOMEM;
  }
  for (int32_t i = 0; i < count; ++i) {
    const uint32_t o = offsets[i], len = offsets[i + 1] - o;
    uint8_t hb[16] = {0};
    if (len) memcpy(hb, bytes + o, len < 16u ? len : 16u);
    memcpy(&h_head[i], hb, 16);
    const bool elig = len > 0 && !(skip && skip[i]);
    h_meta[i] = make_uint2(o, (len & 0x7FFFFFFFu) | (elig ? 0x80000000u : 0u));
  }
  for (int32_t e = 0; e < n_eos; ++e)
    if (eos[e] < width) h_eosw[eos[e] >> 5] |= 1u << (eos[e] & 31);

  strim_grammar* g = new strim_grammar();
  g->device = device;
  g->count = count;
  g->width = width;
  g->words = words;
  g->nblk = nblk;
  g->cache_states = cache_states;
  const size_t o_head = 0;
  const size_t o_meta = g_align(o_head + (size_t)count * sizeof(uint4));
  const size_t o_bytes = g_align(o_meta + (size_t)count * sizeof(uint2));
  const size_t o_eos = g_align(o_bytes + (size_t)total + 16);
  const size_t o_cache = g_align(o_eos + (size_t)words * 4);
  const size_t o_ready = g_align(o_cache + (size_t)cache_states * words * 4);
  const size_t size = g_align(o_ready + (size_t)cache_states * nblk * 4);
  const int rc = g_on_device(device, [&]() -> int {
    if (hipMalloc(&g->base, size) != hipSuccess) {
      g->base = nullptr;
      return STRIM_ENOMEM;
    }
    char* p = (char*)g->base;
    g->head = (uint4*)(p + o_head);
    g->meta = (uint2*)(p + o_meta);
    g->bytes = (uint8_t*)(p + o_bytes);
    g->eosw = (uint32_t*)(p + o_eos);
    g->cache = (uint32_t*)(p + o_cache);
    g->ready = (uint32_t*)(p + o_ready);
    if (hipMemcpy(g->head, h_head, (size_t)count * sizeof(uint4), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(g->meta, h_meta, (size_t)count * sizeof(uint2), hipMemcpyHostToDevice) != hipSuccess ||
        (total > 0 && hipMemcpy(g->bytes, bytes, total, hipMemcpyHostToDevice) != hipSuccess) ||
        hipMemcpy(g->eosw, h_eosw, (size_t)words * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(g->ready, 0, (size_t)cache_states * nblk * 4) != hipSuccess)
      return STRIM_EHIP;
    return STRIM_OK;
  });
  free(h_head);
  free(h_meta);
  free(h_eosw);
  if (rc != STRIM_OK) {
    strim_grammar_destroy(g);
    return rc;
  }
  *out = g;
  return STRIM_OK;
}

int strim_grammar_destroy(strim_grammar* g) {
  if (!g) return STRIM_EINVAL;
  const int rc = g_on_device(g->device, [&]() -> int {
    if (g->next) (void)hipFree(g->next);
    if (g->flags) (void)hipFree(g->flags);
    if (g->base) (void)hipFree(g->base);
    return STRIM_OK;
  });
  delete g;
  return rc;
}

int strim_grammar_set_dfa(strim_grammar* g, void* stream, int32_t n_states,
                          const int32_t* next, const uint8_t* flags) {
  // table offsets stay below 2^31 (the reference caps its DFA at 200,000 states)
  if (!g || n_states <= 0 || n_states > (1 << 23) || !next || !flags) return STRIM_EINVAL;
  const int64_t n = (int64_t)n_states * 256;
  for (int64_t i = 0; i < n; ++i)
    if (next[i] < -1 || next[i] >= n_states) return STRIM_EINVAL;
  return g_on_device(g->device, [&]() -> int {
    hipStream_t st = (hipStream_t)stream;
    // the previous table may still be read by queued work on this stream
    if (hipStreamSynchronize(st) != hipSuccess) return STRIM_EHIP;
    if (g->next) (void)hipFree(g->next);
    if (g->flags) (void)hipFree(g->flags);
    g->next = nullptr;
    g->flags = nullptr;
    g->n_states = 0;
    if (hipMalloc(&g->next, (size_t)n * 4) != hipSuccess) {
      g->next = nullptr;
      return STRIM_ENOMEM;
    }
    if (hipMalloc(&g->flags, (size_t)n_states) != hipSuccess) {
      g->flags = nullptr;
      return STRIM_ENOMEM;
    }
    if (hipMemcpy(g->next, next, (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(g->flags, flags, (size_t)n_states, hipMemcpyHostToDevice) != hipSuccess)
      return STRIM_EHIP;
    const int64_t nr = (int64_t)g->cache_states * g->nblk;
    if (nr > 0) {
      hipLaunchKernelGGL(k_gclear, dim3((unsigned)((nr + 255) / 256 < 1024 ? (nr + 255) / 256 : 1024)),
                         dim3(256), 0, st, g->ready, nr);
      if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
        return STRIM_EHIP;
    }
    g->n_states = n_states;
    return STRIM_OK;
  });
}

int strim_grammar_masks(strim_grammar* g, void* stream, const int32_t* keys, int32_t n,
                        uint32_t* out, int64_t out_stride) {
  if (!g || !keys || !out || n <= 0 || n > 65535 || out_stride < g->words) return STRIM_EINVAL;
  if (g->n_states <= 0) return STRIM_EINVAL;  // no DFA installed
  return g_on_device(g->device, [&]() -> int {
    if (++g->seq == 0u) g->seq = 1u;
    hipLaunchKernelGGL(k_gmask, dim3((unsigned)g->nblk, (unsigned)n), dim3(GM_T), 0,
                       (hipStream_t)stream, view(g), keys, out, out_stride, g->seq);
    return g_status();
  });
}

int strim_grammar_advance(strim_grammar* g, void* stream, const int32_t* state, int32_t B,
                          const int32_t* tokens, int32_t k, int32_t* keys_out) {
  if (!g || !state || !keys_out || B <= 0 || k < 0 || (k > 0 && !tokens)) return STRIM_EINVAL;
  if (g->n_states <= 0) return STRIM_EINVAL;
  return g_on_device(g->device, [&]() -> int {
    hipLaunchKernelGGL(k_gadvance, dim3((unsigned)((B + 63) / 64)), dim3(64), 0,
                       (hipStream_t)stream, view(g), state, B, tokens, k, keys_out);
    return g_status();
  });
}

int strim_request_keys(strim_grammar* g, void* stream, const strim_request_state* states,
                       int32_t B, const int32_t* drafts, int32_t k, int32_t* keys_out) {
  if (!g || !states || !keys_out || B <= 0 || k < 0 || (k > 0 && !drafts)) return STRIM_EINVAL;
  return g_on_device(g->device, [&]() -> int {
    hipLaunchKernelGGL(k_rkeys, dim3((unsigned)((B + 63) / 64)), dim3(64), 0,
                       (hipStream_t)stream, view(g), states, B, drafts, k, keys_out);
    return g_status();
  });
}

int strim_request_advance(strim_grammar* g, void* stream, strim_request_state* states,
                          int32_t B, const int32_t* drafts, int32_t k, const int32_t* accepted,
                          const int32_t* last) {
  if (!g || !states || !last || B <= 0 || k < 0 || (k > 0 && !drafts)) return STRIM_EINVAL;
  return g_on_device(g->device, [&]() -> int {
    hipLaunchKernelGGL(k_radvance, dim3((unsigned)((B + 63) / 64)), dim3(64), 0,
                       (hipStream_t)stream, view(g), states, B, drafts, k, accepted, last);
    return g_status();
  });
}

}  // extern "C"
