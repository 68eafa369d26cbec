// grammar_kernels.hip — on-device grammar masks (include/strim_grammar.h).
//
// The reference walks a byte trie of the vocabulary through the grammar DFA on the host,
// once per new state, and uploads a bool row per use (GrammarVocab.swift:75-102,
// RequestConstraint.swift:16-43). Here a mask row is one launch: every thread takes one
// token and steps the DFA by the token's bytes (a token is allowed iff no step reaches the
// dead state, which is what the trie walk decides for every token below a live trie
// path); a wave ballot packs 64 decisions into the two u32 words that k_stream reads.
// Produced blocks are kept in a bounded HBM cache, so a state seen before costs a copy.
//
// The table holds every program's states under global ids and grows at its end; an entry
// not interned yet (STRIM_DFA_UNKNOWN) is reported to the host by the walks that meet it
// (a bit per entry marks the pairs already listed).
//
// HBM layout of a strim_grammar:
//   head   [count] uint4      the first 16 bytes of each token, zero padded
//   meta   [count] uint2      {offset of the token's bytes, length | eligible << 31}
//   bytes  [total] u8         every token's bytes (read past the first 16)
//   eosw   [words] u32        end-of-turn ids as mask words
//   cache  [slots][words] u32 mask rows; tag [slots][nblk] u64 {state + 1, last call}
//          per block of a row (a block's words belong to the tag's state)
//   plist  [PCAP] u32 pending entries, pcount, err     (the fixed part, one allocation)
//   next   [cap][256] i32, flags [cap] u8, pbits [cap][8] u32   (grown with the table)
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "common.hpp"
#include "../../include/strim_grammar.h"

namespace strim {

constexpr int GM_T = 256;              // threads of a k_gmask workgroup (one token each)
constexpr int GM_W = GM_T / 32;        // mask words per workgroup
constexpr int GM_HEAD = 16;            // bytes held in a token's head
constexpr int GM_LDS_STATES = 16;      // tables up to this many states walk from LDS
constexpr int GM_DUP = 1024;           // rows a producing workgroup copies to, listed in LDS
constexpr int GM_PCAP = 1 << 16;       // pending (state, byte) entries held on the device
constexpr int GM_UNRES = STRIM_GRAMMAR_UNRESOLVED;

struct GView {
  const uint4* head;
  const uint2* meta;
  const uint8_t* bytes;
  const uint32_t* eosw;
  const int32_t* next;
  const uint8_t* flags;
  uint32_t* cache;
  unsigned long long* tag;
  uint32_t* pbits;
  uint32_t* plist;
  uint32_t* pcount;
  int32_t count, width, words, nblk, nsets, n_states;
};

// Records the unknown entry (st, b) for the host, once until it is handed out.
__device__ __forceinline__ void g_note(const GView& g, int st, uint32_t b) {
  const uint32_t e = (uint32_t)st * 256u + b;
  const uint32_t bit = 1u << (e & 31u);
  if (atomicOr(&g.pbits[e >> 5], bit) & bit) return;
  const uint32_t q = atomicAdd(g.pcount, 1u);
  if (q < (uint32_t)GM_PCAP) g.plist[q] = e;
  else atomicAnd(&g.pbits[e >> 5], ~bit);  // (no room: recorded again when met again)
}

// The state after a token's bytes from live state s: -1 dead, GM_UNRES when a step meets
// an unknown entry (recorded). The first 16 bytes come from the head in registers, longer
// tokens continue from the byte array.
__device__ __forceinline__ int walk_token(const GView& g, int s, uint4 h, uint32_t off,
                                          uint32_t len) {
  const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
  int st = s;
  for (uint32_t i = 0; i < len && st >= 0; ++i) {
    const uint32_t b = i < (uint32_t)GM_HEAD ? (hw[i >> 2] >> (8 * (i & 3))) & 0xFFu
                                             : (uint32_t)g.bytes[off + i];
    const int nx = g.next[(int64_t)st * 256 + b];
    if (nx == STRIM_DFA_UNKNOWN) {
      g_note(g, st, b);
      return GM_UNRES;
    }
    st = nx;
  }
  return st;
}

// Steps the thread's token from st through table `tab` (LDS or global); an unknown entry
// is recorded and ends the walk as dead, with unk set.
template <typename Tab>
__device__ __forceinline__ int walk_mask(Tab tab, const GView& g, uint4 h, uint2 m,
                                         uint32_t len, int st, bool& unk) {
  const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
  for (int i = 0; i < GM_HEAD; ++i) {
    if ((uint32_t)i < len && st >= 0) {
      const uint32_t b = (hw[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      const int nx = tab[st * 256 + (int)b];
      if (nx == STRIM_DFA_UNKNOWN) {
        g_note(g, st, b);
        unk = true;
      }
      st = nx;  // (unknown < 0 ends the walk too)
    }
  }
  for (uint32_t i = GM_HEAD; i < len && st >= 0; ++i) {
    const uint32_t b = g.bytes[m.x + i];
    const int nx = tab[st * 256 + (int)b];
    if (nx == STRIM_DFA_UNKNOWN) {
      g_note(g, st, b);
      unk = true;
    }
    st = nx;
  }
  return st;
}

// The cache slot of block blk of grammar state `key` (one lane). Block blk of a state
// maps to the two ways of set key mod nsets; tag[slot][blk] = {state + 1, the call that
// stored the block} (0: empty). A way is taken for another state only if its state is
// not among this call's keys (in0 / in1: the call's keys hold way 0's / way 1's state),
// so a block read in a call is never rewritten in it and a hit needs no atomic; of two
// free ways the one stored first goes, the insertion order DeviceMasks evicts in
// (RequestConstraint.swift:35-43). Competing claims are settled by compare-and-swap.
// Returns mode 1 (stored by an earlier call: copy it) or 2 (produce it and store it)
// with the slot, or slot -1 (produce without storing).
__device__ __forceinline__ int g_slot(const GView& g, int key, int blk, uint32_t seq,
                                      unsigned long long t0, unsigned long long t1, bool in0,
                                      bool in1, int& mode) {
  mode = 0;
  const uint32_t kp = (uint32_t)key + 1u;
  const unsigned long long me = ((unsigned long long)kp << 32) | seq;
  const int s0 = 2 * (key % g.nsets);
  const unsigned long long tt[2] = {t0, t1};
  for (int wy = 0; wy < 2; ++wy)
    if ((uint32_t)(tt[wy] >> 32) == kp) {
      if ((uint32_t)tt[wy] == seq) return -1;  // (one workgroup per key and block)
      mode = 1;
      return s0 + wy;
    }
  // a victim: an empty way, else one whose state this call does not use, the one stored
  // first
  bool ok[2] = {(tt[0] >> 32) == 0ull || !in0, (tt[1] >> 32) == 0ull || !in1};
  for (int it = 0; it < 2; ++it) {
    int wy = -1;
    if (ok[0] && (!ok[1] || (uint32_t)tt[0] <= (uint32_t)tt[1])) wy = 0;
    else if (ok[1]) wy = 1;
    if (wy < 0) return -1;
    unsigned long long* tp = &g.tag[(int64_t)(s0 + wy) * g.nblk + blk];
    if (atomicCAS(tp, tt[wy], me) == tt[wy]) {
      mode = 2;
      return s0 + wy;
    }
    ok[wy] = false;  // taken by another claim of this call (its state is in the call)
  }
  return -1;
}

// Grid (nblk, n): workgroup (blk, r) produces mask words blk * GM_W .. of row r. Thread t
// walks token blk * GM_T + t; wave w's ballot gives words blk * GM_W + 2 w + {0, 1}.
// (One token per thread measured fastest to produce: 8.0 us for a 151,936-token row of a
// JSON-string state against 9.8 and 14.3 with two and four, before LDS staging; the walk
// is a chain of dependent table lookups, and more waves hide more of it than lockstep
// walks do. Staging a small DFA in LDS took 8 such rows from 18.6 to 12.4 us.)
// Rows with one key: the first row's workgroups produce the words and write them to every
// such row; the later rows' workgroups end at once. A cached block is used only when an
// earlier call produced it: the kernel boundary has made its words visible, so plain
// loads and stores suffice; a block whose walk met an unknown entry is not stored.
__global__ __launch_bounds__(GM_T) void k_gmask(GView g, const int32_t* keys, int n,
                                                uint32_t* out, int64_t out_stride,
                                                uint32_t seq) {
  __shared__ int s_tab[GM_LDS_STATES * 256];
  __shared__ int s_dup[GM_DUP];
  __shared__ int s_ndup, s_slot, s_mode;
  const int blk = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  const int lane = t & (WAVE - 1), w = wave_id();
  const int key = keys[r];
  const bool grammar = key >= 0 && key < g.n_states;
  const bool cache = grammar && g.nsets > 0;
  const int s0 = cache ? 2 * (key % g.nsets) : 0;
  // writes word wd of every row with this key
  auto put = [&](int wd, uint32_t word, int ndup) {
    out[(int64_t)r * out_stride + wd] = word;
    if (ndup <= GM_DUP) {
      for (int q = 0; q < ndup; ++q) out[(int64_t)s_dup[q] * out_stride + wd] = word;
    } else {
      for (int i = r + 1; i < n; ++i)
        if (keys[i] == key) out[(int64_t)i * out_stride + wd] = word;
    }
  };
  // Wave 0 decides alone: one scan of the call's keys by ballots (an earlier row with
  // this key: this row's workgroups end, that row writes this one; the later rows with
  // it; whether the ways' states are keys of this call), the slot, and on a hit the copy.
  // The tags, both ways' words of this block (used on a hit: a block of a key of this
  // call is not rewritten in it) and the first 64 keys are loaded together (plain loads:
  // tags written by earlier calls are visible, and a claim in this call never takes a
  // block of a key in the call). Modes: 0 produce uncached, 1 done (copied), 2 produce
  // and store, 3 done (a duplicate row).
  if (w == 0) {
    const int wi = blk * GM_W + (lane & (GM_W - 1));
    uint32_t cw = 0u;
    if (cache && lane < 2 * GM_W && wi < g.words)
      cw = g.cache[(int64_t)(s0 + lane / GM_W) * g.words + wi];
    unsigned long long t0 = 0ull, t1 = 0ull;
    if (cache) {
      t0 = g.tag[(int64_t)s0 * g.nblk + blk];
      t1 = g.tag[(int64_t)(s0 + 1) * g.nblk + blk];
    }
    const int kt0 = (int)(uint32_t)(t0 >> 32) - 1, kt1 = (int)(uint32_t)(t1 >> 32) - 1;
    bool earlier = false, in0 = false, in1 = false;
    int ndup = 0;
    for (int i0 = 0; i0 < n; i0 += WAVE) {
      const int i = i0 + lane;
      const bool kin = i < n;
      const int ki = kin ? keys[i] : 0;
      const uint64_t eq = __ballot(kin && ki == key);
      earlier = earlier || (eq & (i0 + WAVE <= r ? ~0ull : (r > i0 ? (1ull << (r - i0)) - 1ull : 0ull))) != 0ull;
      const uint64_t later = eq & (r >= i0 + WAVE ? 0ull : (r >= i0 ? ~0ull << (r - i0) << 1 : ~0ull));
      if (later & (1ull << lane)) {
        const int q = ndup + __popcll(later & ((1ull << lane) - 1ull));
        if (q < GM_DUP) s_dup[q] = i;
      }
      ndup += __popcll(later);
      in0 = in0 || (kt0 >= 0 && __ballot(kin && ki == kt0) != 0ull);
      in1 = in1 || (kt1 >= 0 && __ballot(kin && ki == kt1) != 0ull);
    }
    int mode = earlier ? 3 : 0, slot = -1;
    if (!earlier && cache) {
      if (lane == 0) slot = g_slot(g, key, blk, seq, t0, t1, in0, in1, mode);
      slot = __builtin_amdgcn_readfirstlane(slot);
      mode = __builtin_amdgcn_readfirstlane(mode);
    }
    if (mode == 1) {
      __builtin_amdgcn_wave_barrier();  // (s_dup of this wave's lanes is written)
      if (lane / GM_W == slot - s0 && lane < 2 * GM_W && wi < g.words) put(wi, cw, ndup);
    }
    if (lane == 0) {
      s_mode = mode;
      s_slot = slot;
      s_ndup = ndup;
    }
  }
  __syncthreads();
  const int mode = s_mode, slot = s_slot, ndup = s_ndup;
  if (mode == 1 || mode == 3) return;
  const int id = blk * GM_T + t;
  bool ok, unk = false;
  if (!grammar) {
    ok = key == -1 ? id < g.width : (key < -1 && id == -2 - key && id < g.width);
  } else {
    const uint32_t f = g.flags[key];
    const bool con = (f & STRIM_DFA_CONSUMING) != 0;
    const bool in = id < g.count && id < g.width;
    const int ii = in ? id : 0;  // clamped: every load issued before any wait
    const uint4 h = g.head[ii];
    const uint2 m = g.meta[ii];
    const uint32_t len = m.y & 0x7FFFFFFFu;
    // a token takes part when it exists, is eligible and the state consumes
    int st = in && con && (m.y >> 31) ? key : -1;
    // a table of at most GM_LDS_STATES states is staged in LDS: the walk's chain of
    // dependent lookups then costs LDS latency per byte instead of a cache hit's
    if (g.n_states <= GM_LDS_STATES) {
      const int4* src = (const int4*)g.next;
      const int n4 = g.n_states * 64;
      for (int e = t; e < n4; e += GM_T) ((int4*)s_tab)[e] = src[e];
      __syncthreads();
      st = walk_mask(s_tab, g, h, m, len, st, unk);
    } else {
      st = walk_mask(g.next, g, h, m, len, st, unk);
    }
    ok = st >= 0;
  }
  const bool incomplete = __syncthreads_or(unk);
  const bool store = slot >= 0 && !incomplete;
  const bool acc = grammar && (g.flags[key] & STRIM_DFA_ACCEPTING);
  const uint64_t bal = __ballot(ok);
  const int wo = blk * GM_W + 2 * w + (lane & 1);
  if (lane < 2 && wo < g.words) {
    uint32_t word = lane == 0 ? (uint32_t)bal : (uint32_t)(bal >> 32);
    if (acc) word |= g.eosw[wo];
    put(wo, word, ndup);
    if (store) g.cache[(int64_t)slot * g.words + wo] = word;
  }
  // a claimed block whose walk met an unknown entry is given back (empty)
  if (slot >= 0 && incomplete && t == 0)
    __hip_atomic_store(&g.tag[(int64_t)slot * g.nblk + blk], 0ull, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
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

// strim_grammar_set_next: every entry where[i] is unknown or already to[i] (else *err).
__global__ void k_gcheck(const int32_t* next, const int64_t* where, const int32_t* to, int n,
                         uint32_t* err) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int old = next[where[i]];
  if (old != STRIM_DFA_UNKNOWN && old != to[i]) atomicOr(err, 1u);
}
__global__ void k_gset(int32_t* next, const int64_t* where, const int32_t* to, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) next[where[i]] = to[i];
}
// strim_grammar_pending: forgets the listed entries' marks.
__global__ void k_gunnote(uint32_t* pbits, const uint32_t* plist, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const uint32_t e = plist[i];
    atomicAnd(&pbits[e >> 5], ~(1u << (e & 31u)));
  }
}
// strim_grammar_drop_masks: empties the blocks held by states [first, first + n).
__global__ void k_gdrop(unsigned long long* tag, int64_t ntag, int first, int n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= ntag) return;
  const long long s = (long long)(tag[i] >> 32) - 1;
  if (s >= first && s < (long long)first + n) tag[i] = 0ull;
}

}  // namespace strim

using namespace strim;

struct strim_grammar {
  int32_t device = 0;
  int32_t count = 0, width = 0, words = 0, nblk = 0, slots = 0;
  int32_t n_states = 0, cap = 0;
  void* base = nullptr;  // vocabulary, end-of-turn words, cache, pending list
  int32_t* next = nullptr;
  uint8_t* flags = nullptr;
  uint32_t* pbits = nullptr;
  uint4* head = nullptr;
  uint2* meta = nullptr;
  uint8_t* bytes = nullptr;
  uint32_t* eosw = nullptr;
  uint32_t* cache = nullptr;
  unsigned long long* tag = nullptr;
  uint32_t* plist = nullptr;
  uint32_t* pcount = nullptr;  // and err right after it
  void* stage = nullptr;       // staging of strim_grammar_set_next's arrays
  size_t stage_bytes = 0;
  uint32_t seq = 0;  // calls of k_gmask, skipping 0
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
  return GView{g->head, g->meta, g->bytes, g->eosw, g->next, g->flags, g->cache, g->tag,
               g->pbits, g->plist, g->pcount, g->count, g->width, g->words,
               g->nblk, g->slots / 2, g->n_states};
}

int g_status() { return hipGetLastError() == hipSuccess ? STRIM_OK : STRIM_EHIP; }

void g_clear(void* p, int64_t words, hipStream_t st) {
  if (words <= 0) return;
  const int64_t nb = (words + 255) / 256;
  hipLaunchKernelGGL(k_gclear, dim3((unsigned)(nb < 1024 ? nb : 1024)), dim3(256), 0, st,
                     (uint32_t*)p, words);
}

constexpr int32_t G_MAX_STATES = 1 << 23;  // table offsets stay below 2^31

// The table's arrays for cap states: the first `keep` states copied from the old arrays,
// the marks of the others cleared. Runs with the device current; synchronises st.
int g_grow(strim_grammar* g, int32_t cap, int32_t keep, hipStream_t st) {
  int32_t* nx = nullptr;
  uint8_t* fl = nullptr;
  uint32_t* pb = nullptr;
  if (hipMalloc(&nx, (size_t)cap * 1024) != hipSuccess) return STRIM_ENOMEM;
  if (hipMalloc(&fl, (size_t)cap) != hipSuccess || hipMalloc(&pb, (size_t)cap * 32) != hipSuccess) {
    (void)hipFree(nx);
    if (fl) (void)hipFree(fl);
    return STRIM_ENOMEM;
  }
  if (keep > 0 &&
      (hipMemcpyAsync(nx, g->next, (size_t)keep * 1024, hipMemcpyDeviceToDevice, st) != hipSuccess ||
       hipMemcpyAsync(fl, g->flags, (size_t)keep, hipMemcpyDeviceToDevice, st) != hipSuccess ||
       hipMemcpyAsync(pb, g->pbits, (size_t)keep * 32, hipMemcpyDeviceToDevice, st) != hipSuccess))
    return STRIM_EHIP;
  g_clear(pb + (size_t)keep * 8, (int64_t)(cap - keep) * 8, st);
  if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) return STRIM_EHIP;
  if (g->next) (void)hipFree(g->next);
  if (g->flags) (void)hipFree(g->flags);
  if (g->pbits) (void)hipFree(g->pbits);
  g->next = nx;
  g->flags = fl;
  g->pbits = pb;
  g->cap = cap;
  return STRIM_OK;
}

// host check of n rows of table entries: in [-2, limit)
bool g_rows_ok(const int32_t* next, int64_t n_entries, int32_t limit) {
  for (int64_t i = 0; i < n_entries; ++i)
    if (next[i] < STRIM_DFA_UNKNOWN || next[i] >= limit) return false;
  return true;
}

}  // namespace

extern "C" {

int strim_grammar_create(strim_grammar** out, int32_t device, int32_t count,
                         const uint32_t* offsets, const uint8_t* bytes, const uint8_t* skip,
                         int32_t width, const int32_t* eos, int32_t n_eos,
                         int32_t cache_slots) {
  if (!out) return STRIM_EINVAL;
  *out = nullptr;
  if (count <= 0 || !offsets || width <= 0 || n_eos < 0 || (n_eos > 0 && !eos) ||
      cache_slots < 0 || offsets[0] != 0u)
    return STRIM_EINVAL;
  for (int32_t i = 0; i < count; ++i)
    if (offsets[i + 1] < offsets[i]) return STRIM_EINVAL;
  const uint32_t total = offsets[count];
  if (total > 0 && !bytes) return STRIM_EINVAL;
  for (int32_t e = 0; e < n_eos; ++e)
    if (eos[e] < 0) return STRIM_EINVAL;
  const int32_t words = (width + 31) / 32;
  const int32_t nblk = (width + GM_T - 1) / GM_T;
  const int32_t slots = cache_slots / 2 * 2;  // two ways a set
  // host staging of the device layout
  std::vector<uint4> h_head((size_t)count);
  std::vector<uint2> h_meta((size_t)count);
  std::vector<uint32_t> h_eosw((size_t)words, 0u);
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
  g->slots = slots;
  const size_t o_head = 0;
  const size_t o_meta = g_align(o_head + (size_t)count * sizeof(uint4));
  const size_t o_bytes = g_align(o_meta + (size_t)count * sizeof(uint2));
  const size_t o_eos = g_align(o_bytes + (size_t)total + 16);
  const size_t o_cache = g_align(o_eos + (size_t)words * 4);
  const size_t o_tag = g_align(o_cache + (size_t)slots * words * 4);
  const size_t o_plist = g_align(o_tag + (size_t)slots * nblk * 8);
  const size_t o_pcount = g_align(o_plist + (size_t)GM_PCAP * 4);
  const size_t size = g_align(o_pcount + 8);
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
    g->tag = (unsigned long long*)(p + o_tag);
    g->plist = (uint32_t*)(p + o_plist);
    g->pcount = (uint32_t*)(p + o_pcount);
    if (hipMemcpy(g->head, h_head.data(), (size_t)count * sizeof(uint4), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(g->meta, h_meta.data(), (size_t)count * sizeof(uint2), hipMemcpyHostToDevice) != hipSuccess ||
        (total > 0 && hipMemcpy(g->bytes, bytes, total, hipMemcpyHostToDevice) != hipSuccess) ||
        hipMemcpy(g->eosw, h_eosw.data(), (size_t)words * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(g->tag, 0, (size_t)slots * nblk * 8) != hipSuccess ||
        hipMemset(g->pcount, 0, 8) != hipSuccess)
      return STRIM_EHIP;
    return STRIM_OK;
  });
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
    if (g->pbits) (void)hipFree(g->pbits);
    if (g->stage) (void)hipFree(g->stage);
    if (g->base) (void)hipFree(g->base);
    return STRIM_OK;
  });
  delete g;
  return rc;
}

int strim_grammar_set_dfa(strim_grammar* g, void* stream, int32_t n_states,
                          const int32_t* next, const uint8_t* flags) {
  // (the reference caps its DFA at 200,000 states, GrammarDFA.swift:16)
  if (!g || n_states <= 0 || n_states > G_MAX_STATES || !next || !flags) return STRIM_EINVAL;
  if (!g_rows_ok(next, (int64_t)n_states * 256, n_states)) return STRIM_EINVAL;
  return g_on_device(g->device, [&]() -> int {
    hipStream_t st = (hipStream_t)stream;
    // the previous table may still be read by queued work on this stream
    if (hipStreamSynchronize(st) != hipSuccess) return STRIM_EHIP;
    g->n_states = 0;
    if (n_states > g->cap) {
      const int rc = g_grow(g, n_states, 0, st);
      if (rc != STRIM_OK) return rc;
    }
    if (hipMemcpy(g->next, next, (size_t)n_states * 1024, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(g->flags, flags, (size_t)n_states, hipMemcpyHostToDevice) != hipSuccess)
      return STRIM_EHIP;
    g_clear(g->pbits, (int64_t)g->cap * 8, st);
    // (a cached block names its state only: a new table invalidates every one)
    g_clear(g->tag, (int64_t)g->slots * g->nblk * 2, st);
    g_clear(g->pcount, 2, st);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
      return STRIM_EHIP;
    g->n_states = n_states;
    return STRIM_OK;
  });
}

int strim_grammar_append_states(strim_grammar* g, void* stream, int32_t n_new,
                                const int32_t* next, const uint8_t* flags, int32_t* first_out) {
  if (!g || n_new <= 0 || !next || !flags || !first_out) return STRIM_EINVAL;
  if (n_new > G_MAX_STATES - g->n_states) return STRIM_ECAPACITY;
  const int32_t first = g->n_states, total = first + n_new;
  if (!g_rows_ok(next, (int64_t)n_new * 256, total)) return STRIM_EINVAL;
  return g_on_device(g->device, [&]() -> int {
    hipStream_t st = (hipStream_t)stream;
    if (total > g->cap) {
      int64_t cap = g->cap < 64 ? 64 : 2 * (int64_t)g->cap;
      if (cap < total) cap = total;
      if (cap > G_MAX_STATES) cap = G_MAX_STATES;
      const int rc = g_grow(g, (int32_t)cap, first, st);
      if (rc != STRIM_OK) return rc;
    }
    // (queued calls read only states below first; the new rows are beyond them)
    if (hipMemcpyAsync(g->next + (size_t)first * 256, next, (size_t)n_new * 1024,
                       hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(g->flags + first, flags, (size_t)n_new, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return STRIM_EHIP;
    g->n_states = total;
    *first_out = first;
    return STRIM_OK;
  });
}

int strim_grammar_set_next(strim_grammar* g, void* stream, int32_t n, const int64_t* where,
                           const int32_t* to) {
  if (!g || n < 0 || (n > 0 && (!where || !to))) return STRIM_EINVAL;
  if (n == 0) return STRIM_OK;
  for (int32_t i = 0; i < n; ++i)
    if (where[i] < 0 || where[i] >= (int64_t)g->n_states * 256 || to[i] < STRIM_DFA_DEAD ||
        to[i] >= g->n_states)
      return STRIM_EINVAL;
  return g_on_device(g->device, [&]() -> int {
    hipStream_t st = (hipStream_t)stream;
    const size_t need = g_align((size_t)n * 8) + (size_t)n * 4;
    if (need > g->stage_bytes) {
      if (g->stage) (void)hipFree(g->stage);
      g->stage = nullptr;
      g->stage_bytes = 0;
      if (hipMalloc(&g->stage, need) != hipSuccess) {
        g->stage = nullptr;
        return STRIM_ENOMEM;
      }
      g->stage_bytes = need;
    }
    int64_t* dw = (int64_t*)g->stage;
    int32_t* dt = (int32_t*)((char*)g->stage + g_align((size_t)n * 8));
    uint32_t* err = g->pcount + 1;
    uint32_t h_err = 0u;
    const unsigned nb = (unsigned)((n + 255) / 256);
    if (hipMemcpyAsync(dw, where, (size_t)n * 8, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(dt, to, (size_t)n * 4, hipMemcpyHostToDevice, st) != hipSuccess)
      return STRIM_EHIP;
    g_clear(err, 1, st);
    hipLaunchKernelGGL(k_gcheck, dim3(nb), dim3(256), 0, st, g->next, dw, dt, n, err);
    if (hipGetLastError() != hipSuccess ||
        hipMemcpyAsync(&h_err, err, 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return STRIM_EHIP;
    if (h_err) return STRIM_EINVAL;
    hipLaunchKernelGGL(k_gset, dim3(nb), dim3(256), 0, st, g->next, dw, dt, n);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
      return STRIM_EHIP;
    return STRIM_OK;
  });
}

int strim_grammar_pending(strim_grammar* g, void* stream, int64_t* out, int32_t cap,
                          int32_t* n_out) {
  if (!g || !n_out || cap < 0 || (cap > 0 && !out)) return STRIM_EINVAL;
  *n_out = 0;
  return g_on_device(g->device, [&]() -> int {
    hipStream_t st = (hipStream_t)stream;
    uint32_t cnt = 0u;
    if (hipMemcpyAsync(&cnt, g->pcount, 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return STRIM_EHIP;
    const int32_t held = (int32_t)(cnt < (uint32_t)GM_PCAP ? cnt : (uint32_t)GM_PCAP);
    const int32_t give = held < cap ? held : cap;
    std::vector<uint32_t> h((size_t)give);
    if (give > 0 &&
        hipMemcpyAsync(h.data(), g->plist, (size_t)give * 4, hipMemcpyDeviceToHost, st) != hipSuccess)
      return STRIM_EHIP;
    if (held > 0)
      hipLaunchKernelGGL(k_gunnote, dim3((unsigned)((held + 255) / 256)), dim3(256), 0, st,
                         g->pbits, g->plist, held);
    g_clear(g->pcount, 1, st);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
      return STRIM_EHIP;
    for (int32_t i = 0; i < give; ++i) out[i] = (int64_t)h[i];
    *n_out = give;
    return STRIM_OK;
  });
}

int strim_grammar_drop_masks(strim_grammar* g, void* stream, int32_t first, int32_t n) {
  if (!g || first < 0 || n < 0) return STRIM_EINVAL;
  if (n == 0 || g->slots == 0) return STRIM_OK;
  const int64_t ntag = (int64_t)g->slots * g->nblk;
  return g_on_device(g->device, [&]() -> int {
    hipLaunchKernelGGL(k_gdrop, dim3((unsigned)((ntag + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, g->tag, ntag, first, n);
    return g_status();
  });
}

int strim_grammar_masks(strim_grammar* g, void* stream, const int32_t* keys, int32_t n,
                        uint32_t* out, int64_t out_stride) {
  if (!g || !keys || !out || n <= 0 || n > 65535 || out_stride < g->words) return STRIM_EINVAL;
  if (g->n_states <= 0) return STRIM_EINVAL;  // no table installed
  return g_on_device(g->device, [&]() -> int {
    if (++g->seq == 0u) g->seq = 1u;
    hipLaunchKernelGGL(k_gmask, dim3((unsigned)g->nblk, (unsigned)n), dim3(GM_T), 0,
                       (hipStream_t)stream, view(g), keys, n, out, out_stride, g->seq);
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
