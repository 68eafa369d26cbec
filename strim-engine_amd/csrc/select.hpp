// select.hpp — workgroup-level building blocks of the finalize steps: block scans and
// reductions, top-2 merges, the ladder bound of a chunk's top-k, rank and bitonic sorts
// of order keys in LDS, and the radix select of the k-th smallest key.
//
// Every helper is called by all NT threads of the workgroup (it contains barriers).
// Floating-point reductions use a fixed combination order, so results do not depend on
// scheduling.
#pragma once

#include <climits>

#include "kernels.hpp"

namespace strim {

// Ladder rung of d >= 0: 0 for d == 0, else ceil(4 log2 d) + 29 clamped to [1, 63].
// Monotone in d (equal d -> equal rung), width ratio 2^(1/4); bounds a chunk's top-k.
constexpr int NRUNG = 64;
__device__ __forceinline__ int ladder_rung(float d) {
  if (!(d > 0.0f)) return 0;
  if (!(d < 1e30f)) return NRUNG - 1;
  const int r = (int)ceilf(4.0f * __log2f(d)) + 29;
  return r < 1 ? 1 : (r > NRUNG - 1 ? NRUNG - 1 : r);
}

__device__ __forceinline__ bool row_nofilter(const RowParams& p, int V) {
  return !(p.top_k > 0 && p.top_k < V) && !(p.min_p > 0.0f) && !(p.top_p < 1.0f);
}

// Exclusive prefix and wave total of per-lane counts in [0, 31] via ballots.
// Exclusive prefix over the wave of a per-lane count c < 2^BITS (one ballot per bit).
template <int BITS>
__device__ __forceinline__ int wave_excl_count_bits(int c, int* total) {
  int ex = 0, tot = 0;
#pragma unroll
  for (int bit = 0; bit < BITS; ++bit) {
    const uint64_t m = __ballot((c >> bit) & 1);
    ex += lanes_below(m) << bit;
    tot += __popcll(m) << bit;
  }
  *total = tot;
  return ex;
}

__device__ __forceinline__ int wave_excl_count32(int c, int* total) {
  int ex = 0, tot = 0;
#pragma unroll
  for (int bit = 0; bit < 5; ++bit) {
    const uint64_t m = __ballot((c >> bit) & 1);
    ex += lanes_below(m) << bit;
    tot += __popcll(m) << bit;
  }
  *total = tot;
  return ex;
}

// Block exclusive scan of one uint32 per thread; *total gets the sum. scratch >= NT/64.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* scratch,
                                                        uint32_t* total) {
  const int lane = threadIdx.x & (WAVE - 1), w = wave_id();
  const uint32_t inc = wave_incl_scan_u32(v);
  if (lane == WAVE - 1) scratch[w] = inc;
  __syncthreads();
  uint32_t base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / WAVE; ++i) {
    const uint32_t s = scratch[i];
    if (i < w) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + inc - v;
}

template <int NT>
__device__ __forceinline__ int block_or(int v, int* scratch) {
  v = wave_or_i(v);
  if ((threadIdx.x & (WAVE - 1)) == 0) scratch[threadIdx.x / WAVE] = v;
  __syncthreads();
  int b = 0;
#pragma unroll
  for (int q = 0; q < NT / WAVE; ++q) b |= scratch[q];
  __syncthreads();
  return b;
}

template <int NT>
__device__ __forceinline__ uint64_t block_or_u64(uint64_t v, uint64_t* scratch) {
  const uint32_t lo = (uint32_t)wave_or_i((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)wave_or_i((int)(uint32_t)(v >> 32));
  if ((threadIdx.x & (WAVE - 1)) == 0) scratch[threadIdx.x / WAVE] = ((uint64_t)hi << 32) | lo;
  __syncthreads();
  uint64_t b = 0;
#pragma unroll
  for (int q = 0; q < NT / WAVE; ++q) b |= scratch[q];
  __syncthreads();
  return b;
}

template <int NT>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* scratch) {
  v = wave_max_u64(v);
  if ((threadIdx.x & (WAVE - 1)) == 0) scratch[threadIdx.x / WAVE] = v;
  __syncthreads();
  uint64_t b = 0;
#pragma unroll
  for (int q = 0; q < NT / WAVE; ++q) b = scratch[q] > b ? scratch[q] : b;
  __syncthreads();
  return b;
}

// Block sum of one double per thread in a fixed order (deterministic).
template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, double* scratch) {
  v = wave_sum(v);
  if ((threadIdx.x & (WAVE - 1)) == 0) scratch[threadIdx.x / WAVE] = v;
  __syncthreads();
  double s = 0.0;
#pragma unroll
  for (int q = 0; q < NT / WAVE; ++q) s += scratch[q];
  __syncthreads();
  return s;
}

// Merge (t0, t1) into the pair (s0 >= s1) of fp32 proxy scores; ids break ties.
__device__ __forceinline__ void top2_merge(float& s0, float& l0, int& i0, float& s1, float& l1,
                                           int& i1, float t0, float tl0, int ti0, float t1,
                                           float tl1, int ti1) {
  auto better = [](float a, int ia, float b, int ib) {
    return ia >= 0 && (ib < 0 || a > b || (a == b && ia < ib));
  };
  float cs[4] = {s0, s1, t0, t1}, cl[4] = {l0, l1, tl0, tl1};
  int ci[4] = {i0, i1, ti0, ti1};
  int bi = 0;
#pragma unroll
  for (int q = 1; q < 4; ++q)
    if (better(cs[q], ci[q], cs[bi], ci[bi])) bi = q;
  int si = bi == 0 ? 1 : 0;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (q != bi && better(cs[q], ci[q], cs[si], ci[si])) si = q;
  float ns0 = -INFINITY, nl0 = 0.f, ns1 = -INFINITY, nl1 = 0.f;
  int ni0 = -1, ni1 = -1;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (q == bi) { ns0 = cs[q]; nl0 = cl[q]; ni0 = ci[q]; }
    if (q == si) { ns1 = cs[q]; nl1 = cl[q]; ni1 = ci[q]; }
  }
  s0 = ns0; l0 = nl0; i0 = ni0;
  s1 = ns1; l1 = nl1; i1 = ni1;
}

// Wave-then-block reduction of the two best (score, l, id); result in thread 0.
// The wave's two best of every lane's (s0, l0, i0) >= (s1, l1, i1) pair under (valid
// first, score desc, id asc), with DPP reductions, in every lane: the best is the largest
// score, the smallest id among equal scores; the runner-up is the best of every lane's
// remaining candidate (the winner lane's second, the others' first). Ids are unique, so
// the winner lane is.
// With `s2` (each lane's third score on entry) the wave's third-best score is returned in
// it: the best of what every lane has left once the two winners are taken.
__device__ __forceinline__ void wave_top2(float& s0, float& l0, int& i0, float& s1, float& l1,
                                          int& i1, float* s2 = nullptr) {
  const int lane = threadIdx.x & (WAVE - 1);
  auto best = [&](float sc, float lv, int id, float& bs, float& bl, int& bi) -> int {
    const bool ok = id >= 0;
    const float m = wave_max_f(ok ? sc : -INFINITY);
    const int mid = wave_min_i(ok && sc == m ? id : INT_MAX);
    if (mid == INT_MAX) {
      bs = -INFINITY; bl = 0.f; bi = -1;
      return -1;
    }
    const uint64_t bal = __ballot(ok && sc == m && id == mid);
    const int wl = (int)__ffsll((long long)bal) - 1;
    bs = m;
    bi = mid;
    bl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lv), wl));
    return wl;
  };
  float bs0, bl0, bs1, bl1;
  int bi0, bi1;
  const int wl = best(s0, l0, i0, bs0, bl0, bi0);
  const bool mine = lane == wl;
  const int wl1 = best(mine ? s1 : s0, mine ? l1 : l0, mine ? i1 : i0, bs1, bl1, bi1);
  if (s2) {
    // left on each lane: the winner of both its third, a winner of one its second
    const float rem = mine ? (lane == wl1 ? *s2 : (i1 >= 0 ? s1 : -INFINITY))
                           : (lane == wl1 ? (i1 >= 0 ? s1 : -INFINITY) : (i0 >= 0 ? s0 : -INFINITY));
    *s2 = wave_max_f(rem);
  }
  s0 = bs0; l0 = bl0; i0 = bi0;
  s1 = bs1; l1 = bl1; i1 = bi1;
}

// Block argmax over (score desc, tie key asc); the winner's id lands in *out_id (-1 when
// no thread holds a candidate).
template <int NT>
__device__ __forceinline__ void block_argmax_score(double sc, uint64_t tk, int id, double* s_sc,
                                                   uint64_t* s_tk, int* s_id, int* out_id) {
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  auto take = [](double& a, uint64_t& ak, int& ai, double b, uint64_t bk, int bi) {
    if (bi >= 0 && (ai < 0 || b > a || (b == a && bk < ak))) { a = b; ak = bk; ai = bi; }
  };
#define STRIM_ARG_STEP(C) take(sc, tk, id, dpp_d<C>(sc), dpp_u64<C>(tk), dpp_i<C>(id))
  STRIM_ARG_STEP(DPP_XOR1);
  STRIM_ARG_STEP(DPP_XOR2);
  STRIM_ARG_STEP(DPP_HALF_MIRROR);
  STRIM_ARG_STEP(DPP_MIRROR);
#undef STRIM_ARG_STEP
  {
    double bs = rl_d(sc, 0);
    uint64_t bk = rl_u64(tk, 0);
    int bi = rl_i(id, 0);
    take(bs, bk, bi, rl_d(sc, 16), rl_u64(tk, 16), rl_i(id, 16));
    take(bs, bk, bi, rl_d(sc, 32), rl_u64(tk, 32), rl_i(id, 32));
    take(bs, bk, bi, rl_d(sc, 48), rl_u64(tk, 48), rl_i(id, 48));
    sc = bs; tk = bk; id = bi;
  }
  __syncthreads();
  if (lane == 0) { s_sc[w] = sc; s_tk[w] = tk; s_id[w] = id; }
  __syncthreads();
  if (t == 0) {
    double bs = s_sc[0];
    uint64_t btk = s_tk[0];
    int bid = s_id[0];
    for (int q = 1; q < NT / WAVE; ++q) {
      if (s_id[q] < 0) continue;
      if (bid < 0 || s_sc[q] > bs || (s_sc[q] == bs && s_tk[q] < btk)) {
        bs = s_sc[q]; btk = s_tk[q]; bid = s_id[q];
      }
    }
    *out_id = bid;
  }
  __syncthreads();
}

// Ascending sort of the n unique keys s_key[0, n), n <= NT: each thread ranks one key
// by counting the smaller ones (broadcast LDS reads), then scatters it.
template <int NT>
__device__ __forceinline__ void rank_sort(uint64_t* s_key, int n) {
  const int t = threadIdx.x;
  const uint64_t k0 = t < n ? s_key[t] : ~0ull;
  uint32_t rank = 0;
  int jj = 0;
  for (; jj + 4 <= n; jj += 4)
    rank += (uint32_t)(s_key[jj] < k0) + (uint32_t)(s_key[jj + 1] < k0) +
            (uint32_t)(s_key[jj + 2] < k0) + (uint32_t)(s_key[jj + 3] < k0);
  for (; jj < n; ++jj) rank += (uint32_t)(s_key[jj] < k0);
  __syncthreads();
  if (t < n) s_key[rank] = k0;
  __syncthreads();
}

// Ascending bitonic sort of s_key[0, n) in LDS, padded with ~0 up to the next power of
// two n2 (s_key must hold n2 entries). One compare-exchange pair per thread per step.
template <int NT>
__device__ __forceinline__ void bitonic_sort_lds(uint64_t* s_key, int n) {
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  for (int i = n + (int)threadIdx.x; i < n2; i += NT) s_key[i] = ~0ull;
  __syncthreads();
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int pidx = threadIdx.x; pidx < n2 / 2; pidx += NT) {
        const int lo = 2 * pidx - (pidx & (stride - 1));
        const int hi = lo + stride;
        const uint64_t a = s_key[lo], b = s_key[hi];
        const bool asc = (lo & size) == 0;
        if ((a > b) == asc) {
          s_key[lo] = b;
          s_key[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

// The k-th smallest (k >= 1) of the keys a thread holds in kk[0, Q) (~0 = empty), by an
// MSD radix select over 8-bit digits starting at the highest bit where the keys differ.
// `ref` is any present key (the same in every thread). s_hist holds 256 counters,
// s_u64 >= NT/64 + 4 entries, s_int >= 4. Keys are unique; the caller guarantees at
// least k present keys.
template <int NT, int Q>
__device__ uint64_t radix_select_kth(const uint64_t (&kk)[Q], uint64_t ref, uint32_t k,
                                     uint32_t* s_hist, uint64_t* s_u64, int* s_int) {
  const int t = threadIdx.x, lane = t & (WAVE - 1);
  uint64_t diff = 0ull;
#pragma unroll
  for (int q = 0; q < Q; ++q)
    if (kk[q] != ~0ull) diff |= kk[q] ^ ref;
  diff = block_or_u64<NT>(diff, s_u64);
  if (diff == 0ull) return ref;  // a single key
  const int hb = 63 - __clzll((long long)diff);
  uint64_t pmask = hb == 63 ? 0ull : ~((2ull << hb) - 1ull);
  uint64_t prefix = ref & pmask;
  int shift = hb >= 7 ? hb - 7 : 0;
  uint32_t need = k;
  for (;;) {
    for (int i = t; i < 256; i += NT) s_hist[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < Q; ++q)
      if (kk[q] != ~0ull && (kk[q] & pmask) == prefix)
        atomicAdd(&s_hist[(uint32_t)(kk[q] >> shift) & 255u], 1u);
    __syncthreads();
    if (t < WAVE) {
      // lane owns digits 4*lane .. 4*lane+3
      const uint32_t h0 = s_hist[4 * lane], h1 = s_hist[4 * lane + 1], h2 = s_hist[4 * lane + 2],
                     h3 = s_hist[4 * lane + 3];
      const uint32_t own = h0 + h1 + h2 + h3;
      uint32_t cum = wave_incl_scan_u32(own) - own;
      const uint32_t hs[4] = {h0, h1, h2, h3};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (cum < need && need <= cum + hs[e]) {
          s_int[0] = 4 * lane + e;
          s_int[1] = (int)cum;
          s_int[2] = (int)hs[e];
        }
        cum += hs[e];
      }
    }
    __syncthreads();
    const int dsel = s_int[0];
    const uint32_t below = (uint32_t)s_int[1], cnt = (uint32_t)s_int[2];
    __syncthreads();
    need -= below;
    prefix = (prefix & ~(255ull << shift)) | ((uint64_t)dsel << shift);
    pmask |= 255ull << shift;
    if (cnt == need) {
      // every key of the bucket is selected: the k-th is the bucket's largest
      uint64_t mx = 0ull;
#pragma unroll
      for (int q = 0; q < Q; ++q)
        if (kk[q] != ~0ull && (kk[q] & pmask) == prefix && kk[q] > mx) mx = kk[q];
      return block_max_u64<NT>(mx, s_u64);
    }
    if (shift == 0) return prefix;
    shift = shift >= 8 ? shift - 8 : 0;
  }
}

}  // namespace strim

// ---------------------------------------------------------------------------------
// single-wave helpers (a 64-thread workgroup: no barriers between its steps)
// ---------------------------------------------------------------------------------
namespace strim {

// Orders the LDS accesses of one wave around this point (other waves of the workgroup
// may have exited, so no workgroup barrier is used). A wave's LDS instructions execute
// in issue order; the fences keep the compiler from moving accesses across.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint64_t shfl_xor_u64v(uint64_t v, int o) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o, WAVE);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, WAVE);
  return ((uint64_t)hi << 32) | lo;
}

// Exclusive prefix over the wave (integer: exact); *total = wave sum.
__device__ __forceinline__ uint32_t wave_excl_scan_u32(uint32_t v, uint32_t* total) {
  const uint32_t inc = wave_incl_scan_u32(v);
  *total = (uint32_t)rl_i((int)inc, WAVE - 1);
  return inc - v;
}

// Exclusive prefix of doubles over the wave in a fixed association order
// (deterministic); *total = wave sum.
__device__ __forceinline__ double wave_excl_scan_f64(double v, double* total) {
  const int lane = threadIdx.x & (WAVE - 1);
  const double inc = wave_incl_scan(v);
  *total = rl_d(inc, WAVE - 1);
  // the previous lane's inclusive value: row_shr within a row, readlane across rows
  double prev = dpp_d<DPP_SHR1>(inc);
  const double e15 = rl_d(inc, 15), e31 = rl_d(inc, 31), e47 = rl_d(inc, 47);
  if (lane == 16) prev = e15;
  if (lane == 32) prev = e31;
  if (lane == 48) prev = e47;
  return lane == 0 ? 0.0 : prev;
}

__device__ __forceinline__ uint64_t wave_or_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)wave_or_i((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)wave_or_i((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Wave argmax over (score desc, tie key asc); returns the winner's id (-1 if none),
// the same in every lane.
__device__ __forceinline__ int wave_argmax_score(double sc, uint64_t tk, int id) {
  auto take = [](double& a, uint64_t& ak, int& ai, double b, uint64_t bk, int bi) {
    if (bi >= 0 && (ai < 0 || b > a || (b == a && bk < ak))) { a = b; ak = bk; ai = bi; }
  };
#define STRIM_ARG_STEP(C) take(sc, tk, id, dpp_d<C>(sc), dpp_u64<C>(tk), dpp_i<C>(id))
  STRIM_ARG_STEP(DPP_XOR1);
  STRIM_ARG_STEP(DPP_XOR2);
  STRIM_ARG_STEP(DPP_HALF_MIRROR);
  STRIM_ARG_STEP(DPP_MIRROR);
#undef STRIM_ARG_STEP
  double bs = rl_d(sc, 0);
  uint64_t bk = rl_u64(tk, 0);
  int bi = rl_i(id, 0);
  take(bs, bk, bi, rl_d(sc, 16), rl_u64(tk, 16), rl_i(id, 16));
  take(bs, bk, bi, rl_d(sc, 32), rl_u64(tk, 32), rl_i(id, 32));
  take(bs, bk, bi, rl_d(sc, 48), rl_u64(tk, 48), rl_i(id, 48));
  return bi;
}

// Ascending sort of key[0, n), n <= 64 distinct keys in LDS, by one wave: each lane
// counts the keys below its own (broadcast LDS reads, eight in flight) and stores its key
// at that rank. Cheaper than a bitonic network of cross-lane exchanges for small n.
__device__ __forceinline__ void wave_rank_sort(uint64_t* key, int n) {
  const int lane = threadIdx.x & (WAVE - 1);
  const uint64_t k = lane < n ? key[lane] : ~0ull;
  int rank = 0;
  int q = 0;
  for (; q + 8 <= n; q += 8) {
    uint64_t c[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) c[e] = key[q + e];
#pragma unroll
    for (int e = 0; e < 8; ++e) rank += c[e] < k ? 1 : 0;
  }
  for (; q < n; ++q) rank += key[q] < k ? 1 : 0;
  wave_sync();
  if (lane < n) key[rank] = k;
  wave_sync();
}

// Ascending bitonic sort of one key per lane (~0 = empty sorts last).
__device__ __forceinline__ uint64_t wave_sort_u64(uint64_t k) {
  const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
  for (int size = 2; size <= WAVE; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t o = shfl_xor_u64v(k, stride);
      const bool asc = (lane & size) == 0;
      const bool lower = (lane & stride) == 0;
      const uint64_t lo = k < o ? k : o, hi = k < o ? o : k;
      k = (lower == asc) ? lo : hi;
    }
  return k;
}

// Ascending bitonic sort of key[0, n) in LDS by one wave (key holds the next power of
// two entries; padding with ~0).
__device__ __forceinline__ void wave_sort_lds(uint64_t* key, int n) {
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  const int lane = threadIdx.x & (WAVE - 1);
  for (int i = n + lane; i < n2; i += WAVE) key[i] = ~0ull;
  wave_sync();
  for (int size = 2; size <= n2; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int pidx = lane; pidx < n2 / 2; pidx += WAVE) {
        const int lo = 2 * pidx - (pidx & (stride - 1));
        const int hi = lo + stride;
        const uint64_t x = key[lo], y = key[hi];
        const bool asc = (lo & size) == 0;
        if ((x > y) == asc) {
          key[lo] = y;
          key[hi] = x;
        }
      }
      wave_sync();
    }
}

// The k-th smallest (k >= 1) of the n unique keys key[0, n) in LDS, by an MSD radix
// select over 8-bit digits from the highest bit where the keys differ. One wave; hist
// holds 256 counters. The caller guarantees n >= k.
__device__ uint64_t wave_radix_kth(const uint64_t* key, int n, uint32_t k, uint32_t* hist) {
  const int lane = threadIdx.x & (WAVE - 1);
  const uint64_t ref = key[0];
  uint64_t diff = 0ull;
  for (int i = lane; i < n; i += WAVE) diff |= key[i] ^ ref;
  diff = wave_or_u64(diff);
  if (diff == 0ull) return ref;
  const int hb = 63 - __clzll((long long)diff);
  uint64_t pmask = hb == 63 ? 0ull : ~((2ull << hb) - 1ull);
  uint64_t prefix = ref & pmask;
  int shift = hb >= 7 ? hb - 7 : 0;
  uint32_t need = k;
  for (;;) {
    *(uint4*)&hist[4 * lane] = make_uint4(0u, 0u, 0u, 0u);
    wave_sync();
    for (int i = lane; i < n; i += WAVE) {
      const uint64_t kv = key[i];
      if ((kv & pmask) == prefix) atomicAdd(&hist[(uint32_t)(kv >> shift) & 255u], 1u);
    }
    wave_sync();
    const uint4 h = *(const uint4*)&hist[4 * lane];
    const uint32_t own = h.x + h.y + h.z + h.w;
    uint32_t tot;
    uint32_t cum = wave_excl_scan_u32(own, &tot);
    const uint32_t hs[4] = {h.x, h.y, h.z, h.w};
    int dl = -1;
    uint32_t bl = 0u, cl = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (dl < 0 && cum < need && need <= cum + hs[e]) {
        dl = 4 * lane + e;
        bl = cum;
        cl = hs[e];
      }
      cum += hs[e];
    }
    const uint64_t who = __ballot(dl >= 0);
    const int src = (int)__ffsll((long long)who) - 1;
    const int dsel = rl_i(dl, src);
    const uint32_t below = (uint32_t)rl_i((int)bl, src);
    const uint32_t cnt = (uint32_t)rl_i((int)cl, src);
    wave_sync();
    need -= below;
    prefix = (prefix & ~(255ull << shift)) | ((uint64_t)dsel << shift);
    pmask |= 255ull << shift;
    if (cnt == need) {
      // every key of the bucket is selected: the k-th is the bucket's largest
      uint64_t mx = 0ull;
      for (int i = lane; i < n; i += WAVE) {
        const uint64_t kv = key[i];
        if ((kv & pmask) == prefix && kv > mx) mx = kv;
      }
      return wave_max_u64(mx);
    }
    if (shift == 0) return prefix;
    shift = shift >= 8 ? shift - 8 : 0;
  }
}

// ---------------------------------------------------------------------------------
// Sorting the candidates of a 1024-thread finalize workgroup (k_final, k_qfinal)
// ---------------------------------------------------------------------------------
// Ascending sort of the n2 (power of two, 64 <= n2 <= CAP) unique keys k[q] (element
// q * FIN_T + t) into s_key, with s_tmp (n2 entries) as the second buffer. Runs of 64
// are sorted by rank within the run, then merged pairwise: a key's place in the merged
// run is its place in its own run plus its lower bound in the partner run (keys are
// unique, so every round is a permutation).
__device__ inline void merge_sort(const uint64_t (&k)[FIN_Q], int n2, uint64_t* s_key,
                           uint64_t* s_tmp) {
  const int t = threadIdx.x, lane = t & (WAVE - 1);
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q)
    if (q * FIN_T < n2) s_key[q * FIN_T + t] = k[q];
  __syncthreads();
  uint64_t* A = s_key;
  uint64_t* B = s_tmp;
  // runs of 64: the wave's 64 consecutive positions of each stripe q
#pragma unroll
  for (int q = 0; q < FIN_Q; ++q) {
    if (q * FIN_T >= n2) continue;
    const int base = q * FIN_T + (t - lane);
    const uint64_t k0 = A[base + lane];
    uint32_t rk = 0;
#pragma unroll 8
    for (int i = 0; i < WAVE; i += 2) {
      const ulonglong2 xy = *(const ulonglong2*)&A[base + i];
      rk += (uint32_t)(xy.x < k0) + (uint32_t)(xy.y < k0);
    }
    B[base + rk] = k0;
  }
  __syncthreads();
  {
    uint64_t* T = A; A = B; B = T;
  }
  for (int R = WAVE; R < n2; R <<= 1) {
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q) {
      const int idx = q * FIN_T + t;
      if (idx >= n2) continue;
      const uint64_t k0 = A[idx];
      const int ri = idx / R, pi = idx & (R - 1);
      const uint64_t* P = A + (ri ^ 1) * R;
      int pos = 0;
      for (int st = R >> 1; st >= 1; st >>= 1)
        if (P[pos + st - 1] < k0) pos += st;
      pos += P[pos] < k0 ? 1 : 0;
      B[(ri & ~1) * R + pi + pos] = k0;
    }
    __syncthreads();
    uint64_t* T = A; A = B; B = T;
  }
  if (A != s_key) {
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q)
      if (q * FIN_T < n2) s_key[q * FIN_T + t] = A[q * FIN_T + t];
    __syncthreads();
  }
}

// Ascending sort of the n <= CAP unique keys kk[q] (element q * FIN_T + t) into s_key
// (2 * FIN_T entries at least); s_tmp (CAP entries) is the merge sort's second buffer.
__device__ inline void sort_keys(uint64_t (&kk)[FIN_Q], int n, uint64_t* s_key, uint64_t* s_tmp) {
  const int t = threadIdx.x;
  int n2 = 64;
  while (n2 < n) n2 <<= 1;
  if (n <= FIN_T) {
    // one key per thread: every wave ranks its 64 keys among themselves and writes them
    // as a sorted run; a key's rank is its rank in its run plus its lower bound in each
    // other run (keys are unique, so the ranks are a permutation of 0..n-1). Pads sort
    // after every key (a finite l has key bits below 0xFF800000 << 32).
    const int w = wave_id(), lane = t & (WAVE - 1);
    const uint64_t k0 = t < n ? kk[0] : (0xFFFFFFFF00000000ull | (uint32_t)t);
    uint64_t* run = s_key + FIN_T;  // FIN_T sorted keys, 64 per run
    s_key[t] = k0;
    wave_sync();
    uint32_t rw = 0;
#pragma unroll 8
    for (int q = 0; q < WAVE; q += 2) {
      const ulonglong2 xy = *(const ulonglong2*)&s_key[w * WAVE + q];
      rw += (uint32_t)(xy.x < k0) + (uint32_t)(xy.y < k0);
    }
    run[w * WAVE + rw] = k0;
    __syncthreads();
    uint32_t rank = rw;
    const int nrun = (n + WAVE - 1) / WAVE;
#pragma unroll
    for (int q = 0; q < FIN_T / WAVE; ++q) {
      if (q >= nrun || q == w) continue;
      const uint64_t* rq = run + q * WAVE;
      uint32_t pos = 0;
#pragma unroll
      for (int st = WAVE / 2; st >= 1; st >>= 1)
        if (rq[pos + st - 1] < k0) pos += st;
      pos += rq[pos] < k0 ? 1u : 0u;
      rank += pos;
    }
    if (t < n) s_key[rank] = k0;
    __syncthreads();
  } else {
    // pads (after every key, see above) fill the power of two
#pragma unroll
    for (int q = 0; q < FIN_Q; ++q) {
      const int idx = q * FIN_T + t;
      if (idx >= n) kk[q] = 0xFFFFFFFF00000000ull | (uint32_t)idx;
    }
    merge_sort(kk, n2, s_key, s_tmp);
  }
}

}  // namespace strim
