// common.hpp — device-side building blocks of the gfx950 token-selection kernels.
//
// Layout of one call: R rows of V logits. Every streaming kernel splits a row into
// chunks of CHUNK tokens; a 512-thread workgroup owns one (row, chunk) and each thread
// owns EPT consecutive tokens (one 16-byte load of bf16, two of fp32). Rows that are a
// multiple of 8 are mapped XCD-locally: all chunks of a row land on the same XCD
// (workgroups are dispatched round-robin over the 8 XCDs), so the row's re-reads and
// its atomics stay in one L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/strim_sampler.h"

namespace strim {

constexpr int CHUNK = 4096;    // tokens per workgroup
constexpr int TPB = 512;       // threads per streaming workgroup (8 waves of 64)
constexpr int EPT = 8;         // tokens per thread
constexpr int NBINS = 2048;    // bins over d = m - l: width 1/32 on [0, 64), last = tail
constexpr float BIN_SCALE = 32.0f;
constexpr int CAP = 4096;      // candidates per row held by the finalize workgroup
constexpr int FIN_T = 1024;    // finalize workgroup size
constexpr int FIN_Q = CAP / FIN_T;
constexpr double FIX_SCALE = 1099511627776.0;  // 2^40 fixed-point mass scale
constexpr float FIX_SCALE_F = 1099511627776.0f;
constexpr int WAVE = 64;

static_assert(CHUNK == TPB * EPT, "chunk geometry");

// ---- row status / mode ---------------------------------------------------------
enum RowMode : int32_t { MODE_NONE = 0, MODE_A = 1, MODE_B = 2 };

// Per (row, chunk) statistics written by k_stats.
struct ChunkStat {
  float m;        // max processed logit of the chunk (-inf if none allowed)
  int32_t arg;    // first id reaching m (greedy rows: over the untempered logits)
  int32_t n;      // allowed tokens
  int32_t flags;  // bit0: non-finite logit seen
};

// Per-chunk best two surely-kept tokens by the fp32 Gumbel proxy l + g.
struct ChunkTop {
  float l0;
  int32_t id0;
  float l1;
  int32_t id1;
};

struct Cand {
  float l;
  int32_t id;
};

// Per-row state shared by the kernels of one call.
struct RowState {
  float m;            // max processed logit
  int32_t status;     // STRIM_OK or STRIM_E*
  int32_t n_allowed;
  int32_t argmax;     // greedy result
  int32_t greedy;
  int32_t mode;       // RowMode
  int32_t s;          // bins < s (and not collected) are surely kept
  int32_t e;          // bins > e (and not collected) are surely dropped
  int32_t s1;         // bins < s1 surely pass min-p and top-k
  int32_t rng[3][2];  // collected bin ranges [lo, hi] (lo > hi = empty)
  int32_t draft;      // verify: draft token of this row or -1
  float l_draft;      // verify: processed logit of the draft (-inf if not allowed)
  int32_t pad0;
  double q_draft;     // verify: q(draft)
  double sum_kept;    // finalize: kept mass (relative to exp(m))
  uint64_t last_key;  // finalize: ckey of the last kept collected token in [s, e] (0 = none)
  int32_t token;      // finalize: row outcome token
  int32_t accept;     // verify: accept flag
};

// ---- scalar helpers --------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// 32-bit key whose ascending order is the float's descending order (-0 == +0).
__device__ __forceinline__ uint32_t fkey_desc(float f) {
  if (f == 0.0f) f = 0.0f;
  uint32_t u = __float_as_uint(f);
  uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ~asc;
}
__device__ __forceinline__ float fkey_desc_inv(uint32_t k) {
  uint32_t asc = ~k;
  uint32_t u = (asc & 0x80000000u) ? (asc & 0x7FFFFFFFu) : ~asc;
  return __uint_as_float(u);
}
// Ascending order = (l descending, id ascending): the token order of every decision.
__device__ __forceinline__ uint64_t ckey(float l, int32_t id) {
  return ((uint64_t)fkey_desc(l) << 32) | (uint32_t)id;
}

// Bin of d = m - l (d >= 0). Monotone in l, equal l share a bin.
__device__ __forceinline__ int dbin(float d) {
  return d < 64.0f ? (int)(d * BIN_SCALE) : (NBINS - 1);
}

// ---- random numbers ----------------------------------------------------------------
// SpecSampling.mix (Sources/StrimCore/SpecSampling.swift:29-34): SplitMix64 finaliser.
__device__ __host__ __forceinline__ uint64_t mix64(uint64_t seed, uint64_t position) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (position + 1u);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Philox4x32-10 (Salmon et al., SC'11).
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint32_t hi0 = __umulhi(0xD2511F53u, c.x), lo0 = 0xD2511F53u * c.x;
    uint32_t hi1 = __umulhi(0xCD9E8D57u, c.z), lo1 = 0xCD9E8D57u * c.z;
    c = make_uint4(hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0);
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}
__device__ __forceinline__ float u01(uint32_t w) {
  return (float)(w >> 8) * 5.9604644775390625e-08f;
}
// Element `idx` of the [V+1] uniform vector of position key `key`.
__device__ __forceinline__ float philox_uniform(uint64_t key, uint64_t idx) {
  uint64_t blk = idx >> 2;
  uint4 w = philox4x32_10(make_uint4((uint32_t)blk, (uint32_t)(blk >> 32), 0u, 0u),
                          (uint32_t)key, (uint32_t)(key >> 32));
  uint32_t j = (uint32_t)(idx & 3u);
  return u01(j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w);
}

// Gumbel transform of SpecSampling.rowOutcome (SpecSampling.swift:79), fp64.
__device__ __forceinline__ double gumbel64(float u) {
  float uu = u > 1e-30f ? u : 1e-30f;
  return -log(-log((double)uu));
}
// fp32 proxy of the same transform, used only to shortlist chunk winners.
__device__ __forceinline__ float gumbel32(float u) {
  float uu = u > 1e-30f ? u : 1e-30f;
  return -logf(-logf(uu));
}

// ---- wave / block reductions (wave64) ---------------------------------------------
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)v, o, WAVE);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, WAVE);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, WAVE));
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, WAVE));
  return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)v, o, WAVE);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, WAVE);
    uint64_t w = ((uint64_t)hi << 32) | lo;
    v = w > v ? w : v;
  }
  return v;
}
// Inclusive scan over the wave (Hillis-Steele, fixed order => deterministic).
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    T w = __shfl_up(v, o, WAVE);
    if (lane >= o) v += w;
  }
  return v;
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    uint32_t lo = __shfl_up((uint32_t)v, o, WAVE);
    uint32_t hi = __shfl_up((uint32_t)(v >> 32), o, WAVE);
    if (lane >= o) v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// (value, id) argmax: larger value wins, equal values -> smaller id.
__device__ __forceinline__ void argmax_merge(float& v, int& id, float v2, int id2) {
  if (id2 >= 0 && (id < 0 || v2 > v || (v2 == v && id2 < id))) {
    v = v2;
    id = id2;
  }
}

// Block-wide exclusive scan of one double per thread, fixed order (deterministic).
// `scratch` holds >= NT/64 doubles. Returns the exclusive prefix; *total gets the sum.
template <int NT>
__device__ __forceinline__ double block_excl_scan_f64(double v, double* scratch, double* total) {
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  double inc = wave_incl_scan(v);
  if (lane == WAVE - 1) scratch[w] = inc;
  __syncthreads();
  double base = 0.0, tot = 0.0;
#pragma unroll
  for (int i = 0; i < NT / WAVE; ++i) {
    double s = scratch[i];
    if (i < w) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + inc - v;
}
template <int NT>
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, uint64_t* scratch,
                                                        uint64_t* total) {
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  uint64_t inc = wave_incl_scan_u64(v);
  if (lane == WAVE - 1) scratch[w] = inc;
  __syncthreads();
  uint64_t base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / WAVE; ++i) {
    uint64_t s = scratch[i];
    if (i < w) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + inc - v;
}

}  // namespace strim
