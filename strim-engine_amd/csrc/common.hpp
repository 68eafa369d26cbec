// common.hpp — device-side building blocks of the gfx950 token-selection kernels.
//
// Layout of one call: R rows of V logits. Every streaming kernel splits a row into
// chunks of CHUNK tokens and launches a (chunks, rows) grid; one workgroup owns one
// (row, chunk) and each thread owns runs of EPT consecutive tokens (one 16-byte load of
// bf16, two of fp32): k_stream with 512 or 128 threads (one or four runs each), k_probs
// and the residual-draw passes with TPB threads (one run each).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/strim_sampler.h"

namespace strim {

// An LDS object named with its address space, for data handed to functions that are
// not inlined: across such a call a plain pointer is generic, and the compiler then
// reaches LDS with flat instructions (slower atomics, and every wait for them also waits
// for the outstanding global loads). Cast to a plain pointer at the use; the compiler
// still sees where it points.
template <typename T>
using lds_t = __attribute__((address_space(3))) T;
// The same for global memory: a pointer re-typed with it at the top of a function that
// is not inlined gives its loads the global instructions again.
template <typename T>
using glb_t = __attribute__((address_space(1))) T;

// A copy of a workgroup-uniform value held in scalar registers. Functions that are not
// inlined receive every argument in vector registers; re-reading the uniform ones with
// readfirstlane at the entry frees those registers (the exact resolution runs in
// 1024-thread workgroups, whose threads get at most 128 of them).
template <typename T>
__device__ __forceinline__ T uniform_copy(const T& v) {
  static_assert(sizeof(T) % 4 == 0, "whole 32-bit words");
  struct W { uint32_t w[sizeof(T) / 4]; };
  W in = __builtin_bit_cast(W, v), out;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i)
    out.w[i] = (uint32_t)__builtin_amdgcn_readfirstlane((int)in.w[i]);
  return __builtin_bit_cast(T, out);
}

constexpr int CHUNK = 4096;    // tokens per workgroup
constexpr int TPB = 512;       // threads per streaming workgroup (8 waves of 64)
constexpr int EPT = 8;         // tokens per thread
constexpr int CAP = 8192;      // candidates per row held by the finalize workgroup
constexpr int FIN_T = 1024;    // finalize workgroup size
constexpr int FIN_Q = CAP / FIN_T;
constexpr int WAVE = 64;

static_assert(CHUNK == TPB * EPT, "chunk geometry");

// ---- scalar helpers --------------------------------------------------------------
// The thread's wave in its workgroup, as a scalar: the compiler cannot tell that
// threadIdx.x / WAVE is uniform over a wave, and would otherwise keep it (and every loop
// bound or branch derived from it) in vector registers under exec masks.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)threadIdx.x / WAVE);
}
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
// Block `blk` of the uniform stream of position key `key`: elements 4 blk .. 4 blk + 3.
__device__ __forceinline__ uint4 philox_block(uint64_t key, uint64_t blk) {
  return philox4x32_10(make_uint4((uint32_t)blk, (uint32_t)(blk >> 32), 0u, 0u),
                       (uint32_t)key, (uint32_t)(key >> 32));
}
// Element `idx` of the [V+1] uniform vector of position key `key`.
__device__ __forceinline__ float philox_uniform(uint64_t key, uint64_t idx) {
  const uint4 w = philox_block(key, idx >> 2);
  uint32_t j = (uint32_t)(idx & 3u);
  return u01(j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w);
}

// Gumbel transform of SpecSampling.rowOutcome (SpecSampling.swift:79), fp64.
__device__ __forceinline__ double gumbel64(float u) {
  float uu = u > 1e-30f ? u : 1e-30f;
  return -log(-log((double)uu));
}
// fp32 proxy of the same transform, used only to shortlist chunk winners: two hardware
// base-2 logarithms, -ln(-ln u) = -ln2 (log2(-log2 u) + log2(ln2)). Over every value u01
// produces (k 2^-24) and the 1e-30 floor its absolute error against the fp64 transform is
// at most 1.98e-6 (at most 1.6e-7 (1 + |g|)), that of a logf-based version 1.68e-6.
__device__ __forceinline__ float gumbel32(float u) {
  const float uu = u > 1e-30f ? u : 1e-30f;
  const float a = -__builtin_amdgcn_logf(uu);  // -log2(u) > 0
  return -0.69314718f * (__builtin_amdgcn_logf(a) - 0.52876637f);
}

// ---- wave64 primitives on DPP ---------------------------------------------------------
// Cross-lane steps use DPP (quad_perm / row_half_mirror / row_mirror / row_shr) and
// v_readlane, never ds_bpermute: a DPP move costs a VALU slot, not an LDS round trip.
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <-> 7 - i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <-> 15 - i within 16
constexpr int DPP_SHR1 = 0x111, DPP_SHR2 = 0x112, DPP_SHR4 = 0x114, DPP_SHR8 = 0x118;

template <int C>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, C, 0xF, 0xF, false);
}
template <int C>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<C>(__float_as_int(v)));
}
template <int C>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)dpp_i<C>((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)dpp_i<C>((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
template <int C>
__device__ __forceinline__ double dpp_d(double v) {
  return __longlong_as_double((long long)dpp_u64<C>((uint64_t)__double_as_longlong(v)));
}
__device__ __forceinline__ int rl_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ float rl_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ uint64_t rl_u64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ double rl_d(double v, int lane) {
  return __longlong_as_double((long long)rl_u64((uint64_t)__double_as_longlong(v), lane));
}

// Reduce within each 16-lane row (every lane ends with its row's value), then combine
// the four rows through readlane: the result is wave-uniform. `op` is associative and
// commutative; the fixed pattern keeps floating-point sums deterministic.
#define STRIM_WAVE_REDUCE(T, v, DPP, RL, OP)              \
  do {                                                    \
    v = OP(v, DPP<DPP_XOR1>(v));                          \
    v = OP(v, DPP<DPP_XOR2>(v));                          \
    v = OP(v, DPP<DPP_HALF_MIRROR>(v));                   \
    v = OP(v, DPP<DPP_MIRROR>(v));                        \
    const T r0 = RL(v, 0), r1 = RL(v, 16), r2 = RL(v, 32), r3 = RL(v, 48); \
    v = OP(OP(r0, r1), OP(r2, r3));                       \
  } while (0)

__device__ __forceinline__ int op_add_i(int a, int b) { return a + b; }
__device__ __forceinline__ int op_min_i(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ int op_max_i(int a, int b) { return a > b ? a : b; }
__device__ __forceinline__ int op_or_i(int a, int b) { return a | b; }
__device__ __forceinline__ double op_add_d(double a, double b) { return a + b; }
__device__ __forceinline__ float op_max_f(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ uint64_t op_add_u64(uint64_t a, uint64_t b) { return a + b; }
__device__ __forceinline__ uint64_t op_max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ int wave_sum(int v) { STRIM_WAVE_REDUCE(int, v, dpp_i, rl_i, op_add_i); return v; }
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) { return (uint32_t)wave_sum((int)v); }
__device__ __forceinline__ int wave_min_i(int v) { STRIM_WAVE_REDUCE(int, v, dpp_i, rl_i, op_min_i); return v; }
__device__ __forceinline__ int wave_max_i(int v) { STRIM_WAVE_REDUCE(int, v, dpp_i, rl_i, op_max_i); return v; }
__device__ __forceinline__ int wave_or_i(int v) { STRIM_WAVE_REDUCE(int, v, dpp_i, rl_i, op_or_i); return v; }
__device__ __forceinline__ float wave_max_f(float v) { STRIM_WAVE_REDUCE(float, v, dpp_f, rl_f, op_max_f); return v; }
__device__ __forceinline__ double wave_sum(double v) { STRIM_WAVE_REDUCE(double, v, dpp_d, rl_d, op_add_d); return v; }
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) { STRIM_WAVE_REDUCE(uint64_t, v, dpp_u64, rl_u64, op_add_u64); return v; }
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) { STRIM_WAVE_REDUCE(uint64_t, v, dpp_u64, rl_u64, op_max_u64); return v; }

// (value, id) argmax: larger value wins, equal values -> smaller id; id < 0 is empty.
__device__ __forceinline__ void argmax_merge(float& v, int& id, float v2, int id2) {
  if (id2 >= 0 && (id < 0 || v2 > v || (v2 == v && id2 < id))) {
    v = v2;
    id = id2;
  }
}
template <int C>
__device__ __forceinline__ void argmax_dpp_step(float& v, int& id) {
  const float v2 = dpp_f<C>(v);
  const int i2 = dpp_i<C>(id);
  argmax_merge(v, id, v2, i2);
}
// Wave-uniform argmax of (v, id).
__device__ __forceinline__ void wave_argmax(float& v, int& id) {
  argmax_dpp_step<DPP_XOR1>(v, id);
  argmax_dpp_step<DPP_XOR2>(v, id);
  argmax_dpp_step<DPP_HALF_MIRROR>(v, id);
  argmax_dpp_step<DPP_MIRROR>(v, id);
  float bv = rl_f(v, 0);
  int bi = rl_i(id, 0);
  argmax_merge(bv, bi, rl_f(v, 16), rl_i(id, 16));
  argmax_merge(bv, bi, rl_f(v, 32), rl_i(id, 32));
  argmax_merge(bv, bi, rl_f(v, 48), rl_i(id, 48));
  v = bv;
  id = bi;
}

// Lanes below this one whose bit is set in `mask`.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}
// Exclusive prefix and wave total of small per-lane counts (0..15) via ballots.
__device__ __forceinline__ int wave_excl_count(int c, int* total) {
  int ex = 0, tot = 0;
#pragma unroll
  for (int bit = 0; bit < 4; ++bit) {
    const uint64_t m = __ballot((c >> bit) & 1);
    ex += lanes_below(m) << bit;
    tot += __popcll(m) << bit;
  }
  *total = tot;
  return ex;
}

// Inclusive scan of doubles over the wave in a fixed order (deterministic): row_shr
// steps within 16-lane rows, then the row totals through readlane.
// Inclusive prefix sum over the wave (integer: exact): row_shr steps within each 16-lane
// row, then the earlier rows' totals through readlane.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  int x = (int)v;
  x += dpp_i<DPP_SHR1>(x);
  x += dpp_i<DPP_SHR2>(x);
  x += dpp_i<DPP_SHR4>(x);
  x += dpp_i<DPP_SHR8>(x);
  const int t0 = rl_i(x, 15), t1 = rl_i(x, 31), t2 = rl_i(x, 47);
  const int row = (threadIdx.x & (WAVE - 1)) >> 4;
  x += (row >= 1 ? t0 : 0) + (row >= 2 ? t1 : 0) + (row >= 3 ? t2 : 0);
  return (uint32_t)x;
}
__device__ __forceinline__ double wave_incl_scan(double v) {
  v += dpp_d<DPP_SHR1>(v);
  v += dpp_d<DPP_SHR2>(v);
  v += dpp_d<DPP_SHR4>(v);
  v += dpp_d<DPP_SHR8>(v);
  const double t0 = rl_d(v, 15), t1 = rl_d(v, 31), t2 = rl_d(v, 47);
  const int row = (threadIdx.x & (WAVE - 1)) >> 4;
  if (row >= 1) v += t0;
  if (row >= 2) v += t1;
  if (row >= 3) v += t2;
  return v;
}

// Block-wide exclusive scan of one double per thread, fixed order (deterministic).
// `scratch` holds >= NT/64 doubles. Returns the exclusive prefix; *total gets the sum.
template <int NT>
__device__ __forceinline__ double block_excl_scan_f64(double v, double* scratch, double* total) {
  const int lane = threadIdx.x & (WAVE - 1), w = wave_id();
  const double inc = wave_incl_scan(v);
  if (lane == WAVE - 1) scratch[w] = inc;
  __syncthreads();
  double base = 0.0, tot = 0.0;
#pragma unroll
  for (int i = 0; i < NT / WAVE; ++i) {
    const double s = scratch[i];
    if (i < w) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + inc - v;
}

// Inclusive scan of 64-bit integers over the wave (same pattern as the fp64 scan).
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  v += dpp_u64<DPP_SHR1>(v);
  v += dpp_u64<DPP_SHR2>(v);
  v += dpp_u64<DPP_SHR4>(v);
  v += dpp_u64<DPP_SHR8>(v);
  const uint64_t t0 = rl_u64(v, 15), t1 = rl_u64(v, 31), t2 = rl_u64(v, 47);
  const int row = (threadIdx.x & (WAVE - 1)) >> 4;
  if (row >= 1) v += t0;
  if (row >= 2) v += t1;
  if (row >= 3) v += t2;
  return v;
}

// Block-wide exclusive scans of two 64-bit integers per thread (exact). `scratch` holds
// >= 2 * NT / 64 values.
template <int NT>
__device__ __forceinline__ void block_excl_scan2_u64(uint64_t v1, uint64_t v2, uint64_t* scratch,
                                                     uint64_t& ex1, uint64_t& ex2,
                                                     uint64_t& tot1, uint64_t& tot2) {
  const int lane = threadIdx.x & (WAVE - 1), w = wave_id();
  const uint64_t i1 = wave_incl_scan_u64(v1), i2 = wave_incl_scan_u64(v2);
  if (lane == WAVE - 1) {
    scratch[w] = i1;
    scratch[NT / WAVE + w] = i2;
  }
  __syncthreads();
  uint64_t b1 = 0, b2 = 0, t1 = 0, t2 = 0;
#pragma unroll
  for (int i = 0; i < NT / WAVE; ++i) {
    const uint64_t s1 = scratch[i], s2 = scratch[NT / WAVE + i];
    if (i < w) {
      b1 += s1;
      b2 += s2;
    }
    t1 += s1;
    t2 += s2;
  }
  __syncthreads();
  ex1 = b1 + i1 - v1;
  ex2 = b2 + i2 - v2;
  tot1 = t1;
  tot2 = t2;
}

// Block-wide min of one int per thread; every thread gets the result.
template <int NT>
__device__ __forceinline__ int block_min(int v, int* scratch) {
  v = wave_min_i(v);
  if ((threadIdx.x & (WAVE - 1)) == 0) scratch[threadIdx.x / WAVE] = v;
  __syncthreads();
  int b = scratch[0];
#pragma unroll
  for (int q = 1; q < NT / WAVE; ++q) b = min(b, scratch[q]);
  __syncthreads();
  return b;
}

}  // namespace strim
