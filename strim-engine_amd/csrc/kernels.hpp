// kernels.hpp — argument block and per-row processing shared by the gfx950 kernels.
#pragma once

#include "common.hpp"

namespace strim {

// Device scratch owned by a context (allocated once in strim_ctx_create).
struct Scratch {
  ChunkStat* cstat;     // [rows][wmax]
  RowState* rs;         // [rows]
  uint32_t* cnt_stats;  // [rows] last-block counters, kept at zero between calls
  uint32_t* cnt_hist;   // [rows]
  uint32_t* hcnt;       // [rows][NBINS]
  unsigned long long* hmass;  // [rows][NBINS] fixed-point 2^40
  Cand* cand;           // [rows][CAP]
  uint32_t* ncand;      // [rows]
  ChunkTop* ctop;       // [rows][wmax]
  int32_t wmax;
};

// One launch argument block (passed by value to every kernel of a call).
struct Args {
  const void* logits;
  int64_t row_stride;
  int32_t dtype;
  int32_t vec_ok;  // 16-byte vector loads are aligned for every row
  int32_t R, V, W; // rows, vocab, chunks per row
  int32_t B, k;    // batch and draft length (k = 0 for strim_sample)
  int32_t verify;
  int32_t xcd_map;
  const strim_sampling_params* params;
  const uint32_t* mask;
  int64_t mask_stride;
  const int32_t* hist;
  const int32_t* hist_len;
  int32_t H;
  const int32_t* drafts;  // [B][k]
  int32_t noise_mode;
  const float* noise;
  int64_t noise_stride;
  Scratch s;
  int32_t* out_ids;
  int32_t* out_status;
  float* out_probs;
  // verify outputs
  int32_t* out_accepted;
  int32_t* out_token;
  int32_t* out_row_accept;
  int32_t* out_row_token;
};

// Row parameters in registers.
struct RowParams {
  float T, rep, pres, freq, min_p, top_p;
  int32_t top_k;
  uint32_t flags;
  uint64_t seed, position;
  bool greedy, pen, valid;
};

__device__ __forceinline__ void row_bj(const Args& a, int r, int& b, int& j) {
  if (a.verify) {
    b = r / (a.k + 1);
    j = r - b * (a.k + 1);
  } else {
    b = r;
    j = 0;
  }
}

// Workgroup -> (row, chunk). With rows a multiple of 8, row r's chunks all run on
// XCD r % 8 (hardware dispatches workgroup i to XCD i % 8).
__device__ __forceinline__ void map_block(const Args& a, int bid, int& r, int& c) {
  if (a.xcd_map) {
    int x = bid & 7, slot = bid >> 3;
    r = x + 8 * (slot / a.W);
    c = slot - (slot / a.W) * a.W;
  } else {
    r = bid / a.W;
    c = bid - r * a.W;
  }
}

__device__ __forceinline__ bool params_valid(const strim_sampling_params& p) {
  if (!isfinite(p.temperature)) return false;
  if (!(p.top_p > 0.0f && p.top_p <= 1.0f)) return false;
  if (p.top_k < 0) return false;
  if (!(p.min_p >= 0.0f && p.min_p <= 1.0f)) return false;
  if (!(p.repetition_penalty > 0.0f) || isinf(p.repetition_penalty)) return false;
  if (!isfinite(p.presence_penalty) || !isfinite(p.frequency_penalty)) return false;
  return true;
}

__device__ __forceinline__ RowParams load_params(const Args& a, int b, int j) {
  const strim_sampling_params& sp = a.params[b];
  RowParams p;
  p.T = sp.temperature;
  p.rep = sp.repetition_penalty;
  p.pres = sp.presence_penalty;
  p.freq = sp.frequency_penalty;
  p.min_p = sp.min_p;
  p.top_p = sp.top_p;
  p.top_k = sp.top_k;
  p.flags = sp.flags;
  if (a.verify) p.flags &= STRIM_FLAG_TOPK_KEEP_TIES;  // verify is the SpecSampling path
  p.seed = sp.seed;
  p.position = sp.position + (uint64_t)j;
  p.valid = params_valid(sp);
  p.greedy = !(p.T > 0.0f);
  const bool active = p.rep != 1.0f || p.pres != 0.0f || p.freq != 0.0f;
  p.pen = active && (a.hist != nullptr || (a.verify && j > 0));
  return p;
}

// History counts of the chunk [c0, c0 + CHUNK) in LDS (plus the verify draft prefix).
// Called by every thread of the workgroup when p.pen.
__device__ __forceinline__ void build_counts(const Args& a, int b, int j, int c0,
                                             uint32_t* s_cnt) {
  for (int i = threadIdx.x; i < CHUNK; i += TPB) s_cnt[i] = 0u;
  __syncthreads();
  if (a.hist) {
    int hl = a.hist_len ? a.hist_len[b] : a.H;
    hl = hl < 0 ? 0 : (hl > a.H ? a.H : hl);
    const int32_t* h = a.hist + (int64_t)b * a.H;
    for (int i = threadIdx.x; i < hl; i += TPB) {
      int id = h[i];
      unsigned o = (unsigned)(id - c0);
      if (o < (unsigned)CHUNK && id < a.V) atomicAdd(&s_cnt[o], 1u);
    }
  }
  if (a.verify && (int)threadIdx.x < j) {
    int id = a.drafts[(int64_t)b * a.k + threadIdx.x];
    unsigned o = (unsigned)(id - c0);
    if (o < (unsigned)CHUNK && id < a.V) atomicAdd(&s_cnt[o], 1u);
  }
  __syncthreads();
}

// Processed logits of this thread's EPT tokens: penalties -> mask -> temperature.
// Masked and out-of-range tokens get -inf. Greedy rows skip the temperature.
// Each step is one IEEE float32 operation (the file is built with -ffp-contract=off).
__device__ __forceinline__ void process_tokens(const Args& a, int r, int c0, const RowParams& p,
                                               const uint32_t* s_cnt, float (&l)[EPT],
                                               bool& nonfinite) {
  const int i0 = c0 + (int)threadIdx.x * EPT;
  float x[EPT];
  const int64_t base = (int64_t)r * a.row_stride;
  if (a.dtype == STRIM_DTYPE_BF16) {
    const uint16_t* xb = (const uint16_t*)a.logits + base;
    if (a.vec_ok && i0 + EPT <= a.V) {
      uint4 v = *(const uint4*)(xb + i0);
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
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
      float4 v0 = *(const float4*)(xf + i0);
      float4 v1 = *(const float4*)(xf + i0 + 4);
      x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w;
      x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) x[e] = (i0 + e < a.V) ? xf[i0 + e] : 0.0f;
    }
  }
  uint32_t bits = 0xFFu;
  if (a.mask && i0 < a.V) {
    uint32_t wd = a.mask[(int64_t)r * a.mask_stride + (i0 >> 5)];
    bits = (wd >> (i0 & 31)) & 0xFFu;
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    float v = x[e];
    if (p.pen) {
      uint32_t cnt = s_cnt[threadIdx.x * EPT + e];
      if (cnt > 0u) {
        v = v > 0.0f ? v / p.rep : v * p.rep;
        v = v - p.freq * (float)cnt;
        v = v - p.pres;
      }
    }
    const bool ok = (i0 + e < a.V) && ((bits >> e) & 1u);
    if (!ok) {
      l[e] = -INFINITY;
      continue;
    }
    if (isnan(v) || v == INFINITY) nonfinite = true;
    float lv = p.greedy ? v : v / p.T;
    if (lv == INFINITY) nonfinite = true;
    l[e] = lv;
  }
}

}  // namespace strim
