// head_kernels.hip — the producer of the logits the path reads: the decode step's final
// RMSNorm and lm_head linear (QwenModel.swift:202-212; Weights.swift:244-255,270-273), for
// dense bf16 weights, on MFMA, writing the bf16 logits in the layout strim_sample takes.
//
// k_head_norm: one workgroup per row, xn = bf16(w * bf16(x * inv)) with
//   inv = 1 / sqrt(mean(x^2) + eps), the squares summed in double.
// k_head_gemv: logits[b][v] = bf16(sum_k xn[b][k] W[v][k]) with float accumulation. A
//   workgroup owns 128 vocabulary rows (four waves of two 16-row tiles) over the whole of K,
//   so the 1,187 workgroups of V = 151,936 each stream 1.3 MB of weights once, and the
//   weight matrix is read exactly once per call whatever the batch. The batch is the
//   MFMA's N side (16 rows per tile, up to four tiles), read from the L2-resident xn.
//   For a greedy pick (strim_head_greedy) its epilogue also writes each batch row's first
//   maximum over the workgroup's 128 logits (as bf16 values, as the sampler reads them),
//   and the logits may be left unwritten.
// k_head_pick: one workgroup per batch row merges the rows' tile maxima into the first
//   maximum of the row: the greedy token, with the sampler's statuses (a NaN or +inf logit:
//   STRIM_ENONFINITE; every logit -inf: STRIM_EEMPTY).
//
// MFMA operand layout (v_mfma_f32_16x16x32_bf16; checked on the device): lane l holds
// A[l % 16][8 (l / 16) + i] and B[8 (l / 16) + i][l % 16] for i < 8, and C[4 (l / 16) + i]
// [l % 16] for i < 4. A step of 128 elements of K is four MFMAs; MFMA q takes elements
// 32 q + 8 (l / 16) + i of the weight row and of the xn row, so each wave-wide load reads
// 64 contiguous bytes of each of 16 rows.
#include "kernels.hpp"

namespace strim {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int HN_T = 256;               // k_head_norm threads
constexpr int HG_W = 4;                 // k_head_gemv waves per workgroup
constexpr int HG_MT = 2;                // 16-row vocabulary tiles per wave
constexpr int HG_KS = 128;              // K elements per step (four MFMAs of K 32)

// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t head_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__global__ __launch_bounds__(HN_T) void k_head_norm(const uint16_t* x, int64_t x_stride, int K,
                                                    const uint16_t* w, float eps,
                                                    uint16_t* xn) {
  __shared__ double s_d[HN_T / WAVE];
  const int b = blockIdx.x, t = threadIdx.x;
  const uint16_t* xr = x + (int64_t)b * x_stride;
  double ss = 0.0;
  for (int k = 8 * t; k < K; k += 8 * HN_T) {
    const uint4 q = *(const uint4*)(xr + k);
    const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = __uint_as_float(wd[e] << 16), hi = __uint_as_float(wd[e] & 0xFFFF0000u);
      ss += (double)lo * (double)lo + (double)hi * (double)hi;
    }
  }
  ss = wave_sum(ss);
  if ((t & (WAVE - 1)) == 0) s_d[t / WAVE] = ss;
  __syncthreads();
  double tot = 0.0;
#pragma unroll
  for (int q = 0; q < HN_T / WAVE; ++q) tot += s_d[q];
  const float inv = 1.0f / sqrtf((float)(tot / (double)K) + eps);
  for (int k = 8 * t; k < K; k += 8 * HN_T) {
    const uint4 q = *(const uint4*)(xr + k);
    const uint4 g = *(const uint4*)(w + k);
    const uint32_t xd[4] = {q.x, q.y, q.z, q.w}, gd[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t r = 0u;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const float xv = __uint_as_float(hf ? (xd[e] & 0xFFFF0000u) : (xd[e] << 16));
        const float gv = __uint_as_float(hf ? (gd[e] & 0xFFFF0000u) : (gd[e] << 16));
        const float y = bf16_to_f32(head_bf16(xv * inv));
        r |= (uint32_t)head_bf16(gv * y) << (16 * hf);
      }
      o[e] = r;
    }
    *(uint4*)(xn + (int64_t)b * K + k) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// NT: 16-row batch tiles (B <= 16 NT). VO: 8-byte logit stores (rows 4-element aligned).
// MT: 16-row vocabulary tiles per wave; NW: waves per workgroup; NTL: weights loaded
// nontemporal (streamed once, kept out of the caches that hold xn).
// The larger of two (value, id) pairs, the smaller id on equal values (NaN never taken).
__device__ __forceinline__ void hb_take(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// TB: write the tile maxima to tbest[n][blockIdx.x] = {value bits (NaN: the tile holds a
// NaN or +inf), id}; out NULL: no logits stored.
template <int NT, bool VO, bool TB = false, int MT = HG_MT, int NW = HG_W, bool NTL = false>
__global__ __launch_bounds__(NW* WAVE) void k_head_gemv(const uint16_t* xn, int64_t xn_stride,
                                                          int B, int K, const uint16_t* W,
                                                          int64_t w_stride, int V,
                                                          uint16_t* out, int64_t out_stride,
                                                          uint2* tbest) {
  const int lane = threadIdx.x & (WAVE - 1), wv = wave_id();
  const int h = lane >> 4, r16 = lane & 15;
  const int v0 = blockIdx.x * (NW * MT * 16) + wv * (MT * 16);
  // rows past V or B read a clamped row; their results are not stored
  const uint16_t* arow[MT];
  const uint16_t* brow[NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int v = min(v0 + mt * 16 + r16, V - 1);
    arow[mt] = W + (int64_t)v * w_stride + 8 * h;
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = min(nt * 16 + r16, B - 1);
    brow[nt] = xn + (int64_t)n * xn_stride + 8 * h;
  }
  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // two register buffers: the next step's loads are in flight while this step multiplies
  uint4 a[2][MT][4], bq[2][NT][4];
  auto loada = [&](int buf, int kb) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4_t* src = (const u32x4_t*)(arow[mt] + kb + 32 * q);
        const u32x4_t v = NTL ? __builtin_nontemporal_load(src) : *src;
        a[buf][mt][q] = make_uint4(v[0], v[1], v[2], v[3]);
      }
  };
  auto load = [&](int buf, int kb) {
    loada(buf, kb);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int q = 0; q < 4; ++q) bq[buf][nt][q] = *(const uint4*)(brow[nt] + kb + 32 * q);
  };
  auto mma = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, a[buf][mt][q]),
              __builtin_bit_cast(bf16x8_t, bq[buf][nt][q]), acc[mt][nt], 0, 0, 0);
  };
  // K is a multiple of 2 steps (the host checks), so every load and multiply is
  // unconditional (the last prefetch reloads the last step and is not used), and the
  // scheduling barriers keep each buffer's loads issued before the other buffer's
  // multiplies: left alone, the compiler sinks the loads next to their use
  const int nsteps = K / HG_KS;
  if constexpr (NT == 1) {
    load(0, 0);
    for (int s = 0; s < nsteps; s += 2) {
      load(1, (s + 1) * HG_KS);
      __builtin_amdgcn_sched_barrier(0);
      mma(0);
      __builtin_amdgcn_sched_barrier(0);
      load(0, min(s + 2, nsteps - 2) * HG_KS);
      __builtin_amdgcn_sched_barrier(0);
      mma(1);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    // Several batch tiles: every wave needs the same 16 NT rows of xn at each step, so
    // the workgroup stages them in LDS once (double-buffered, rows padded by 16 bytes so
    // the 16 rows a wave reads fall in different banks) instead of each wave reading
    // them from L2 (four times the bytes: that bound B = 64 at 2.7 TB/s). Thread t
    // carries NT 16-byte pieces of the next step's slice while this step multiplies.
    constexpr int XR = 16 * NT, XW = HG_KS + 8;  // rows, padded row length (bf16)
    __shared__ __attribute__((aligned(16))) uint16_t s_x[2][XR][XW];
    struct Slice {
      uint4 v[NT];
    };
    auto xload = [&](int kb) -> Slice {
      Slice xr;
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const int e = (int)threadIdx.x + NW * WAVE * i;  // piece e: row e / 16, column 8 (e % 16)
        const int row = e >> 4, col = (e & 15) * 8;
        const int n = min(row, B - 1);
        xr.v[i] = *(const uint4*)(xn + (int64_t)n * xn_stride + kb + col);
      }
      return xr;
    };
    auto xstore = [&](int buf, const Slice& xr) {
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const int e = (int)threadIdx.x + NW * WAVE * i;
        *(uint4*)&s_x[buf][e >> 4][(e & 15) * 8] = xr.v[i];
      }
    };
    // the multiplies of one step from LDS buffer buf, the B operand read one K slice (q)
    // at a time next to its MFMAs: NT registers of it live instead of 4 NT
    auto mma_lds = [&](int buf, int abuf) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint4 bx[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          bx[nt] = *(const uint4*)&s_x[buf][nt * 16 + r16][32 * q + 8 * h];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, a[abuf][mt][q]), __builtin_bit_cast(bf16x8_t, bx[nt]),
                acc[mt][nt], 0, 0, 0);
      }
    };
    static_assert(NT * NW * WAVE * 8 == XR * HG_KS, "one step's slice: NT pieces a thread");
    // The barrier waits for the LDS stores alone: __syncthreads' fence would also wait
    // for the next step's weight loads, the prefetch this loop depends on. The slice's
    // loads are issued before the weights', so its store waits for them only.
    auto sync_lds = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    // Unrolled by two so each register buffer has a fixed index (the host checks that K
    // is a multiple of two steps; the last prefetch reloads the last step, unused).
    xstore(0, xload(0));
    loada(0, 0);
    sync_lds();
    for (int s = 0; s < nsteps; s += 2) {
      const Slice x1 = xload((s + 1) * HG_KS);
      loada(1, (s + 1) * HG_KS);
      __builtin_amdgcn_sched_barrier(0);
      mma_lds(0, 0);
      __builtin_amdgcn_sched_barrier(0);
      xstore(1, x1);
      sync_lds();
      const int s2 = min(s + 2, nsteps - 2) * HG_KS;
      const Slice x0 = xload(s2);
      loada(0, s2);
      __builtin_amdgcn_sched_barrier(0);
      mma_lds(1, 1);
      __builtin_amdgcn_sched_barrier(0);
      xstore(0, x0);
      sync_lds();
    }
  }
  // lane l holds rows 4 h + i of each tile for batch row nt 16 + r16
  float bv[NT];
  int bi[NT];
  bool bad[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    bv[nt] = -INFINITY;
    bi[nt] = INT_MAX;
    bad[nt] = false;
    const int n = nt * 16 + r16;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int vb = v0 + mt * 16 + 4 * h;
      uint16_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = head_bf16(acc[mt][nt][i]);
      if constexpr (TB) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (vb + i < V) {
            const float f = __uint_as_float((uint32_t)o[i] << 16);
            bad[nt] = bad[nt] || !(f < INFINITY);  // NaN or +inf
            hb_take(bv[nt], bi[nt], f, vb + i);
          }
      }
      if (n >= B || out == nullptr) continue;
      uint16_t* dst = out + (int64_t)n * out_stride + vb;
      if (VO && vb + 3 < V) {
        *(uint2*)dst = make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16),
                                  (uint32_t)o[2] | ((uint32_t)o[3] << 16));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (vb + i < V) dst[i] = o[i];
      }
    }
  }
  if constexpr (TB) {
    // the four lanes of a batch row (h = 0..3), then the workgroup's waves
    __shared__ float s_v[NW][16 * NT];
    __shared__ int s_i[NW][16 * NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int sh = 16; sh < WAVE; sh <<= 1) {
        const float v2 = __shfl_xor(bv[nt], sh);
        const int i2 = __shfl_xor(bi[nt], sh);
        const bool b2 = __shfl_xor((int)bad[nt], sh) != 0;
        hb_take(bv[nt], bi[nt], v2, i2);
        bad[nt] = bad[nt] || b2;
      }
      if (h == 0) {
        s_v[wv][nt * 16 + r16] = bad[nt] ? __uint_as_float(0x7FC00000u) : bv[nt];
        s_i[wv][nt * 16 + r16] = bi[nt];
      }
    }
    __syncthreads();
    const int n = (int)threadIdx.x;
    if (n < B && n < 16 * NT) {
      float v = s_v[0][n];
      int i = s_i[0][n];
      bool nan = !(v == v);
#pragma unroll
      for (int q = 1; q < NW; ++q) {
        nan = nan || !(s_v[q][n] == s_v[q][n]);
        hb_take(v, i, s_v[q][n], s_i[q][n]);
      }
      tbest[(int64_t)n * gridDim.x + blockIdx.x] =
          make_uint2(__float_as_uint(nan ? __uint_as_float(0x7FC00000u) : v), (uint32_t)i);
    }
  }
}

constexpr int HP_T = 256;  // k_head_pick threads

__global__ __launch_bounds__(HP_T) void k_head_pick(const uint2* tbest, int ntiles,
                                                     int32_t* out_ids, int32_t* out_status) {
  __shared__ float s_v[HP_T / WAVE];
  __shared__ int s_i[HP_T / WAVE], s_bad[HP_T / WAVE];
  const int n = blockIdx.x, t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  float v = -INFINITY;
  int i = INT_MAX;
  bool bad = false;
  for (int q = t; q < ntiles; q += HP_T) {
    const uint2 r = tbest[(int64_t)n * ntiles + q];
    const float f = __uint_as_float(r.x);
    bad = bad || !(f == f);
    hb_take(v, i, f, (int)r.y);
  }
#pragma unroll
  for (int sh = 1; sh < WAVE; sh <<= 1) {
    const float v2 = __shfl_xor(v, sh);
    const int i2 = __shfl_xor(i, sh);
    bad = bad || (__shfl_xor((int)bad, sh) != 0);
    hb_take(v, i, v2, i2);
  }
  if (lane == 0) {
    s_v[w] = v;
    s_i[w] = i;
    s_bad[w] = bad ? 1 : 0;
  }
  __syncthreads();
  if (t == 0) {
    for (int q = 1; q < HP_T / WAVE; ++q) {
      hb_take(v, i, s_v[q], s_i[q]);
      bad = bad || s_bad[q];
    }
    const int st = bad ? STRIM_ENONFINITE : (v > -INFINITY ? STRIM_OK : STRIM_EEMPTY);
    out_ids[n] = st == STRIM_OK ? i : -1;
    if (out_status) out_status[n] = st;
  }
}

hipError_t launch_head(const void* hidden, int64_t hidden_stride, int B, int K,
                       const void* norm_w, float eps, void* xn, const void* W, int64_t w_stride,
                       int V, void* out, int64_t out_stride, bool vo, hipStream_t st,
                       uint2* tbest, int32_t* out_ids, int32_t* out_status) {
  const uint16_t* src = (const uint16_t*)hidden;
  int64_t src_stride = hidden_stride;
  if (norm_w) {
    hipLaunchKernelGGL(k_head_norm, dim3((unsigned)B), dim3(HN_T), 0, st, (const uint16_t*)hidden,
                       hidden_stride, K, (const uint16_t*)norm_w, eps, (uint16_t*)xn);
    src = (const uint16_t*)xn;
    src_stride = K;
  }
  // vocabulary rows per workgroup: 4 waves of HG_MT 16-row tiles (one tile a wave above
  // B = 16 measured slower: 767 against 534 us at B = 64, the staged batch slice is then
  // loaded for half as many weight rows)
  const int nt = (B + 15) / 16;
  const int rows = HG_W * HG_MT * 16;
  const dim3 grid((unsigned)((V + rows - 1) / rows)), blk(HG_W * WAVE);
#define STRIM_HEAD_GEMV(NT_, MT_)                                                                \
  if (tbest && vo)                                                                               \
    hipLaunchKernelGGL((k_head_gemv<NT_, true, true, MT_>), grid, blk, 0, st, src, src_stride, B, \
                       K, (const uint16_t*)W, w_stride, V, (uint16_t*)out, out_stride, tbest);    \
  else if (tbest)                                                                                \
    hipLaunchKernelGGL((k_head_gemv<NT_, false, true, MT_>), grid, blk, 0, st, src, src_stride,   \
                       B, K, (const uint16_t*)W, w_stride, V, (uint16_t*)out, out_stride, tbest); \
  else if (vo)                                                                                   \
    hipLaunchKernelGGL((k_head_gemv<NT_, true, false, MT_>), grid, blk, 0, st, src, src_stride,   \
                       B, K, (const uint16_t*)W, w_stride, V, (uint16_t*)out, out_stride,         \
                       nullptr);                                                                 \
  else                                                                                           \
    hipLaunchKernelGGL((k_head_gemv<NT_, false, false, MT_>), grid, blk, 0, st, src, src_stride,  \
                       B, K, (const uint16_t*)W, w_stride, V, (uint16_t*)out, out_stride,         \
                       nullptr);
  if (nt == 1) {
    STRIM_HEAD_GEMV(1, HG_MT)
  } else if (nt == 2) {
    STRIM_HEAD_GEMV(2, HG_MT)
  } else {
    STRIM_HEAD_GEMV(4, HG_MT)
  }
#undef STRIM_HEAD_GEMV
  if (tbest)
    hipLaunchKernelGGL(k_head_pick, dim3((unsigned)B), dim3(HP_T), 0, st, tbest, (int)grid.x,
                       out_ids, out_status);
  return hipGetLastError();
}

}  // namespace strim
