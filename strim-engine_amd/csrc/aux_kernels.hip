// aux_kernels.hip — standalone ops of the path: the mask applier and the draft map.
#include "kernels.hpp"

namespace strim {

// maskLogits (Sources/StrimCore/TokenMask.swift:15-17): where(mask, f32(logits), -inf),
// reading the packed allow-bits directly instead of a host-expanded bool row.
__global__ __launch_bounds__(256) void k_mask_logits(const void* logits, int dtype, int V,
                                                     int64_t row_stride, const uint32_t* mask,
                                                     int64_t mask_stride, float* out) {
  const int r = blockIdx.y;
  const int i0 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (i0 >= V) return;
  uint32_t bits = 0xFu;
  if (mask) bits = (mask[(int64_t)r * mask_stride + (i0 >> 5)] >> (i0 & 31)) & 0xFu;
  for (int e = 0; e < 4 && i0 + e < V; ++e) {
    const int64_t src = (int64_t)r * row_stride + i0 + e;
    const float x = dtype == STRIM_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)logits)[src])
                                              : ((const float*)logits)[src];
    out[(int64_t)r * V + i0 + e] = ((bits >> e) & 1u) ? x : -INFINITY;
  }
}

// MTP.nextTokenIndex (Sources/StrimCore/MTP.swift:104-111): argMax over the truncated
// draft vocab (first max), then the draft->full index table.
__global__ __launch_bounds__(256) void k_draft_argmax(const void* logits, int dtype, int Vd,
                                                      int64_t row_stride, const int32_t* table,
                                                      int32_t* out) {
  __shared__ float s_v[256 / WAVE];
  __shared__ int s_i[256 / WAVE];
  const int r = blockIdx.x;
  float bv = -INFINITY;
  int bi = -1;
  for (int i = threadIdx.x; i < Vd; i += 256) {
    const int64_t src = (int64_t)r * row_stride + i;
    const float x = dtype == STRIM_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)logits)[src])
                                              : ((const float*)logits)[src];
    // NaN never wins; -inf rows fall back to index 0 like argMax over all -inf
    if (!isnan(x)) argmax_merge(bv, bi, x, i);
  }
  wave_argmax(bv, bi);
  if ((threadIdx.x & (WAVE - 1)) == 0) {
    s_v[threadIdx.x / WAVE] = bv;
    s_i[threadIdx.x / WAVE] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < 256 / WAVE; ++q) argmax_merge(s_v[0], s_i[0], s_v[q], s_i[q]);
    int am = s_i[0] < 0 ? 0 : s_i[0];
    out[r] = table ? table[am] : am;
  }
}

}  // namespace strim
