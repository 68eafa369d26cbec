// stream_kernels.hip — the k_stream variants of one (dtype, penalties, segments) triple
// and their launcher. Built once per triple with STRIM_DT (STRIM_DTYPE_BF16 or
// STRIM_DTYPE_F32), STRIM_PEN (0: none, 1: 32-bit history counts, 2: 16-bit) and
// STRIM_SSEG (1 or 4) defined, so the variants compile in parallel objects.
#include "stream.hpp"

#if !defined(STRIM_DT) || !defined(STRIM_PEN) || !defined(STRIM_SSEG)
#error "build with -DSTRIM_DT=<dtype> -DSTRIM_PEN=<0|1|2> -DSTRIM_SSEG=<1|4>"
#endif

namespace strim {

// One k_stream launch: the preloaded leading arguments, then the argument block.
inline hipError_t launch_stream_args(const void* fn, dim3 grid, dim3 blk, const Args& a,
                                     hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  const void* lg = a.logits;
  int rs = pre_wide(a) ? 0 : (int)a.row_stride, ms = pre_wide(a) ? 0 : (int)a.mask_stride;
  const int32_t* h = a.hist;
  const uint32_t* mk = a.mask;
  int H = a.H, V = a.V, W = a.W, R = a.R, f = pre_bits(a);
  void* args[] = {&lg, &rs, &h, &mk, &ms, &H, &V, &W, &R, &f, const_cast<Args*>(&a)};
  if (e0 || e1) return hipExtLaunchKernel(fn, grid, blk, args, 0, st, e0, e1, 0);
  return hipLaunchKernel(fn, grid, blk, args, 0, st);
}

template <int DT, int PEN, int SSEG>
hipError_t launch_stream_group(const Args& a, dim3 grid, hipStream_t st, hipEvent_t e0,
                               hipEvent_t e1) {
  const dim3 blk(stpb<SSEG>());
#define STRIM_K(VEC, MASK, GEN) \
  launch_stream_args((const void*)k_stream<DT, VEC, PEN, MASK, SSEG, GEN>, grid, blk, a, st, \
                     e0, e1)
  if constexpr (PEN == 1) {
    // unaligned logits take the general variant (penalties and mask checked per row)
    if (a.vec_ok == 0) return a.gen ? STRIM_K(false, true, true) : STRIM_K(false, true, false);
  }
  if (a.mask != nullptr) return a.gen ? STRIM_K(true, true, true) : STRIM_K(true, true, false);
  return a.gen ? STRIM_K(true, false, true) : STRIM_K(true, false, false);
#undef STRIM_K
}

template hipError_t launch_stream_group<STRIM_DT, STRIM_PEN, STRIM_SSEG>(
    const Args&, dim3, hipStream_t, hipEvent_t, hipEvent_t);

}  // namespace strim
