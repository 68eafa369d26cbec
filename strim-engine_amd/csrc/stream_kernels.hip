// stream_kernels.hip — the k_stream variants of one (dtype, penalties, segments) triple
// and their launcher. Built once per triple with STRIM_DT (STRIM_DTYPE_BF16 or
// STRIM_DTYPE_F32), STRIM_PEN (0: none, 1: 32-bit history counts, 2: 16-bit) and
// STRIM_SSEG (1 or 4) defined, so the variants compile in parallel objects.
#include "stream.hpp"

#if !defined(STRIM_DT) || !defined(STRIM_PEN) || !defined(STRIM_SSEG)
#error "build with -DSTRIM_DT=<dtype> -DSTRIM_PEN=<0|1|2> -DSTRIM_SSEG=<1|4>"
#endif

namespace strim {

template <int DT, int PEN, int SSEG>
hipError_t launch_stream_group(const Args& a, dim3 grid, hipStream_t st, hipEvent_t e0,
                               hipEvent_t e1) {
  const dim3 blk(stpb<SSEG>());
#define STRIM_K(VEC, MASK, GEN) \
  launch_args((const void*)k_stream<DT, VEC, PEN, MASK, SSEG, GEN>, grid, blk, a, st, e0, e1)
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
