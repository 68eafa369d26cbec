// stream_kernels.hip — the k_stream variants of one (dtype, penalties, segments) triple
// and their launcher. Built once per triple with STRIM_DT (STRIM_DTYPE_BF16 or
// STRIM_DTYPE_F32), STRIM_PEN (0 or 1) and STRIM_SSEG (1 or 4) defined, so the variants
// compile in parallel objects.
#include "stream.hpp"

#if !defined(STRIM_DT) || !defined(STRIM_PEN) || !defined(STRIM_SSEG)
#error "build with -DSTRIM_DT=<dtype> -DSTRIM_PEN=<0|1> -DSTRIM_SSEG=<1|4>"
#endif

namespace strim {

template <int DT, bool PEN, int SSEG>
hipError_t launch_stream_group(const Args& a, dim3 grid, hipStream_t st, hipEvent_t e0,
                               hipEvent_t e1) {
  const dim3 blk(stpb<SSEG>());
  if constexpr (PEN) {
    // unaligned logits take the general variant (penalties and mask checked per row)
    if (a.vec_ok == 0)
      return launch_args((const void*)k_stream<DT, false, true, true, SSEG>, grid, blk, a, st,
                         e0, e1);
  }
  if (a.mask != nullptr)
    return launch_args((const void*)k_stream<DT, true, PEN, true, SSEG>, grid, blk, a, st, e0, e1);
  return launch_args((const void*)k_stream<DT, true, PEN, false, SSEG>, grid, blk, a, st, e0, e1);
}

template hipError_t launch_stream_group<STRIM_DT, (STRIM_PEN != 0), STRIM_SSEG>(
    const Args&, dim3, hipStream_t, hipEvent_t, hipEvent_t);

}  // namespace strim
