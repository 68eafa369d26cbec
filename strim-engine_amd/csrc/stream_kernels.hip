// stream_kernels.hip — the k_stream variants of one (dtype, penalties) pair and their
// launcher. Built once per pair with STRIM_DT (STRIM_DTYPE_BF16 or STRIM_DTYPE_F32) and
// STRIM_PEN (0 or 1) defined, so the variants compile in parallel objects.
#include "stream.hpp"

#if !defined(STRIM_DT) || !defined(STRIM_PEN)
#error "build with -DSTRIM_DT=<dtype> -DSTRIM_PEN=<0|1>"
#endif

namespace strim {

template <int DT, bool PEN>
hipError_t launch_stream_group(const Args& a, dim3 grid, hipStream_t st, hipEvent_t e0,
                               hipEvent_t e1) {
  const dim3 blk(STPB);
  if constexpr (PEN) {
    // unaligned logits take the general variant (penalties and mask checked per row)
    if (a.vec_ok == 0)
      return launch_args((const void*)k_stream<DT, false, true, true>, grid, blk, a, st, e0, e1);
  }
  if (a.mask != nullptr)
    return launch_args((const void*)k_stream<DT, true, PEN, true>, grid, blk, a, st, e0, e1);
  return launch_args((const void*)k_stream<DT, true, PEN, false>, grid, blk, a, st, e0, e1);
}

template hipError_t launch_stream_group<STRIM_DT, (STRIM_PEN != 0)>(const Args&, dim3, hipStream_t,
                                                                    hipEvent_t, hipEvent_t);

}  // namespace strim
