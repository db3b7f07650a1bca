// The LDS-tiled GEMM (gemm_f32_mfma, gemm_kernels.h): the launcher of one
// tile form and one A orientation, chosen by IH_TILE_FORM and IH_TILE_TA.
// inferc_amd/build.py compiles this file once per (form, orientation), so
// the eight sets of kernels compile in parallel.
#include "gemm_kernels.h"

#if !defined(IH_TILE_FORM) || !defined(IH_TILE_TA)
#error "gemm_tile.hip is compiled once per tile form by inferc_amd/build.py"
#endif

namespace ih {

template <int FORM, bool TA>
void gemm_launch_tile(const GemmParams& p, int64_t slices, bool tb, bool vec, hipStream_t s) {
  if constexpr (FORM == 0)
    launch_tile<128, 128, 16, 2, 2, TA>(p, slices, tb, vec, s);
  else if constexpr (FORM == 1)
    launch_tile<128, 96, 32, 4, 1, TA>(p, slices, tb, vec, s);
  else if constexpr (FORM == 2)
    launch_tile<128, 64, 16, 2, 2, TA>(p, slices, tb, vec, s);
  else
    launch_tile<64, 64, 32, 2, 2, TA>(p, slices, tb, vec, s);
}

template void gemm_launch_tile<IH_TILE_FORM, bool(IH_TILE_TA)>(const GemmParams&, int64_t, bool,
                                                               bool, hipStream_t);

}  // namespace ih
