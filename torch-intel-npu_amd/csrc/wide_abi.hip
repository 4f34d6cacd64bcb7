// Launches of the several-row GEMV of lb_wide.h (a translation unit of its own, so the library's
// sources compile in parallel).
#include <hip/hip_runtime.h>

#include "lb_wide.h"

namespace lb {

template <int FMT, int GL>
void launch_wide_t(const WideParams &p, int slices, hipStream_t s) {
  const dim3 grid((unsigned)((p.N + kWideRows - 1) / kWideRows), (unsigned)slices);
  hipLaunchKernelGGL((wide_rows_kernel<FMT, GL, kWidePC, kWidePD>), grid, dim3(64 * kWideWaves), 0, s, p.codes, p.x,
                     p.scales, p.M, p.N, p.K, p.G, p.group_shift, p.ldx, p.kslice, p);
}

template <int FMT>
void launch_wide_f(const WideParams &p, int gl, int slices, hipStream_t s) {
  switch (gl) {
    case 2: launch_wide_t<FMT, 2>(p, slices, s); break;
    case 4: launch_wide_t<FMT, 4>(p, slices, s); break;
    case 8: launch_wide_t<FMT, 8>(p, slices, s); break;
    default:
      if constexpr (FMT == FMT_INT8) launch_wide_t<FMT, 0>(p, slices, s);
      break;
  }
}

void launch_wide(const WideParams &p, int format, int gl, int slices, hipStream_t s) {
  if (format == FMT_INT4) launch_wide_f<FMT_INT4>(p, gl, slices, s);
  else if (format == FMT_NF4) launch_wide_f<FMT_NF4>(p, gl, slices, s);
  else launch_wide_f<FMT_INT8>(p, gl, slices, s);
}

}  // namespace lb
