// Forward scan kernel instantiations and launcher.
#include "ltv_scan_kernels.hpp"

namespace ltv {
namespace {

template <typename TIO, int CL, bool VEC, bool LG>
void launch_fwd_t(const FwdArgs& a, int grid, hipStream_t st) {
  hipLaunchKernelGGL((scan_fwd_kernel<TIO, CL, kScanL, kScanNW, VEC, LG>), dim3(grid),
                     dim3(kScanNW * 64), 0, st, a);
}

template <typename TIO, int CL>
void launch_fwd_cl(const FwdArgs& a, int grid, bool vec, bool lg, hipStream_t st) {
  if (vec) {
    if (lg) launch_fwd_t<TIO, CL, true, true>(a, grid, st);
    else launch_fwd_t<TIO, CL, true, false>(a, grid, st);
  } else {
    if (lg) launch_fwd_t<TIO, CL, false, true>(a, grid, st);
    else launch_fwd_t<TIO, CL, false, false>(a, grid, st);
  }
}

template <typename TIO>
int launch_fwd(const FwdArgs& a, int CL, int grid, bool vec, bool lg, hipStream_t st) {
  switch (CL) {
    case 1: launch_fwd_cl<TIO, 1>(a, grid, vec, lg, st); break;
    case 2: launch_fwd_cl<TIO, 2>(a, grid, vec, lg, st); break;
    case 4: launch_fwd_cl<TIO, 4>(a, grid, vec, lg, st); break;
    case 8: launch_fwd_cl<TIO, 8>(a, grid, vec, lg, st); break;
    case 16: launch_fwd_cl<TIO, 16>(a, grid, vec, lg, st); break;
    case 32: launch_fwd_cl<TIO, 32>(a, grid, vec, lg, st); break;
    case 64: launch_fwd_cl<TIO, 64>(a, grid, vec, lg, st); break;
    default:
      set_error("internal: unsupported channel-lane count %d", CL);
      return LTV_ERR_UNSUPPORTED;
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

}  // namespace

int scan_launch_fwd(bool bf16, const FwdArgs& a, int CL, int grid, bool vec, bool lanegate,
                    hipStream_t st) {
  return bf16 ? launch_fwd<bf16_t>(a, CL, grid, vec, lanegate, st)
              : launch_fwd<float>(a, CL, grid, vec, lanegate, st);
}

}  // namespace ltv
