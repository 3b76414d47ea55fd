// Backward scan kernel instantiations and launchers.
#include "ltv_scan_kernels.hpp"

namespace ltv {
namespace {

// dbias[h, j] = sum_b partial[b, h, j], fixed order.
__global__ void dbias_reduce_kernel(const float* __restrict__ partial, float* __restrict__ dbias,
                                    int B, int HDa) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < HDa; i += gridDim.x * blockDim.x) {
    float acc = 0.0f;
    for (int b = 0; b < B; ++b) acc += partial[(int64_t)b * HDa + i];
    dbias[i] = acc;
  }
}

template <typename TIO, int CL, bool VEC, bool LG>
void launch_bwd_t(const BwdArgs& a, int grid, hipStream_t st) {
  hipLaunchKernelGGL((scan_bwd_kernel<TIO, CL, kScanL, kScanNW, VEC, LG>), dim3(grid),
                     dim3(kScanNW * 64), 0, st, a);
}

template <typename TIO, int CL>
void launch_bwd_cl(const BwdArgs& a, int grid, bool vec, bool lg, hipStream_t st) {
  if (vec) {
    if (lg) launch_bwd_t<TIO, CL, true, true>(a, grid, st);
    else launch_bwd_t<TIO, CL, true, false>(a, grid, st);
  } else {
    if (lg) launch_bwd_t<TIO, CL, false, true>(a, grid, st);
    else launch_bwd_t<TIO, CL, false, false>(a, grid, st);
  }
}

template <typename TIO>
int launch_bwd(const BwdArgs& a, int CL, int grid, bool vec, bool lg, hipStream_t st) {
  switch (CL) {
    case 1: launch_bwd_cl<TIO, 1>(a, grid, vec, lg, st); break;
    case 2: launch_bwd_cl<TIO, 2>(a, grid, vec, lg, st); break;
    case 4: launch_bwd_cl<TIO, 4>(a, grid, vec, lg, st); break;
    case 8: launch_bwd_cl<TIO, 8>(a, grid, vec, lg, st); break;
    case 16: launch_bwd_cl<TIO, 16>(a, grid, vec, lg, st); break;
    case 32: launch_bwd_cl<TIO, 32>(a, grid, vec, lg, st); break;
    case 64: launch_bwd_cl<TIO, 64>(a, grid, vec, lg, st); break;
    default:
      set_error("internal: unsupported channel-lane count %d", CL);
      return LTV_ERR_UNSUPPORTED;
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

}  // namespace

int scan_launch_bwd(bool bf16, const BwdArgs& a, int CL, int grid, bool vec, bool lanegate,
                    hipStream_t st) {
  return bf16 ? launch_bwd<bf16_t>(a, CL, grid, vec, lanegate, st)
              : launch_bwd<float>(a, CL, grid, vec, lanegate, st);
}

int scan_launch_bwd_channel(bool bf16, const BwdArgs& a, float* dalpha, hipStream_t st) {
  const ScanShape& S = a.sh;
  const int64_t n = (int64_t)S.B * S.H * S.D;
  const int threads = 256;
  const int blocks = (int)((n + threads - 1) / threads);
  const int64_t ng = (int64_t)S.B * S.H * S.Da;
  const int gblocks = (int)((ng + threads - 1) / threads);
  if (bf16) {
    hipLaunchKernelGGL(scan_bwd_channel_kernel<bf16_t>, dim3(blocks), dim3(threads), 0, st, a,
                       dalpha);
    LTV_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_bwd_group_reduce_kernel<bf16_t>, dim3(gblocks), dim3(threads), 0,
                       st, a, dalpha);
  } else {
    hipLaunchKernelGGL(scan_bwd_channel_kernel<float>, dim3(blocks), dim3(threads), 0, st, a,
                       dalpha);
    LTV_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_bwd_group_reduce_kernel<float>, dim3(gblocks), dim3(threads), 0, st,
                       a, dalpha);
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

int scan_launch_dbias_reduce(const float* partial, float* dbias, int B, int HDa,
                             hipStream_t st) {
  hipLaunchKernelGGL(dbias_reduce_kernel, dim3((HDa + 255) / 256), dim3(256), 0, st, partial,
                     dbias, B, HDa);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

}  // namespace ltv
