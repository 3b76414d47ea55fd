// Scan backward kernels for fp32 I/O.
#include "ltv_scan_launch.hpp"

namespace ltv {
int scan_bwd_launch_f32(const BwdArgs& a, ScanCfg c, int grid, bool vec, int gm, bool lb,
                        hipStream_t st) {
  return scan_bwd_launch_t<float>(a, c, grid, vec, gm, lb, st);
}
int scan_bwd_chain_launch_f32(const BwdArgs& a, ScanCfg c, int grid, int gm, hipStream_t st) {
  return scan_bwd_chain_launch_t<float>(a, c, grid, gm, st);
}
}  // namespace ltv
