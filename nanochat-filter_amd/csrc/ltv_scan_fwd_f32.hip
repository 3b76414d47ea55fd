// Scan forward kernels for fp32 I/O.
#include "ltv_scan_launch.hpp"

namespace ltv {
int scan_fwd_launch_f32(const FwdArgs& a, ScanCfg c, int grid, bool vec, int gm,
                        hipStream_t st) {
  return scan_fwd_launch_t<float>(a, c, grid, vec, gm, st);
}
int scan_fwd_chain_launch_f32(const FwdArgs& a, const ChainArgs& ch, ScanCfg c, int gm,
                              hipStream_t st) {
  return scan_fwd_chain_launch_t<float>(a, ch, c, gm, st);
}
}  // namespace ltv
