// Scan forward kernels for bf16 I/O.
#include "ltv_scan_launch.hpp"

namespace ltv {
int scan_fwd_launch_bf16(const FwdArgs& a, ScanCfg c, int grid, bool vec, int gm,
                        hipStream_t st) {
  return scan_fwd_launch_t<bf16_t>(a, c, grid, vec, gm, st);
}
int scan_fwd_chain_launch_bf16(const FwdArgs& a, const ChainArgs& ch, ScanCfg c, int gm,
                               hipStream_t st) {
  return scan_fwd_chain_launch_t<bf16_t>(a, ch, c, gm, st);
}
}  // namespace ltv
