// Kernel instantiation and dispatch of the scan for one I/O dtype.  Included by
// ltv_scan_{fwd,bwd}_{bf16,f32}.hip, one translation unit per direction and
// dtype so the instantiations build in parallel.
//
// Launch shapes (CL channel lanes, L steps per lane, NW wavefronts) are template
// parameters.  Every CL in {1, ..., 64} is built with (L, NW) = (4, 4); for the
// channel-lane counts the d12 shapes use, a few more (L, NW) pairs are built so
// the launch shape can be tuned (LTV_SCAN_FWD_CFG / LTV_SCAN_BWD_CFG).
#pragma once

#include "ltv_scan_kernels.hpp"

namespace ltv {
namespace detail {

template <int CL, int L, int NW>
constexpr bool is_base_cfg() {
  return L == 4 && NW == 4;
}

template <typename TIO, int CL, int L, int NW>
bool fwd_dispatch(const FwdArgs& a, int grid, bool vec, int gm, hipStream_t st) {
  const dim3 blk(NW * 64);
  if (vec) {
    switch (gm) {
      case GATE_LANE:
        hipLaunchKernelGGL((scan_fwd_kernel<TIO, CL, L, NW, true, GATE_LANE>), dim3(grid), blk, 0, st, a);
        return true;
      case GATE_CHAN:
        hipLaunchKernelGGL((scan_fwd_kernel<TIO, CL, L, NW, true, GATE_CHAN>), dim3(grid), blk, 0, st, a);
        return true;
      case GATE_CHANVEC:
        hipLaunchKernelGGL((scan_fwd_kernel<TIO, CL, L, NW, true, GATE_CHANVEC>), dim3(grid), blk, 0, st, a);
        return true;
      default:
        return false;
    }
  }
  if constexpr (is_base_cfg<CL, L, NW>()) {
    switch (gm) {
      case GATE_LANE:
        hipLaunchKernelGGL((scan_fwd_kernel<TIO, CL, L, NW, false, GATE_LANE>), dim3(grid), blk, 0, st, a);
        return true;
      case GATE_CHAN:
        hipLaunchKernelGGL((scan_fwd_kernel<TIO, CL, L, NW, false, GATE_CHAN>), dim3(grid), blk, 0, st, a);
        return true;
      default:
        return false;
    }
  }
  return false;
}

template <typename TIO, int CL, int L, int NW>
bool fwd_chain_dispatch(const FwdArgs& a, const ChainArgs& ch, int grid, int gm, hipStream_t st) {
  const dim3 blk(NW * 64);
  switch (gm) {
    case GATE_LANE:
      hipLaunchKernelGGL((scan_fwd_chain_kernel<TIO, CL, L, NW, true, GATE_LANE>), dim3(grid), blk, 0, st, a, ch);
      return true;
    case GATE_CHANVEC:
      hipLaunchKernelGGL((scan_fwd_chain_kernel<TIO, CL, L, NW, true, GATE_CHANVEC>), dim3(grid), blk, 0, st, a, ch);
      return true;
    default:
      return false;
  }
}

// The look-back backward is built for the base shapes and for the shape the
// d12 heads use (16 channel lanes, 4 steps per lane, 2 wavefronts).
template <int CL, int L, int NW>
constexpr bool is_lb_cfg() {
  return is_base_cfg<CL, L, NW>() || (CL == 16 && L == 4 && NW == 2);
}

template <typename TIO, int CL, int L, int NW, bool LB>
bool bwd_dispatch_lb(const BwdArgs& a, int grid, bool vec, int gm, hipStream_t st) {
  const dim3 blk(NW * 64);
  if (vec) {
    switch (gm) {
      case GATE_LANE:
        hipLaunchKernelGGL((scan_bwd_kernel<TIO, CL, L, NW, true, GATE_LANE, LB>), dim3(grid), blk, 0, st, a);
        return true;
      case GATE_CHAN:
        hipLaunchKernelGGL((scan_bwd_kernel<TIO, CL, L, NW, true, GATE_CHAN, LB>), dim3(grid), blk, 0, st, a);
        return true;
      case GATE_CHANVEC:
        hipLaunchKernelGGL((scan_bwd_kernel<TIO, CL, L, NW, true, GATE_CHANVEC, LB>), dim3(grid), blk, 0, st, a);
        return true;
      default:
        return false;
    }
  }
  if constexpr (is_base_cfg<CL, L, NW>()) {
    switch (gm) {
      case GATE_LANE:
        hipLaunchKernelGGL((scan_bwd_kernel<TIO, CL, L, NW, false, GATE_LANE, LB>), dim3(grid), blk, 0, st, a);
        return true;
      case GATE_CHAN:
        hipLaunchKernelGGL((scan_bwd_kernel<TIO, CL, L, NW, false, GATE_CHAN, LB>), dim3(grid), blk, 0, st, a);
        return true;
      default:
        return false;
    }
  }
  return false;
}

template <typename TIO, int CL, int L, int NW>
bool bwd_dispatch(const BwdArgs& a, int grid, bool vec, int gm, bool lb, hipStream_t st) {
  if (!lb) return bwd_dispatch_lb<TIO, CL, L, NW, false>(a, grid, vec, gm, st);
  if constexpr (is_lb_cfg<CL, L, NW>()) return bwd_dispatch_lb<TIO, CL, L, NW, true>(a, grid, vec, gm, st);
  return false;
}

template <typename TIO, int CL, int L, int NW>
bool bwd_chain_dispatch(const BwdArgs& a, int grid, int gm, hipStream_t st) {
  const dim3 blk(NW * 64);
  switch (gm) {
    case GATE_LANE:
      hipLaunchKernelGGL((scan_bwd_kernel<TIO, CL, L, NW, true, GATE_LANE, false, true>), dim3(grid), blk, 0, st, a);
      return true;
    case GATE_CHANVEC:
      hipLaunchKernelGGL((scan_bwd_kernel<TIO, CL, L, NW, true, GATE_CHANVEC, false, true>), dim3(grid), blk, 0, st, a);
      return true;
    default:
      return false;
  }
}

}  // namespace detail

// The launch shapes built for each direction: (CL, L, NW).
#define LTV_SCAN_FWD_CONFIGS(X)                                                        \
  X(1, 4, 4) X(2, 4, 4) X(4, 4, 4) X(8, 4, 4) X(16, 4, 4) X(32, 4, 4) X(64, 4, 4)      \
  X(8, 8, 4) X(8, 2, 4) X(8, 4, 2) X(16, 8, 4) X(4, 8, 4)
#define LTV_SCAN_BWD_CONFIGS(X)                                                        \
  X(1, 4, 4) X(2, 4, 4) X(4, 4, 4) X(8, 4, 4) X(16, 4, 4) X(32, 4, 4) X(64, 4, 4)      \
  X(16, 4, 2) X(16, 2, 4)

template <typename TIO>
int scan_fwd_launch_t(const FwdArgs& a, ScanCfg c, int grid, bool vec, int gm, hipStream_t st) {
  bool ok = false;
#define LTV_X(CL_, L_, NW_)                                                   \
  if (!ok && c.CL == CL_ && c.L == L_ && c.NW == NW_)                         \
    ok = detail::fwd_dispatch<TIO, CL_, L_, NW_>(a, grid, vec, gm, st);
  LTV_SCAN_FWD_CONFIGS(LTV_X)
#undef LTV_X
  if (!ok) {
    set_error("scan forward: launch shape CL=%d L=%d NW=%d (vec=%d gate=%d) is not built",
              c.CL, c.L, c.NW, (int)vec, gm);
    return LTV_ERR_UNSUPPORTED;
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

// Chained forward shapes (CL, L, NW); a slab's CL * V channels fit one
// wavefront (CL <= 8 for bf16, <= 16 for fp32).
#define LTV_SCAN_FWD_CHAIN_CONFIGS(X) \
  X(8, 16, 4) X(8, 8, 4) X(8, 8, 8) X(8, 4, 4) X(8, 4, 8) X(8, 2, 4)

template <typename TIO>
int scan_fwd_chain_launch_t(const FwdArgs& a, const ChainArgs& ch, ScanCfg c, int gm,
                            hipStream_t st) {
  const int64_t grid = (int64_t)ch.nseq * ch.nchunk;
  if (grid <= 0 || grid >= (1ll << 31)) {
    set_error("scan forward (chained): grid of %lld workgroups", (long long)grid);
    return LTV_ERR_UNSUPPORTED;
  }
  bool ok = false;
#define LTV_X(CL_, L_, NW_)                                                   \
  if (!ok && c.CL == CL_ && c.L == L_ && c.NW == NW_)                         \
    ok = detail::fwd_chain_dispatch<TIO, CL_, L_, NW_>(a, ch, (int)grid, gm, st);
  LTV_SCAN_FWD_CHAIN_CONFIGS(LTV_X)
#undef LTV_X
  if (!ok) {
    set_error("scan forward (chained): launch shape CL=%d L=%d NW=%d (gate=%d) is not built",
              c.CL, c.L, c.NW, gm);
    return LTV_ERR_UNSUPPORTED;
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

template <typename TIO>
int scan_bwd_launch_t(const BwdArgs& a, ScanCfg c, int grid, bool vec, int gm, bool lb,
                      hipStream_t st) {
  bool ok = false;
#define LTV_X(CL_, L_, NW_)                                                   \
  if (!ok && c.CL == CL_ && c.L == L_ && c.NW == NW_)                         \
    ok = detail::bwd_dispatch<TIO, CL_, L_, NW_>(a, grid, vec, gm, lb, st);
  LTV_SCAN_BWD_CONFIGS(LTV_X)
#undef LTV_X
  if (!ok) {
    set_error("scan backward: launch shape CL=%d L=%d NW=%d (vec=%d gate=%d look-back=%d) is not built",
              c.CL, c.L, c.NW, (int)vec, gm, (int)lb);
    return LTV_ERR_UNSUPPORTED;
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

// Chained backward shapes (CL, L, NW): a whole head per workgroup, its CL V
// channel slots at most the workgroup's threads.
#define LTV_SCAN_BWD_CHAIN_CONFIGS(X) \
  X(16, 4, 2) X(16, 4, 4) X(16, 8, 2) X(16, 8, 4) X(16, 2, 4) X(8, 4, 4) X(32, 4, 4) X(32, 4, 2)

template <typename TIO>
int scan_bwd_chain_launch_t(const BwdArgs& a, ScanCfg c, int grid, int gm, hipStream_t st) {
  bool ok = false;
#define LTV_X(CL_, L_, NW_)                                                   \
  if constexpr (CL_ * Pack<TIO>::V <= NW_ * 64)                               \
    if (!ok && c.CL == CL_ && c.L == L_ && c.NW == NW_)                       \
      ok = detail::bwd_chain_dispatch<TIO, CL_, L_, NW_>(a, grid, gm, st);
  LTV_SCAN_BWD_CHAIN_CONFIGS(LTV_X)
#undef LTV_X
  if (!ok) {
    set_error("scan backward (chained): launch shape CL=%d L=%d NW=%d (gate=%d) is not built",
              c.CL, c.L, c.NW, gm);
    return LTV_ERR_UNSUPPORTED;
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

// Per-dtype entry points (defined in the four translation units).
int scan_fwd_launch_bf16(const FwdArgs& a, ScanCfg c, int grid, bool vec, int gm, hipStream_t st);
int scan_fwd_launch_f32(const FwdArgs& a, ScanCfg c, int grid, bool vec, int gm, hipStream_t st);
int scan_fwd_chain_launch_bf16(const FwdArgs& a, const ChainArgs& ch, ScanCfg c, int gm,
                               hipStream_t st);
int scan_fwd_chain_launch_f32(const FwdArgs& a, const ChainArgs& ch, ScanCfg c, int gm,
                              hipStream_t st);
int scan_bwd_launch_bf16(const BwdArgs& a, ScanCfg c, int grid, bool vec, int gm, bool lb,
                         hipStream_t st);
int scan_bwd_launch_f32(const BwdArgs& a, ScanCfg c, int grid, bool vec, int gm, bool lb,
                        hipStream_t st);
int scan_bwd_chain_launch_bf16(const BwdArgs& a, ScanCfg c, int grid, int gm, hipStream_t st);
int scan_bwd_chain_launch_f32(const BwdArgs& a, ScanCfg c, int grid, int gm, hipStream_t st);

}  // namespace ltv
