// C-ABI entry points of the scan: argument checks, layout views, gate-mode and
// launch-shape selection.  The main kernels are built in ltv_scan_{fwd,bwd}_*.hip.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "ltv_scan_launch.hpp"

namespace ltv {

// dbias[h, j] = sum over (b, c) of partial[b, h, c, j]: one workgroup per
// output, thread i summing the pairs i, i + 256, ... in order, then a fixed
// tree over the threads (deterministic).  Workgroups from H Da on form the
// inits gradient's batch sum (DinitSum), one thread per (h, d), in batch
// order; after them, nbp workgroups zero the padding slots (PadZero), one
// thread per (b, t) row.
__global__ void __launch_bounds__(256) dbias_reduce_kernel(const float* __restrict__ partial,
                                                           float* __restrict__ dbias, int B,
                                                           int H, int NC, int Da, DinitSum ds,
                                                           int nbd, PadZero pz) {
  if ((int)blockIdx.x >= H * Da + nbd) {
    const int64_t row = ((int64_t)blockIdx.x - H * Da - nbd) * 256 + threadIdx.x;
    if (row < (int64_t)pz.B * pz.T) {
      const int64_t b = row / pz.T, t = row - b * pz.T;
      char* p = pz.base + (b * pz.sb + t * pz.st + (int64_t)pz.q0 * pz.sq) * pz.esize;
      for (int q = 0; q < pz.pad; ++q) {
        char* e = p + (int64_t)q * pz.sq * pz.esize;
        if (pz.esize == 2)
          *reinterpret_cast<unsigned short*>(e) = 0;
        else
          *reinterpret_cast<float*>(e) = 0.0f;
      }
    }
    return;
  }
  if ((int)blockIdx.x >= H * Da) {
    const int i = ((int)blockIdx.x - H * Da) * 256 + (int)threadIdx.x;
    if (i < H * ds.D) {
      const int h = i / ds.D, d = i - h * ds.D;
      // groups of 16 loads in flight, added in batch order (a plain loop waits
      // for each load in turn: 9.6 us instead of 4.4 at d12)
      const float* src = ds.ws + (int64_t)h * ds.D + d;
      const int64_t bs = (int64_t)H * ds.D;
      float acc = 0.0f;
      int b = 0;
      for (; b + 16 <= B; b += 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = src[(int64_t)(b + k) * bs];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc += v[k];
      }
      for (; b < B; ++b) acc += src[(int64_t)b * bs];
      const int64_t o = (int64_t)h * ds.sh + (int64_t)d * ds.sd;
      if (ds.out_bf16)
        reinterpret_cast<bf16_t*>(ds.out)[o] = (bf16_t)(cvt_pk_bf16(acc, 0.0f) & 0xffffu);
      else
        reinterpret_cast<float*>(ds.out)[o] = acc;
    }
    return;
  }
  __shared__ float red[256];
  const int i = blockIdx.x;  // h * Da + j
  const int h = i / Da, j = i - h * Da;
  const int n = B * NC;
  float acc = 0.0f;
  for (int k = threadIdx.x; k < n; k += 256) {
    const int b = k / NC, c = k - b * NC;
    acc += partial[(((int64_t)b * H + h) * NC + c) * Da + j];
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) dbias[i] = red[0];
}

// Zeroes a (B, H, D) view of any strides in the I/O dtype (esize bytes per
// element) and, from the first workgroup, n0 floats at f0.  A kernel rather
// than a memset so that the calls stay valid inside a captured HIP graph.
__global__ void __launch_bounds__(256) zero_bhd_kernel(char* __restrict__ p, View4 v, int B, int H,
                                                       int D, int esize, float* __restrict__ f0,
                                                       int n0) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.x == 0)
    for (int k = threadIdx.x; k < n0; k += 256) f0[k] = 0.0f;
  if (i >= (int64_t)B * H * D) return;
  const int d = (int)(i % D);
  const int64_t bh = i / D;
  const int h = (int)(bh % H), b = (int)(bh / H);
  char* q = p + (b * v.s[0] + h * v.s[1] + d * v.s[3]) * esize;
  if (esize == 2)
    *reinterpret_cast<uint16_t*>(q) = 0;
  else
    *reinterpret_cast<float*>(q) = 0.0f;
}

int scan_launch_fwd(bool bf16, const FwdArgs& a, ScanCfg cfg, int grid, bool vec, int gm,
                    hipStream_t st) {
  return bf16 ? scan_fwd_launch_bf16(a, cfg, grid, vec, gm, st)
              : scan_fwd_launch_f32(a, cfg, grid, vec, gm, st);
}

int scan_launch_fwd_chain(bool bf16, const FwdArgs& a, const ChainArgs& ch, ScanCfg cfg, int gm,
                          hipStream_t st) {
  return bf16 ? scan_fwd_chain_launch_bf16(a, ch, cfg, gm, st)
              : scan_fwd_chain_launch_f32(a, ch, cfg, gm, st);
}

int scan_launch_bwd(bool bf16, const BwdArgs& a, ScanCfg cfg, int grid, bool vec, int gm,
                    bool lb, hipStream_t st) {
  return bf16 ? scan_bwd_launch_bf16(a, cfg, grid, vec, gm, lb, st)
              : scan_bwd_launch_f32(a, cfg, grid, vec, gm, lb, st);
}

int scan_launch_bwd_chain(bool bf16, const BwdArgs& a, ScanCfg cfg, int grid, int gm,
                          hipStream_t st) {
  return bf16 ? scan_bwd_chain_launch_bf16(a, cfg, grid, gm, st)
              : scan_bwd_chain_launch_f32(a, cfg, grid, gm, st);
}

int scan_launch_lb_fold(bool bf16, const BwdArgs& a, hipStream_t st) {
  const ScanShape& S = a.sh;
  const int64_t n = (int64_t)S.B * S.H * a.nchunk * a.kw * (S.D + S.Da);
  const int64_t blocks = (n + 255) / 256;
  LTV_REQUIRE(blocks < (1ll << 31), LTV_ERR_UNSUPPORTED, "look-back warm-up too large");
  if (bf16)
    hipLaunchKernelGGL(scan_lb_fold_kernel<bf16_t>, dim3((int)blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(scan_lb_fold_kernel<float>, dim3((int)blocks), dim3(256), 0, st, a);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

int scan_launch_lb_dinit(bool bf16, const BwdArgs& a, hipStream_t st) {
  const ScanShape& S = a.sh;
  const int64_t n = (int64_t)S.B * S.H * S.D;
  const int blocks = (int)((n + 255) / 256);
  if (bf16)
    hipLaunchKernelGGL(scan_lb_dinit_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(scan_lb_dinit_kernel<float>, dim3(blocks), dim3(256), 0, st, a);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
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
                       st, a, dalpha, nullptr);
  } else {
    hipLaunchKernelGGL(scan_bwd_channel_kernel<float>, dim3(blocks), dim3(threads), 0, st, a,
                       dalpha);
    LTV_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_bwd_group_reduce_kernel<float>, dim3(gblocks), dim3(threads), 0, st,
                       a, dalpha, nullptr);
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

int scan_launch_lb_channel(bool bf16, const BwdArgs& a, float* dalpha, float* du_ws,
                           hipStream_t st) {
  const ScanShape& S = a.sh;
  const int64_t n = (int64_t)S.B * S.H * S.D;
  const int threads = 256;
  const int blocks = (int)((n + threads - 1) / threads);
  const int64_t ng = (int64_t)S.B * S.H * S.Da;
  const int gblocks = (int)((ng + threads - 1) / threads);
  if (bf16) {
    hipLaunchKernelGGL(scan_lb_channel_kernel<bf16_t>, dim3(blocks), dim3(threads), 0, st, a,
                       dalpha, du_ws);
    LTV_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_bwd_group_reduce_kernel<bf16_t>, dim3(gblocks), dim3(threads), 0,
                       st, a, dalpha, du_ws);
  } else {
    hipLaunchKernelGGL(scan_lb_channel_kernel<float>, dim3(blocks), dim3(threads), 0, st, a,
                       dalpha, du_ws);
    LTV_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_bwd_group_reduce_kernel<float>, dim3(gblocks), dim3(threads), 0, st,
                       a, dalpha, du_ws);
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

// carry[bh, k, c] = g entering chunk k from its end: the maps of the
// sub-chunks after chunk k applied to 0, last to first.  One thread per
// (b h, channel); the maps are read in batches so the walk is not one load
// latency per sub-chunk.
__global__ void __launch_bounds__(256) scan_bwd_carry_kernel(const BwdArgs args) {
  const ScanShape& S = args.sh;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * S.D) return;
  const int c = (int)(idx % S.D);
  const int64_t bh = idx / S.D;
  const int64_t plane = (int64_t)S.B * S.H * args.nfine * S.D;
  const int fpc = args.chunk_steps / args.fine_steps;  // sub-chunks per chunk
  const float* ap = args.agg + bh * args.nfine * S.D + c;
  float* cp = args.carry + bh * args.nchunk * S.D + c;
  cp[(int64_t)(args.nchunk - 1) * S.D] = 0.0f;
  float g = 0.0f;
  constexpr int KB = 16;
  for (int fb = args.nfine; fb > 0; fb -= KB) {
    float A[KB], G[KB];
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      const int f = fb - 1 - q;
      A[q] = f >= 0 ? ap[(int64_t)f * S.D] : 1.0f;
      G[q] = f >= 0 ? ap[plane + (int64_t)f * S.D] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      const int f = fb - 1 - q;
      if (f >= 0) {
        // f is the last sub-chunk of chunk k = f / fpc: g is that chunk's carry
        const int k = f / fpc;
        if ((f + 1) % fpc == 0 && k < args.nchunk - 1) cp[(int64_t)k * S.D] = g;
        g = fmaf(A[q], g, G[q]);
      }
    }
  }
}

// The per-chunk maps of the reverse recurrence, then each chunk's carry.
int scan_launch_bwd_chunk_maps(bool bf16, const BwdArgs& a, bool vec, hipStream_t st) {
  const ScanShape& S = a.sh;
  const int V = bf16 ? 8 : 4;
  const int64_t n = (int64_t)S.B * S.H * a.nfine * ((S.D + V - 1) / V);
  const int blocks = (int)((n + 255) / 256);
  if (bf16) {
    if (vec)
      hipLaunchKernelGGL((scan_bwd_agg_kernel<bf16_t, true>), dim3(blocks), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((scan_bwd_agg_kernel<bf16_t, false>), dim3(blocks), dim3(256), 0, st, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((scan_bwd_agg_kernel<float, true>), dim3(blocks), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((scan_bwd_agg_kernel<float, false>), dim3(blocks), dim3(256), 0, st, a);
  }
  LTV_LAUNCH_CHECK();
  const int64_t nc = (int64_t)S.B * S.H * S.D;
  hipLaunchKernelGGL(scan_bwd_carry_kernel, dim3((int)((nc + 255) / 256)), dim3(256), 0, st, a);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

int scan_launch_dbias_reduce(const float* partial, float* dbias, int B, int H, int NC, int Da,
                             hipStream_t st, const DinitSum& ds, const PadZero& pz) {
  const int nbd = ds.ws != nullptr ? (H * ds.D + 255) / 256 : 0;
  const int64_t nbp =
      pz.base != nullptr && pz.pad > 0 ? ((int64_t)pz.B * pz.T + 255) / 256 : 0;
  LTV_REQUIRE(H * Da + nbd + nbp < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL(dbias_reduce_kernel, dim3((unsigned)(H * Da + nbd + nbp)), dim3(256), 0, st,
                     partial, dbias, B, H, NC, Da, ds, nbd, pz);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

namespace {

struct HostView4 {
  const void* p;
  int64_t s[4];
};

inline View4 to_dev(const HostView4& v) {
  View4 o;
  o.p = v.p;
  for (int i = 0; i < 4; ++i) o.s[i] = v.s[i];
  return o;
}

// A view can be read/written as 16-byte vectors along the channel axis.
inline bool vec_ok(const void* p, const int64_t* s, int nd_outer, int V) {
  if (!aligned16(p)) return false;
  if (s[nd_outer] != 1) return false;
  for (int i = 0; i < nd_outer; ++i)
    if (s[i] % V != 0) return false;
  return true;
}

// Launch-shape overrides, read once: LTV_SCAN_FWD_CFG="CL,L,NW" (CL = channel
// lanes per wavefront, L = steps per lane, NW = wavefronts per workgroup) and
// LTV_SCAN_BWD_CFG="L,NW" (the backward always spans the whole head).
struct ScanTuning {
  int fwd_cl = 0, fwd_l = 0, fwd_nw = 0;
  // LTV_SCAN_CHAIN_CFG="CL,L,NW" (chained forward shape) or "0" (tile kernel only)
  int chain_cl = 0, chain_l = 0, chain_nw = 0;
  bool chain = true;
  int bwd_l = 0, bwd_nw = 0;
  int bwd_chunks = 0;  // time chunks per (b, h) in the backward; 0 = automatic
  // LTV_SCAN_BWD_CHAIN_CFG="L,NW" (chained backward shape, forced) or "0"
  // (never chained)
  int bwd_chain_l = 0, bwd_chain_nw = 0;
  bool bwd_chain = true;
  bool lb_short = true;  // LTV_SCAN_LB_SHORT=0: look-back windows through the tile kernels
  // LTV_SCAN_LB_WPL=n: windows per lane of the short-window backward (0 = automatic)
  int lb_wpl = 0;
  ScanTuning() {
    if (const char* e = getenv("LTV_SCAN_LB_SHORT")) lb_short = atoi(e) != 0;
    if (const char* e = getenv("LTV_SCAN_LB_WPL")) lb_wpl = atoi(e) > 0 ? atoi(e) : 0;
    if (const char* e = getenv("LTV_SCAN_BWD_CHUNKS")) bwd_chunks = atoi(e) > 0 ? atoi(e) : 0;
    if (const char* e = getenv("LTV_SCAN_FWD_CFG")) {
      if (sscanf(e, "%d,%d,%d", &fwd_cl, &fwd_l, &fwd_nw) != 3) fwd_cl = fwd_l = fwd_nw = 0;
    }
    if (const char* e = getenv("LTV_SCAN_CHAIN_CFG")) {
      if (sscanf(e, "%d,%d,%d", &chain_cl, &chain_l, &chain_nw) != 3) {
        chain_cl = chain_l = chain_nw = 0;
        chain = atoi(e) != 0;
      }
    }
    if (const char* e = getenv("LTV_SCAN_BWD_CFG")) {
      if (sscanf(e, "%d,%d", &bwd_l, &bwd_nw) != 2) bwd_l = bwd_nw = 0;
    }
    if (const char* e = getenv("LTV_SCAN_BWD_CHAIN_CFG")) {
      if (sscanf(e, "%d,%d", &bwd_chain_l, &bwd_chain_nw) != 2) {
        bwd_chain_l = bwd_chain_nw = 0;
        bwd_chain = atoi(e) != 0;
      }
    }
  }
};

const ScanTuning& tuning() {
  static const ScanTuning t;
  return t;
}

// ltv_lb_set_windows_per_lane: 0 = LTV_SCAN_LB_WPL or automatic
std::atomic<int> g_lb_wpl{0};

// Compute units of the current device (cached per device).
int scan_cu_count() {
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

int check_shape(int dtype, int B, int T, int NH, int NKVH, int Da, int r) {
  LTV_REQUIRE(dtype == LTV_DTYPE_F32 || dtype == LTV_DTYPE_BF16, LTV_ERR_INVALID_ARG,
              "dtype must be LTV_DTYPE_F32 or LTV_DTYPE_BF16, got %d", dtype);
  LTV_REQUIRE(B >= 0 && T >= 0 && NH >= 0 && NKVH >= 0, LTV_ERR_INVALID_ARG,
              "negative size (B=%d T=%d NH=%d NKVH=%d)", B, T, NH, NKVH);
  LTV_REQUIRE(Da >= 1 && r >= 1, LTV_ERR_INVALID_ARG, "Da and r must be >= 1 (Da=%d r=%d)", Da,
              r);
  const int V = dtype == LTV_DTYPE_BF16 ? 8 : 4;
  const int D = Da * r;
  LTV_REQUIRE(D <= 64 * V, LTV_ERR_UNSUPPORTED,
              "head_dim D=%d exceeds the supported maximum %d for this dtype", D, 64 * V);
  return LTV_OK;
}

// The main backward kernel reduces dalpha over gate groups that fill whole
// lanes (r % V == 0, at most kMaxLaneGroups groups per head) or that fit in one
// lane (V % r == 0); anything else goes to the per-channel kernel.
inline int bwd_gate_mode(int r, int Da, int V) {
  if (r % V == 0) return Da <= kMaxLaneGroups ? GATE_LANE : -1;
  if (V % r == 0) return GATE_CHAN;
  return -1;
}

// r == 1 with channel-contiguous, 16-byte addressable logits: vector gate loads.
inline bool chanvec_ok(int r, int D, int V, const HostView4& lg) {
  return r == 1 && D % V == 0 && vec_ok(lg.p, lg.s, 3, V);
}

// The short-window look-back kernels (one lane per window, ltv_scan_lb.hip)
// take chunks of at most 64 steps, a warm-up no longer than 16 steps nor than
// a chunk (so a step is read by at most its own and the next window), and gate
// groups the reverse pass reduces: r | V inside a lane, or r / V lanes a power
// of two.
inline bool lb_short_ok(int V, int r, int Q, int K) {
  if (Q > 64 || K - 1 > 16 || K - 1 > Q) return false;
  if (r % V == 0) return is_pow2(r / V);
  return V % r == 0;
}

// The tile kernels address a view through 32-bit byte offsets from its (b, h)
// slice at the tile's first step (or the step before): at most
// kTileRowsMax time steps plus the channel extent.  Every such offset stays
// below 2^31 when this holds.
constexpr int64_t kTileRowsMax = 1024 + 2;  // the largest built tile, the step before, one spare
// The offsets are unsigned: time and channel strides must be non-negative.
inline bool tile_offsets_fit(const int64_t* s, int64_t chan_extent, int esize) {
  return s[2] >= 0 && s[3] >= 0 &&
         (kTileRowsMax * s[2] + chan_extent * s[3]) * esize + 64 < (1ll << 31);
}

int check_tile_offsets(const char* what, const int64_t* s, int64_t chan_extent, int esize) {
  LTV_REQUIRE(tile_offsets_fit(s, chan_extent, esize), LTV_ERR_UNSUPPORTED,
              "%s: time stride %lld / channel stride %lld negative or too large for the scan's "
              "32-bit tile offsets", what, (long long)s[2], (long long)s[3]);
  return LTV_OK;
}

// Backward launch shape for a head of cl channel lanes: 4 steps per lane and 4
// wavefronts, except at 16 vector lanes (D = 128 in bf16, the d12 heads) where
// 2 wavefronts are measured fastest on MI355X (134 us at d12 against 143 us
// for 2 steps per lane x 4 wavefronts and 145 us for 2 x 2): a tile spans 32
// steps either way, and fewer wavefronts shorten the per-tile composition of
// the wavefront carries while 4 steps per lane amortise the lane scan levels.
inline ScanCfg bwd_default_cfg(int cl, bool vec) {
  return vec && cl == 16 ? ScanCfg{16, 4, 2} : ScanCfg{cl, 4, 4};
}
// The whole-head tile backward at 16 vector lanes: 2 wavefronts per workgroup
// where that keeps the grid to one round of resident workgroups (four per CU
// at two wavefronts per SIMD) and 4 wavefronts would need two; 4 otherwise.
// Measured on MI355X (heads of 128, bf16, T = 1024; sequences = B H): B = 16
// (288 sequences) 85.3 -> 75.1 us with 4 wavefronts, B = 32 (576) 113.8 ->
// 117.5 us, B = 48 (864) 151.3 -> 153.4 us, B = 64 (1152) 232.7 -> 214.1 us.
inline ScanCfg bwd_tile_cfg(int cl, bool vec, int64_t nseq) {
  ScanCfg c = bwd_default_cfg(cl, vec);
  const int64_t slots = (int64_t)scan_cu_count() * 2;  // 4-wavefront workgroups per round
  if (c.CL == 16 && c.NW == 2 && (nseq <= slots || nseq > 2 * slots)) c.NW = 4;
  return c;
}

// Bytes from a view's first to its last element, (B, NX, T, X) elements
// (non-negative strides, checked by check_tile_offsets).
inline int64_t view_span_bytes(const int64_t* s, int B, int NX, int T, int X, int esize) {
  auto ext = [](int n, int64_t st) { return n > 0 ? (int64_t)(n - 1) * st : 0; };
  return (ext(B, s[0]) + ext(NX, s[1]) + ext(T, s[2]) + ext(X, s[3]) + 1) * esize;
}
constexpr int64_t kBufSpanMax = (1ll << 31) - 64;

int check_pqk(int P, int Q, int K) {
  LTV_REQUIRE(P >= 0 && Q >= 1 && K >= 1, LTV_ERR_INVALID_ARG,
              "chunking needs P >= 0, Q >= 1, K >= 1 (P=%d Q=%d K=%d)", P, Q, K);
  return LTV_OK;
}

// The chained forward (scan_fwd_chain_kernel): its launch shape for a head of
// D channels with gate groups of r, or CL = 0 where it is not used.  It needs
// the full recurrence, 16-byte channel vectors and one gate per lane or r == 1,
// and it is chosen where the tile kernel would run fewer than 1,024
// workgroups and each sequence spans at least 8 chunks (long T at small
// batch).  Measured on MI355X:
//   configs[4] prefill (B = 8, T = 8192, 288 sequences): tile 172 us, chained
//     (8, 8, 8) 127 us, (8, 16, 4) 128 us, (8, 8, 4) 145 us, (8, 4, 8) 135 us;
//   d12 (1,152 sequences, T = 1024): tile 62.6 us, chained (8, 8, 8) 66.6 us,
//     (8, 16, 4) 70.4 us -- with every sequence's workgroup resident the tile
//     kernel streams without per-chunk start-up;
//   configs[1] (r = 1, 1,152 sequences): tile 99.6 us, chained (8, 8, 4)
//     96.5 us, (8, 4, 4) 128 us.
// Chunks shorter than 256 steps lose to the per-workgroup start-up (ticket,
// two barriers, the hand-off): (8, 4, 4) 124 us, (8, 2, 4) 222 us at d12.
// Few chunks per sequence do not repay it either: tile against chained (8, 8, 8)
// at T = 1024 (2 chunks): B = 4 / 8 / 16 18.5 / 23.3 / 32.9 against 22.8 /
// 26.2 / 39.4 us; T = 2048 (4): B = 8 / 16 37.9 / 70.0 against 39.4 / 70.9 us;
// T = 4096 (8): B = 2 / 4 / 16 49.0 / 48.6 / 146.9 against 27.8 / 40.7 /
// 126.6 us; so the automatic choice also needs kFwdChainMinChunks chunks.
// LTV_SCAN_CHAIN_CFG="CL,L,NW" forces the chained kernel with that shape.
struct ChainPlan {
  ScanCfg cfg;
  int gm, nslab, nchunk;
  int64_t nseq;
  size_t bytes;  // workspace: header + tagged states
};
constexpr size_t kChainHeader = 256;
constexpr int kFwdChainMinChunks = 8;

// Error mailbox of the chained kernels: one mapped, pinned host word that a
// failing launch stores its code into (ChainCtl::host_err), read and cleared
// by ltv_chain_take_error without synchronising the device.  Allocated once,
// on the first chained launch made outside stream capture (an allocation
// during capture could invalidate the capture; such launches report into the
// workspace header only); if the allocation fails the kernels report into the
// workspace header only.
struct ChainHost {
  std::mutex mu;
  bool tried = false;
  uint32_t* host = nullptr;  // host view
  uint32_t* dev = nullptr;   // device view
  int spin_max = kChainSpinMax;
  int no_publish = 0;
};
ChainHost& chain_host() {
  static ChainHost h;
  return h;
}

ChainCtl chain_ctl(hipStream_t st) {
  ChainHost& h = chain_host();
  std::lock_guard<std::mutex> lk(h.mu);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (!h.tried && (hipStreamIsCapturing(st, &cs) != hipSuccess ||
                   cs != hipStreamCaptureStatusNone)) {
    (void)hipGetLastError();
    return ChainCtl{nullptr, h.spin_max, h.no_publish};
  }
  if (!h.tried) {
    h.tried = true;
    void* p = nullptr;
    if (hipHostMalloc(&p, 256, hipHostMallocMapped | hipHostMallocPortable |
                                   hipHostMallocCoherent) == hipSuccess) {
      void* d = nullptr;
      if (hipHostGetDevicePointer(&d, p, 0) == hipSuccess && d != nullptr) {
        h.host = static_cast<uint32_t*>(p);
        h.dev = static_cast<uint32_t*>(d);
        __atomic_store_n(h.host, 0u, __ATOMIC_SEQ_CST);
      } else {
        (void)hipHostFree(p);
      }
    }
    (void)hipGetLastError();  // a failed allocation is not the caller's error
  }
  return ChainCtl{h.dev, h.spin_max, h.no_publish};
}
// (b, h) sequences from which the backward keeps the tile kernel (which runs
// unchunked from 256 sequences on).  Measured on MI355X (heads of 128,
// r = 128, bf16; chained shape L = 4, NW = 4), tile against chained:
//   B = 32, T = 1024 (576 sequences): 112 against 171 us (L = 4, NW = 2:
//     242 us) -- 16 chunks per sequence and about two chunk rows resident
//     make the chain's critical path the time;
//   B = 16 (288): T = 1024 84 against 89 us, T = 2048 160 against 156 us;
//   below 256, where the tile kernel needs the chunk-map passes: B = 8 / 4,
//     T = 1024 (144 / 72) 90 / 72 against 54 / 36 us; B = 8, T = 4096 222
//     against 157 us; T = 8192: B = 8 / 4 / 2 / 1 (configs[4]'s shape is
//     B = 8) 400 / 232 / 139 / 108 against 298 / 166 / 120 / 103 us.
constexpr int64_t kBwdChainMaxSeqs = 256;

ChainPlan chain_plan(int dtype, int B, int T, int H, int Da, int r) {
  ChainPlan p{{0, 0, 0}, -1, 0, 0, 0, 0};
  const ScanTuning& tu = tuning();
  const int V = dtype == LTV_DTYPE_BF16 ? 8 : 4;
  const int D = Da * r;
  if (!tu.chain || B <= 0 || T <= 0 || H <= 0 || D % V != 0) return p;
  int gm = -1;
  if (r % V == 0) gm = GATE_LANE;
  else if (r == 1) gm = GATE_CHANVEC;
  else return p;
  ScanCfg c{8, 8, 8};
  if (gm == GATE_CHANVEC) c = ScanCfg{8, 8, 4};
  if (tu.chain_cl > 0) {
    c = ScanCfg{tu.chain_cl, tu.chain_l, tu.chain_nw};
  } else {
    // the tile kernel's workgroups: slabs of up to 8 channel lanes
    const int cl_full = next_pow2(D / V);
    const int fcl = cl_full < 8 ? cl_full : 8;
    const int64_t tile_wgs = (int64_t)B * H * ((D + fcl * V - 1) / (fcl * V));
    if (tile_wgs >= 1024) return p;
  }
  if (c.CL * V > 64 || c.CL < 1 || c.L < 1 || c.NW < 1) return p;
  const int TW = c.NW * (64 / c.CL) * c.L;
  const int nchunk = (int)(((int64_t)T + TW - 1) / TW);
  // (and only for sequences of at least kFwdChainMinChunks chunks)
  if (tu.chain_cl == 0 && nchunk < kFwdChainMinChunks) return p;
  p.cfg = c;
  p.gm = gm;
  p.nslab = (D + c.CL * V - 1) / (c.CL * V);
  p.nchunk = nchunk;
  p.nseq = (int64_t)B * H * p.nslab;
  p.bytes = kChainHeader + (size_t)p.nseq * (size_t)(p.nchunk - 1) * (size_t)(c.CL * V) * 8u;
  return p;
}

// Forward launch over B * H * nwin windows x channel slabs (a.P/Q/K/nwin, and
// a.wst / a.kw for the warm-up mode, already set): gate mode and launch shape.
int launch_forward(int dtype, FwdArgs& a, bool vec, const HostView4& lg, int B, int T, int NH,
                   int NKVH, int Da, int r, int use_sigmoid, hipStream_t st) {
  const int H = NH + 2 * NKVH;
  const int D = Da * r;
  const int V = dtype == LTV_DTYPE_BF16 ? 8 : 4;
  const int cl_full = next_pow2((D + V - 1) / V);
  int gm = GATE_CHAN;
  if (r % V == 0) gm = GATE_LANE;
  else if (vec && chanvec_ok(r, D, V, lg)) gm = GATE_CHANVEC;

  // Channels are independent in the forward: slabs of up to 8 channel lanes
  // (64 bf16 / 32 fp32 channels), 4 wavefronts, 2 steps per lane at 8 lanes.
  // Measured on MI355X at d12 this is the fastest built shape (74 us against
  // 89 us with 4 steps per lane): 81 VGPRs let all 1152 workgroups be resident
  // at once (111 VGPRs left 128 of them for a second round), and each load
  // instruction covers 8 rows of 128 bytes.
  // With fewer workgroups than fill the chip once (long T at small batch:
  // B = 8, T = 8192 at d12 heads gives 288), each one is latency-bound and 4
  // steps per lane put twice the bytes in flight: 174 against 190 us there.
  // (Cutting T into chunks entered from composed chunk maps measured no
  // better, 199 us: the maps cost a second read of all but the last chunk.)
  const int fcl = cl_full < 8 ? cl_full : 8;
  const int nslab0 = (D + fcl * V - 1) / (fcl * V);
  const bool few = (int64_t)B * H * a.nwin * nslab0 < 1024;
  ScanCfg cfg{fcl, fcl == 8 && vec && !few ? 2 : 4, 4};
  const ScanTuning& tu = tuning();
  if (vec && tu.fwd_cl > 0) cfg = ScanCfg{tu.fwd_cl < cl_full ? tu.fwd_cl : cl_full, tu.fwd_l, tu.fwd_nw};
  const int nslab = (D + cfg.CL * V - 1) / (cfg.CL * V);
  a.sh = ScanShape{B, T, NH, NKVH, Da, r, D, H, nslab, use_sigmoid};
  const int64_t grid = (int64_t)B * H * a.nwin * nslab;
  LTV_REQUIRE(grid < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
  return scan_launch_fwd(dtype == LTV_DTYPE_BF16, a, cfg, (int)grid, vec, gm, st);
}

// The inits' dtype: the values' own, or fp32 with bf16 values (the parameter
// the reference casts to bf16 before its kernel; rounded to bf16 when read).
int check_inits_dtype(int dtype, int inits_dtype) {
  LTV_REQUIRE(inits_dtype == dtype || (inits_dtype == LTV_DTYPE_F32 && dtype == LTV_DTYPE_BF16),
              LTV_ERR_INVALID_ARG,
              "inits dtype %d: must be the values' dtype (%d), or fp32 with bf16 values",
              inits_dtype, dtype);
  return LTV_OK;
}

int scan_forward_impl(int dtype, const HostView4& u, const HostView4& lg, const HostView4& init,
                      int inits_dtype, const float* bias, void* const outp[3],
                      const int64_t* const outs[3], int B, int T, int NH, int NKVH, int Da, int r,
                      int P, int Q, int K, int use_sigmoid, void* chain_ws,
                      size_t chain_ws_bytes, hipStream_t st) {
  int rc = check_shape(dtype, B, T, NH, NKVH, Da, r);
  if (rc) return rc;
  rc = check_pqk(P, Q, K);
  if (rc) return rc;
  rc = check_inits_dtype(dtype, inits_dtype);
  if (rc) return rc;
  const bool init_f32 = inits_dtype != dtype;
  const int H = NH + 2 * NKVH;
  const int D = Da * r;
  if (B == 0 || T == 0 || H == 0) return LTV_OK;
  LTV_REQUIRE(bias != nullptr && u.p && lg.p && init.p, LTV_ERR_INVALID_ARG,
              "null tensor pointer");
  const int V = dtype == LTV_DTYPE_BF16 ? 8 : 4;

  FwdArgs a;
  a.u = to_dev(u);
  a.lg = to_dev(lg);
  a.init = to_dev(init);
  a.init_f32 = init_f32 ? 1 : 0;
  a.bias = bias;
  a.P = P;
  a.Q = Q;
  a.K = K;
  a.nwin = look_back_nwin(T, P, Q);
  a.wst = nullptr;
  a.kw = 0;
  LTV_REQUIRE(!init_f32 || a.nwin == 1 || (tuning().lb_short && lb_short_ok(V, r, Q, K)),
              LTV_ERR_UNSUPPORTED,
              "fp32 inits with bf16 values need the full recurrence (P >= T) or look-back "
              "windows the short-window kernels take");
  const int E = dtype == LTV_DTYPE_BF16 ? 2 : 4;
  if ((rc = check_tile_offsets("values", u.s, D, E)) || (rc = check_tile_offsets("logits", lg.s, D, E)) ||
      (rc = check_tile_offsets("inits", init.s, D, init_f32 ? 4 : E)))
    return rc;
  bool vec = (D % V == 0) && vec_ok(u.p, u.s, 3, V) && vec_ok(init.p, init.s, 3, V);
  for (int i = 0; i < 3; ++i) {
    a.out.p[i] = outp[i];
    for (int k = 0; k < 4; ++k) a.out.s[i][k] = outs[i][k];
    const int nh = i == 0 ? NH : NKVH;
    if (nh > 0) {
      LTV_REQUIRE(outp[i] != nullptr, LTV_ERR_INVALID_ARG, "null output pointer");
      if ((rc = check_tile_offsets("outputs", outs[i], D, E))) return rc;
      vec = vec && vec_ok(outp[i], outs[i], 3, V);
    }
  }
  if (a.nwin > 1 && (tuning().lb_short && lb_short_ok(V, r, Q, K))) {
    a.sh = ScanShape{B, T, NH, NKVH, Da, r, D, H, 1, use_sigmoid};
    a.lanes = next_pow2((D + V - 1) / V);
    int gm = GATE_CHAN;
    if (r % V == 0) gm = GATE_LANE;
    else if (vec && chanvec_ok(r, D, V, lg)) gm = GATE_CHANVEC;
    // the buffer-addressed kernels take 32-bit offsets within each view's
    // (b, h) slice
    bool buf = view_span_bytes(u.s, 1, 1, T, D, E) <= kBufSpanMax &&
               view_span_bytes(lg.s, 1, 1, T, std::max(D, Da), E) <= kBufSpanMax;
    for (int i = 0; i < 3; ++i)
      if ((i == 0 ? NH : NKVH) > 0)
        buf = buf && view_span_bytes(outs[i], 1, 1, T, D, E) <= kBufSpanMax;
    LTV_REQUIRE(!init_f32 || buf, LTV_ERR_UNSUPPORTED,
                "fp32 inits with look-back windows need views whose (b, h) slices span less "
                "than 2 GiB");
    return scan_launch_lb_short_fwd(dtype == LTV_DTYPE_BF16, a, vec, gm, buf, st);
  }
  if (a.nwin == 1 && chain_ws != nullptr) {
    const ChainPlan pl = chain_plan(dtype, B, T, H, Da, r);
    const bool lg_ok = pl.gm == GATE_LANE || (pl.gm == GATE_CHANVEC && chanvec_ok(r, D, V, lg));
    if (pl.cfg.CL > 0 && vec && lg_ok) {
      LTV_REQUIRE(chain_ws_bytes >= pl.bytes, LTV_ERR_WORKSPACE,
                  "chained scan workspace too small: %zu bytes, need %zu", chain_ws_bytes,
                  pl.bytes);
      LTV_REQUIRE((reinterpret_cast<uintptr_t>(chain_ws) & 255u) == 0, LTV_ERR_INVALID_ARG,
                  "chained scan workspace must be 256-byte aligned");
      a.sh = ScanShape{B, T, NH, NKVH, Da, r, D, H, pl.nslab, use_sigmoid};
      ChainArgs ch;
      ch.ticket = reinterpret_cast<uint32_t*>(chain_ws);
      ch.err = reinterpret_cast<uint32_t*>(chain_ws) + 1;
      ch.words = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(chain_ws) +
                                                       kChainHeader);
      LTV_REQUIRE(pl.nseq * pl.nchunk < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
      ch.nseq = (int)pl.nseq;
      ch.nchunk = pl.nchunk;
      ch.ctl = chain_ctl(st);
      return scan_launch_fwd_chain(dtype == LTV_DTYPE_BF16, a, ch, pl.cfg, pl.gm, st);
    }
  }
  return launch_forward(dtype, a, vec, lg, B, T, NH, NKVH, Da, r, use_sigmoid, st);
}

// Upper bound on the backward's time chunks per (b, h).  With at least 256
// (b, h) sequences (one per CU on MI355X) chunking only adds the chunk-map
// passes (measured: 288 sequences, 1 chunk 132 us, 2-4 chunks 150 us); with
// fewer (long T, small batch) the sequences are cut into chunks of at least
// one 64-step tile until about 512 workgroups run (144 sequences at T = 8192:
// 827 us unchunked, 504 us in 4 chunks).  The
// launch rounds the chunk length up to whole tiles, which never raises the
// count above this bound.
int bwd_max_chunks(int B, int H, int T) {
  const int64_t bh = (int64_t)B * H;
  int nc = tuning().bwd_chunks;
  if (nc == 0) nc = bh >= 256 ? 1 : (int)((512 + bh - 1) / bh);
  const int cap = (T + 63) / 64;
  return std::max(1, std::min(nc, cap));
}

// Sub-chunk length of the backward's chunk maps (steps).
constexpr int kBwdFineSteps = 64;

// The chained backward (scan_bwd_kernel in its CHAIN mode): launch shape,
// gate mode and chunk count for a head of D channels, or CL = 0 where it is
// not used.  It needs the full recurrence, 16-byte channel vectors, one gate
// per lane group or r == 1, and a built shape; it is chosen below
// kBwdChainMaxSeqs sequences, where the tile kernel's workgroups are too few
// to hide its per-tile latency and it needs the chunk-map passes.  LTV_SCAN_BWD_CHAIN_CFG="L,NW" forces it with that shape.
struct BwdChainPlan {
  ScanCfg cfg;
  int gm, nchunk;
  int64_t nseq;
  size_t bytes;  // workspace: header + tagged carries
};

bool bwd_chain_built(ScanCfg c, int V) {
  bool built = false;
#define LTV_X(CL_, L_, NW_) \
  built = built || (c.CL == CL_ && c.L == L_ && c.NW == NW_ && CL_ * V <= NW_ * 64);
  LTV_SCAN_BWD_CHAIN_CONFIGS(LTV_X)
#undef LTV_X
  return built;
}

BwdChainPlan bwd_chain_plan(int dtype, int B, int T, int H, int Da, int r) {
  BwdChainPlan p{{0, 0, 0}, -1, 0, 0, 0};
  const ScanTuning& tu = tuning();
  const int V = dtype == LTV_DTYPE_BF16 ? 8 : 4;
  const int D = Da * r;
  if (!tu.bwd_chain || B <= 0 || T <= 0 || H <= 0 || D % V != 0) return p;
  int gm = bwd_gate_mode(r, Da, V);
  if (gm == GATE_CHAN) gm = r == 1 ? GATE_CHANVEC : -1;
  if (gm < 0) return p;
  const int cl = next_pow2(D / V);
  ScanCfg c{cl, 4, 4};
  if (tu.bwd_chain_l > 0) {
    c = ScanCfg{cl, tu.bwd_chain_l, tu.bwd_chain_nw};
  } else {
    if ((int64_t)B * H >= kBwdChainMaxSeqs) return p;
  }
  if (!bwd_chain_built(c, V)) return p;
  const int TW = c.NW * (64 / c.CL) * c.L;
  p.nchunk = (int)(((int64_t)T + TW - 1) / TW);
  if (p.nchunk < 2) return BwdChainPlan{{0, 0, 0}, -1, 0, 0, 0};
  p.cfg = c;
  p.gm = gm;
  p.nseq = (int64_t)B * H;
  p.bytes = kChainHeader + (size_t)p.nseq * (size_t)(p.nchunk - 1) * (size_t)(c.CL * V) * 8u;
  return p;
}

struct BwdWorkspace {
  // byte offsets
  size_t partial = 0, agg = 0, carry = 0, dalpha = 0;
  size_t dinit = 0;  // per-(b, h) inits gradients for their batch sum
  size_t wst = 0, wdu = 0, wdl = 0, wdi = 0;  // look-back windows
  size_t du = 0;  // look-back windows, per-channel kernel: value-gradient sums
  size_t total = 0;
};

// Warm-up rows per look-back window (no window's warm-up is longer).
inline int look_back_kw(int T, int K) { return std::min(K - 1, T); }

BwdWorkspace bwd_workspace_plan(int dtype, int B, int T, int NH, int NKVH, int Da, int r, int P,
                                int Q, int K) {
  const int H = NH + 2 * NKVH;
  const int V = dtype == LTV_DTYPE_BF16 ? 8 : 4;
  const int D = Da * r;
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  BwdWorkspace w;
  const int nwin = look_back_nwin(T, P, Q);
  if (nwin > 1 && (tuning().lb_short && lb_short_ok(V, r, Q, K))) {
    // short windows: dbias partials, per-window grad_inits shares and the
    // per-(b, h) inits gradients of the batch sum
    const size_t rows = (size_t)B * H * nwin;
    size_t off = al(rows * Da * sizeof(float));
    w.wdi = off;
    off += al(rows * D * sizeof(float));
    w.dinit = off;
    off += al((size_t)B * H * D * sizeof(float));
    w.total = off;
    return w;
  }
  if (nwin > 1) {
    const size_t es = dtype == LTV_DTYPE_BF16 ? 2 : 4;
    const size_t rows = (size_t)B * H * nwin;
    const size_t kw = (size_t)look_back_kw(T, K);
    size_t off = al(rows * Da * sizeof(float));
    w.wst = off;
    off += al(rows * kw * D * es);
    w.wdu = off;
    off += al(rows * kw * D * sizeof(float));
    w.wdl = off;
    off += al(rows * kw * Da * sizeof(float));
    w.wdi = off;
    off += al(rows * D * sizeof(float));
    if (bwd_gate_mode(r, Da, V) < 0) {
      // the per-channel kernel's dalpha and value-gradient sums
      w.dalpha = off;
      off += al((size_t)B * H * T * D * sizeof(float));
      w.du = off;
      off += al((size_t)B * H * T * D * sizeof(float));
    }
    w.total = off;
    return w;
  }
  const int NC = bwd_max_chunks(B, H, T);
  // dbias partials for the tile kernel's chunks or the chained kernel's
  const int NP = std::max(NC, bwd_chain_plan(dtype, B, T, H, Da, r).nchunk);
  size_t off = al((size_t)B * H * NP * Da * sizeof(float));
  if (NC > 1) {
    w.agg = off;
    off += al((size_t)2 * B * H * ((T + kBwdFineSteps - 1) / kBwdFineSteps) * D * sizeof(float));
    w.carry = off;
    off += al((size_t)B * H * NC * D * sizeof(float));
  }
  w.dinit = off;
  off += al((size_t)B * H * D * sizeof(float));
  if (bwd_gate_mode(r, Da, V) < 0) {
    w.dalpha = off;
    off += (size_t)B * H * T * D * sizeof(float);
  }
  w.total = off;
  return w;
}

size_t bwd_workspace_bytes(int dtype, int B, int T, int NH, int NKVH, int Da, int r, int P,
                          int Q, int K) {
  return bwd_workspace_plan(dtype, B, T, NH, NKVH, Da, r, P, Q, K).total;
}

int scan_backward_impl(int dtype, const HostView4& u, const HostView4& lg, const HostView4& init,
                       int inits_dtype, const float* bias, const void* const hp[3],
                       const int64_t* const hs[3], const void* const gp[3],
                       const int64_t* const gs[3], const HostView4& du, const HostView4& dlg,
                       int dlg_pad, const HostView4& dinit, float* dbias, void* ws,
                       size_t ws_bytes,
                       void* chain_ws, size_t chain_ws_bytes, int B, int T, int NH, int NKVH,
                       int Da, int r, int P, int Q, int K, int use_sigmoid, hipStream_t st) {
  int rc = check_shape(dtype, B, T, NH, NKVH, Da, r);
  if (rc) return rc;
  rc = check_pqk(P, Q, K);
  if (rc) return rc;
  rc = check_inits_dtype(dtype, inits_dtype);
  if (rc) return rc;
  const bool init_f32 = inits_dtype != dtype;
  const int EI = inits_dtype == LTV_DTYPE_BF16 ? 2 : 4;  // bytes per inits element
  // grad_inits with batch stride 0: the sum over the batch (what the
  // broadcast of one set of inits to every sequence gives back)
  const bool dinit_sum = B > 1 && dinit.s[0] == 0;
  const int H = NH + 2 * NKVH;
  const int D = Da * r;
  LTV_REQUIRE(dlg_pad >= 0 && dlg_pad <= 64, LTV_ERR_INVALID_ARG,
              "grad_logits padding of %d slots: must be 0 .. 64", dlg_pad);
  LTV_REQUIRE(dlg_pad == 0 || dlg.s[1] == (int64_t)Da * dlg.s[3], LTV_ERR_INVALID_ARG,
              "grad_logits padding needs the heads' gate slots contiguous (head stride = Da x "
              "gate stride)");
  if (H == 0) return LTV_OK;
  LTV_REQUIRE(dbias != nullptr, LTV_ERR_INVALID_ARG, "null grad_logit_bias");
  if (B == 0 || T == 0) {
    // nothing flows back: grad_logit_bias and grad_inits are zero
    const int64_t n = (int64_t)B * H * D;
    LTV_REQUIRE(n == 0 || dinit.p != nullptr, LTV_ERR_INVALID_ARG, "null grad_inits");
    const int64_t blocks = std::max<int64_t>(1, (n + 255) / 256);
    LTV_REQUIRE(blocks < (1ll << 31), LTV_ERR_UNSUPPORTED, "grad_inits too large");
    hipLaunchKernelGGL(zero_bhd_kernel, dim3((int)blocks), dim3(256), 0, st,
                       reinterpret_cast<char*>(const_cast<void*>(dinit.p)), to_dev(dinit), B, H, D,
                       EI, dbias, H * Da);
    LTV_LAUNCH_CHECK();
    return LTV_OK;
  }
  const size_t need = bwd_workspace_bytes(dtype, B, T, NH, NKVH, Da, r, P, Q, K);
  LTV_REQUIRE(ws != nullptr && ws_bytes >= need, LTV_ERR_WORKSPACE,
              "workspace too small: need %zu bytes, got %zu", need, ws_bytes);
  const int V = dtype == LTV_DTYPE_BF16 ? 8 : 4;

  BwdArgs a;
  a.sh = ScanShape{B, T, NH, NKVH, Da, r, D, H, 1, use_sigmoid};
  a.u = to_dev(u);
  a.lg = to_dev(lg);
  a.init = to_dev(init);
  a.init_f32 = init_f32 ? 1 : 0;
  a.dinit_ws = nullptr;
  a.bias = bias;
  a.wpl = 1;
  const int E = dtype == LTV_DTYPE_BF16 ? 2 : 4;
  if ((rc = check_tile_offsets("values", u.s, D, E)) || (rc = check_tile_offsets("logits", lg.s, D, E)) ||
      (rc = check_tile_offsets("grad values", du.s, D, E)) ||
      (rc = check_tile_offsets("grad logits", dlg.s, D, E)) ||
      (rc = check_tile_offsets("inits", init.s, D, EI)))
    return rc;
  bool vec = (D % V == 0) && vec_ok(u.p, u.s, 3, V) && vec_ok(init.p, init.s, 3, V) &&
             vec_ok(du.p, du.s, 3, V) && vec_ok(dinit.p, dinit.s, 3, V);
  for (int i = 0; i < 3; ++i) {
    a.h.p[i] = const_cast<void*>(hp[i]);
    a.gy.p[i] = const_cast<void*>(gp[i]);
    for (int k = 0; k < 4; ++k) {
      a.h.s[i][k] = hs[i][k];
      a.gy.s[i][k] = gs[i][k];
    }
    const int nh = i == 0 ? NH : NKVH;
    if (nh > 0) {
      LTV_REQUIRE(hp[i] && gp[i], LTV_ERR_INVALID_ARG, "null saved output or gradient pointer");
      if ((rc = check_tile_offsets("saved outputs", hs[i], D, E)) ||
          (rc = check_tile_offsets("output gradients", gs[i], D, E)))
        return rc;
      vec = vec && vec_ok(hp[i], hs[i], 3, V) && vec_ok(gp[i], gs[i], 3, V);
    }
  }
  a.du = to_dev(du);
  a.dlg = to_dev(dlg);
  a.dinit = to_dev(dinit);
  const BwdWorkspace wp = bwd_workspace_plan(dtype, B, T, NH, NKVH, Da, r, P, Q, K);
  char* wsb = reinterpret_cast<char*>(ws);
  a.dbias_partial = reinterpret_cast<float*>(wsb + wp.partial);
  a.nchunk = 1;
  a.chunk_steps = T;
  a.nfine = 1;
  a.fine_steps = T;
  a.agg = nullptr;
  a.carry = nullptr;
  a.P = P;
  a.Q = Q;
  a.K = K;
  a.kw = 0;
  a.wst = nullptr;
  a.wdu = a.wdl = a.wdi = nullptr;
  a.ch_ticket = a.ch_err = nullptr;
  a.ch_ctl = ChainCtl{nullptr, kChainSpinMax, 0};
  a.ch_words = nullptr;

  int gm = bwd_gate_mode(r, Da, V);
  if (gm == GATE_CHAN && vec && chanvec_ok(r, D, V, lg) && chanvec_ok(r, D, V, dlg))
    gm = GATE_CHANVEC;
  const int nwin = look_back_nwin(T, P, Q);
  const bool lb_short = nwin > 1 && tuning().lb_short && lb_short_ok(V, r, Q, K);
  LTV_REQUIRE(!(init_f32 || dinit_sum) || (nwin == 1 && gm >= 0) || lb_short,
              LTV_ERR_UNSUPPORTED,
              "fp32 inits with bf16 values, or grad_inits summed over the batch (batch stride "
              "0), need the full recurrence (P >= T) and gate groups of r channels with r a "
              "multiple of %d and Da <= %d, or r dividing %d (r=%d Da=%d), or look-back "
              "windows the short-window kernels take",
              V, kMaxLaneGroups, V, r, Da);
  PadZero pz;
  if (dlg_pad > 0) {
    pz.base = reinterpret_cast<char*>(const_cast<void*>(dlg.p));
    pz.sb = dlg.s[0];
    pz.st = dlg.s[2];
    pz.sq = dlg.s[3];
    pz.B = B;
    pz.T = T;
    pz.q0 = H * Da;
    pz.pad = dlg_pad;
    pz.esize = E;
  }
  DinitSum ds;
  if (dinit_sum) {
    a.dinit_ws = reinterpret_cast<float*>(wsb + wp.dinit);
    ds.ws = a.dinit_ws;
    ds.out = const_cast<void*>(dinit.p);
    ds.sh = dinit.s[1];
    ds.sd = dinit.s[3];
    ds.D = D;
    ds.out_bf16 = inits_dtype == LTV_DTYPE_BF16 ? 1 : 0;
  }
  if (nwin > 1 && (tuning().lb_short && lb_short_ok(V, r, Q, K))) {
    // Short look-back windows: one lane per window gathers its steps' whole
    // gradient (ltv_scan_lb.hip); then the per-window grad_inits shares and
    // dbias partials are summed.
    const bool bf16 = dtype == LTV_DTYPE_BF16;
    a.nchunk = nwin;
    a.lanes = next_pow2((D + V - 1) / V);
    a.wdi = reinterpret_cast<float*>(wsb + wp.wdi);
    int sgm = GATE_CHAN;
    if (r % V == 0) sgm = GATE_LANE;
    else if (vec && chanvec_ok(r, D, V, lg) && chanvec_ok(r, D, V, dlg)) sgm = GATE_CHANVEC;
    bool buf = view_span_bytes(u.s, 1, 1, T, D, E) <= kBufSpanMax &&
               view_span_bytes(lg.s, 1, 1, T, std::max(D, Da), E) <= kBufSpanMax &&
               view_span_bytes(du.s, 1, 1, T, D, E) <= kBufSpanMax &&
               view_span_bytes(dlg.s, 1, 1, T, std::max(D, Da), E) <= kBufSpanMax;
    for (int i = 0; i < 3; ++i)
      if ((i == 0 ? NH : NKVH) > 0)
        buf = buf && view_span_bytes(hs[i], 1, 1, T, D, E) <= kBufSpanMax &&
              view_span_bytes(gs[i], 1, 1, T, D, E) <= kBufSpanMax;
    // Several consecutive windows per lane, each handing its chain value and
    // warm-up to the window before it (u and gy then read once per step), as
    // long as about 1.5 rounds of resident wavefronts remain (two workgroups
    // of four per CU: the kernel's 64 KB of LDS).  The kernel is bound by its
    // load latency more than by its bytes: measured at the d12 look-back shape
    // (B = 32, 9,216 wavefronts with one window each), 1 / 3 / 5 windows per
    // lane read 680 / 555 / 519 MB, and the backward with its two reduction
    // launches takes 178 / 171 / 194 us.
    if (buf && K - 1 <= 8 && K - 1 < Q && K - 1 < P) {
      const int64_t waves1 = (int64_t)B * H * (((int64_t)nwin * a.lanes + 63) / 64);
      const int64_t slots = (int64_t)scan_cu_count() * 8;
      int64_t w = waves1 * 2 / (3 * slots);
      if (tuning().lb_wpl > 0) w = tuning().lb_wpl;
      if (g_lb_wpl.load(std::memory_order_relaxed) > 0) w = g_lb_wpl.load(std::memory_order_relaxed);
      a.wpl = (int)std::max<int64_t>(1, std::min<int64_t>(w, nwin));
    }
    LTV_REQUIRE(!init_f32 || buf, LTV_ERR_UNSUPPORTED,
                "fp32 inits with look-back windows need views whose (b, h) slices span less "
                "than 2 GiB");
    rc = scan_launch_lb_short_bwd(bf16, a, vec, sgm, K - 1, buf, st);
    if (rc) return rc;
    rc = scan_launch_lb_dinit(bf16, a, st);
    if (rc) return rc;
    return scan_launch_dbias_reduce(a.dbias_partial, dbias, B, H, nwin, Da, st, ds, pz);
  }
  if (nwin > 1) {
    // Look-back windows: recompute each window's warm-up states, run every
    // window's reverse chain, then fold the warm-up contributions into the
    // owning windows' steps and sum the inits gradients (gate groups outside
    // the tile kernel's patterns: one thread per channel walks the windows).
    const int64_t grid = (int64_t)B * H * nwin;
    LTV_REQUIRE(grid < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
    a.nchunk = nwin;
    a.kw = look_back_kw(T, K);
    a.wst = wsb + wp.wst;
    a.wdu = reinterpret_cast<float*>(wsb + wp.wdu);
    a.wdl = reinterpret_cast<float*>(wsb + wp.wdl);
    a.wdi = reinterpret_cast<float*>(wsb + wp.wdi);
    const bool bf16 = dtype == LTV_DTYPE_BF16;
    if (a.kw > 0) {
      FwdArgs f;
      f.u = a.u;
      f.lg = a.lg;
      f.init = a.init;
      f.init_f32 = 0;
      f.bias = bias;
      for (int i = 0; i < 3; ++i) {
        f.out.p[i] = nullptr;
        for (int k = 0; k < 4; ++k) f.out.s[i][k] = 0;
      }
      f.P = P;
      f.Q = Q;
      f.K = K;
      f.nwin = nwin;
      f.wst = const_cast<void*>(a.wst);
      f.kw = a.kw;
      const bool fvec = (D % V == 0) && vec_ok(u.p, u.s, 3, V) && vec_ok(init.p, init.s, 3, V);
      rc = launch_forward(dtype, f, fvec, lg, B, T, NH, NKVH, Da, r, use_sigmoid, st);
      if (rc) return rc;
    }
    if (gm < 0) {
      LTV_REQUIRE((int64_t)B * H * D < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
      rc = scan_launch_lb_channel(bf16, a, reinterpret_cast<float*>(wsb + wp.dalpha),
                                  reinterpret_cast<float*>(wsb + wp.du), st);
      if (rc) return rc;
      return scan_launch_dbias_reduce(a.dbias_partial, dbias, B, H, 1, Da, st, ds, pz);
    }
    ScanCfg cfg = bwd_default_cfg(next_pow2((D + V - 1) / V), vec);
    const ScanTuning& tu = tuning();
    if (vec && tu.bwd_l > 0) {
      cfg.L = tu.bwd_l;
      cfg.NW = tu.bwd_nw;
    }
    rc = scan_launch_bwd(bf16, a, cfg, (int)grid, vec, gm, true, st);
    if (rc) return rc;
    if (a.kw > 0) {
      rc = scan_launch_lb_fold(bf16, a, st);
      if (rc) return rc;
    }
    rc = scan_launch_lb_dinit(bf16, a, st);
    if (rc) return rc;
    return scan_launch_dbias_reduce(a.dbias_partial, dbias, B, H, nwin, Da, st, ds, pz);
  }
  if (gm >= 0 && vec && chain_ws != nullptr) {
    // chained: one tile per chunk, the carries handed between workgroups
    const BwdChainPlan pl = bwd_chain_plan(dtype, B, T, H, Da, r);
    if (pl.cfg.CL > 0 && pl.gm == gm) {
      LTV_REQUIRE(chain_ws_bytes >= pl.bytes, LTV_ERR_WORKSPACE,
                  "chained scan workspace too small: %zu bytes, need %zu", chain_ws_bytes,
                  pl.bytes);
      LTV_REQUIRE((reinterpret_cast<uintptr_t>(chain_ws) & 255u) == 0, LTV_ERR_INVALID_ARG,
                  "chained scan workspace must be 256-byte aligned");
      const int64_t grid = pl.nseq * pl.nchunk;
      LTV_REQUIRE(grid < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
      a.nchunk = pl.nchunk;
      a.chunk_steps = pl.cfg.NW * (64 / pl.cfg.CL) * pl.cfg.L;
      a.ch_ticket = reinterpret_cast<uint32_t*>(chain_ws);
      a.ch_err = reinterpret_cast<uint32_t*>(chain_ws) + 1;
      a.ch_words = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(chain_ws) +
                                                         kChainHeader);
      a.ch_ctl = chain_ctl(st);
      rc = scan_launch_bwd_chain(dtype == LTV_DTYPE_BF16, a, pl.cfg, (int)grid, gm, st);
      if (rc) return rc;
      return scan_launch_dbias_reduce(a.dbias_partial, dbias, B, H, a.nchunk, Da, st, ds, pz);
    }
  }
  if (gm >= 0) {
    // whole head per workgroup
    ScanCfg cfg = bwd_tile_cfg(next_pow2((D + V - 1) / V), vec, (int64_t)B * H);
    const ScanTuning& tu = tuning();
    if (vec && tu.bwd_l > 0) {
      cfg.L = tu.bwd_l;
      cfg.NW = tu.bwd_nw;
    }
    // time chunks of whole tiles; each chunk enters with its exact gradient
    // carry from the chunk-map kernels
    // (TW and the sub-chunk length are powers of two: the larger is a multiple
    // of the smaller)
    const int TW = cfg.NW * (64 / cfg.CL) * cfg.L;
    const int unit = std::max(TW, kBwdFineSteps);
    const int nc_max = bwd_max_chunks(B, H, T);
    const int per = (T + nc_max - 1) / nc_max;
    a.chunk_steps = (per + unit - 1) / unit * unit;
    a.nchunk = (T + a.chunk_steps - 1) / a.chunk_steps;
    a.fine_steps = kBwdFineSteps;
    a.nfine = (T + kBwdFineSteps - 1) / kBwdFineSteps;
    const int64_t grid = (int64_t)B * H * a.nchunk;
    LTV_REQUIRE(grid < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
    if (a.nchunk > 1) {
      a.agg = reinterpret_cast<float*>(wsb + wp.agg);
      a.carry = reinterpret_cast<float*>(wsb + wp.carry);
      rc = scan_launch_bwd_chunk_maps(dtype == LTV_DTYPE_BF16, a, vec, st);
      if (rc) return rc;
    }
    rc = scan_launch_bwd(dtype == LTV_DTYPE_BF16, a, cfg, (int)grid, vec, gm, false, st);
    if (rc) return rc;
  } else {
    LTV_REQUIRE((int64_t)B * H < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
    float* dalpha = reinterpret_cast<float*>(wsb + wp.dalpha);
    rc = scan_launch_bwd_channel(dtype == LTV_DTYPE_BF16, a, dalpha, st);
    if (rc) return rc;
  }
  return scan_launch_dbias_reduce(a.dbias_partial, dbias, B, H, a.nchunk, Da, st, ds, pz);
}

// (B, T, F) interleaved tensor -> value / logit 4-D views
inline HostView4 values_view(const void* p, const int64_t* cs, int D, int Da) {
  HostView4 v;
  v.p = p;
  v.s[0] = cs[0];
  v.s[1] = (int64_t)(D + Da) * cs[2];
  v.s[2] = cs[1];
  v.s[3] = cs[2];
  return v;
}

inline HostView4 logits_view(const void* p, const int64_t* cs, int D, int Da, int esize) {
  HostView4 v = values_view(p, cs, D, Da);
  v.p = reinterpret_cast<const char*>(p) + (int64_t)D * cs[2] * esize;
  return v;
}

inline HostView4 view3(const void* p, const int64_t* s) {
  HostView4 v;
  v.p = p;
  v.s[0] = s[0];
  v.s[1] = s[1];
  v.s[2] = 0;
  v.s[3] = s[2];
  return v;
}

inline HostView4 view4(const void* p, const int64_t* s) {
  HostView4 v;
  v.p = p;
  for (int i = 0; i < 4; ++i) v.s[i] = s[i];
  return v;
}

}  // namespace
}  // namespace ltv

using namespace ltv;

namespace {
constexpr int kUnboundedP = 2147483647;  // P of the full recurrence: one window
}

extern "C" int ltv_hm_look_back_scan_forward(
    int dtype, const void* combined, const int64_t combined_strides[3], const void* inits,
    const int64_t inits_strides[3], const float* logit_bias, void* out_q,
    const int64_t out_q_strides[4], void* out_k, const int64_t out_k_strides[4], void* out_v,
    const int64_t out_v_strides[4], int B, int T, int NH, int NKVH, int Da, int r, int P, int Q,
    int K, int use_sigmoid, void* stream) {
  LTV_REQUIRE(combined_strides && inits_strides && out_q_strides && out_k_strides &&
                  out_v_strides,
              LTV_ERR_INVALID_ARG, "null stride array");
  const int D = Da * r;
  const int es = dtype == LTV_DTYPE_BF16 ? 2 : 4;
  void* outp[3] = {out_q, out_k, out_v};
  const int64_t* outs[3] = {out_q_strides, out_k_strides, out_v_strides};
  return scan_forward_impl(dtype, values_view(combined, combined_strides, D, Da),
                           logits_view(combined, combined_strides, D, Da, es),
                           view3(inits, inits_strides), dtype, logit_bias, outp, outs, B, T, NH, NKVH,
                           Da, r, P, Q, K, use_sigmoid, nullptr, 0, (hipStream_t)stream);
}

extern "C" int ltv_hm_scan_forward(int dtype, const void* combined,
                                   const int64_t combined_strides[3], const void* inits,
                                   const int64_t inits_strides[3], const float* logit_bias,
                                   void* out_q, const int64_t out_q_strides[4], void* out_k,
                                   const int64_t out_k_strides[4], void* out_v,
                                   const int64_t out_v_strides[4], int B, int T, int NH, int NKVH,
                                   int Da, int r, int use_sigmoid, void* stream) {
  return ltv_hm_look_back_scan_forward(dtype, combined, combined_strides, inits, inits_strides,
                                       logit_bias, out_q, out_q_strides, out_k, out_k_strides,
                                       out_v, out_v_strides, B, T, NH, NKVH, Da, r, kUnboundedP,
                                       1, 1, use_sigmoid, stream);
}

extern "C" int ltv_hm_look_back_scan_forward_split(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    const float* logit_bias, void* out_q, const int64_t out_q_strides[4], void* out_k,
    const int64_t out_k_strides[4], void* out_v, const int64_t out_v_strides[4], int B, int T,
    int NH, int NKVH, int Da, int r, int P, int Q, int K, int use_sigmoid, void* stream) {
  LTV_REQUIRE(values_strides && logits_strides && inits_strides && out_q_strides &&
                  out_k_strides && out_v_strides,
              LTV_ERR_INVALID_ARG, "null stride array");
  void* outp[3] = {out_q, out_k, out_v};
  const int64_t* outs[3] = {out_q_strides, out_k_strides, out_v_strides};
  return scan_forward_impl(dtype, view4(values, values_strides), view4(logits, logits_strides),
                           view3(inits, inits_strides), dtype, logit_bias, outp, outs, B, T, NH, NKVH,
                           Da, r, P, Q, K, use_sigmoid, nullptr, 0, (hipStream_t)stream);
}

extern "C" int ltv_hm_scan_forward_split(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    const float* logit_bias, void* out_q, const int64_t out_q_strides[4], void* out_k,
    const int64_t out_k_strides[4], void* out_v, const int64_t out_v_strides[4], int B, int T,
    int NH, int NKVH, int Da, int r, int use_sigmoid, void* stream) {
  return ltv_hm_look_back_scan_forward_split(
      dtype, values, values_strides, logits, logits_strides, inits, inits_strides, logit_bias,
      out_q, out_q_strides, out_k, out_k_strides, out_v, out_v_strides, B, T, NH, NKVH, Da, r,
      kUnboundedP, 1, 1, use_sigmoid, stream);
}

extern "C" size_t ltv_hm_scan_forward_chain_workspace_size(int dtype, int B, int T, int NH,
                                                          int NKVH, int Da, int r) {
  if (check_shape(dtype, B, T, NH, NKVH, Da, r) != LTV_OK) return 0;
  return chain_plan(dtype, B, T, NH + 2 * NKVH, Da, r).bytes;
}

extern "C" int ltv_hm_scan_forward_ws(int dtype, const void* combined,
                                      const int64_t combined_strides[3], const void* inits,
                                      const int64_t inits_strides[3], const float* logit_bias,
                                      void* out_q, const int64_t out_q_strides[4], void* out_k,
                                      const int64_t out_k_strides[4], void* out_v,
                                      const int64_t out_v_strides[4], void* chain_workspace,
                                      size_t chain_workspace_bytes, int B, int T, int NH,
                                      int NKVH, int Da, int r, int use_sigmoid, void* stream) {
  LTV_REQUIRE(combined_strides && inits_strides && out_q_strides && out_k_strides &&
                  out_v_strides,
              LTV_ERR_INVALID_ARG, "null stride array");
  const int D = Da * r;
  const int es = dtype == LTV_DTYPE_BF16 ? 2 : 4;
  void* outp[3] = {out_q, out_k, out_v};
  const int64_t* outs[3] = {out_q_strides, out_k_strides, out_v_strides};
  return scan_forward_impl(dtype, values_view(combined, combined_strides, D, Da),
                           logits_view(combined, combined_strides, D, Da, es),
                           view3(inits, inits_strides), dtype, logit_bias, outp, outs, B, T, NH, NKVH,
                           Da, r, kUnboundedP, 1, 1, use_sigmoid, chain_workspace,
                           chain_workspace_bytes, (hipStream_t)stream);
}

extern "C" int ltv_hm_look_back_scan_forward_split_ws(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    int inits_dtype, const float* logit_bias, void* out_q, const int64_t out_q_strides[4],
    void* out_k, const int64_t out_k_strides[4], void* out_v, const int64_t out_v_strides[4],
    void* chain_workspace, size_t chain_workspace_bytes, int B, int T, int NH, int NKVH, int Da,
    int r, int P, int Q, int K, int use_sigmoid, void* stream) {
  LTV_REQUIRE(values_strides && logits_strides && inits_strides && out_q_strides &&
                  out_k_strides && out_v_strides,
              LTV_ERR_INVALID_ARG, "null stride array");
  void* outp[3] = {out_q, out_k, out_v};
  const int64_t* outs[3] = {out_q_strides, out_k_strides, out_v_strides};
  return scan_forward_impl(dtype, view4(values, values_strides), view4(logits, logits_strides),
                           view3(inits, inits_strides), inits_dtype, logit_bias, outp, outs, B, T,
                           NH, NKVH, Da, r, P, Q, K, use_sigmoid, chain_workspace,
                           chain_workspace_bytes, (hipStream_t)stream);
}

extern "C" size_t ltv_hm_look_back_scan_backward_workspace_size(int dtype, int B, int T, int NH,
                                                                int NKVH, int Da, int r, int P,
                                                                int Q, int K) {
  if (P < 0 || Q < 1 || K < 1) return 0;
  return bwd_workspace_bytes(dtype, B, T, NH, NKVH, Da, r, P, Q, K);
}

extern "C" size_t ltv_hm_scan_backward_workspace_size(int dtype, int B, int T, int NH, int NKVH,
                                                      int Da, int r) {
  return bwd_workspace_bytes(dtype, B, T, NH, NKVH, Da, r, kUnboundedP, 1, 1);
}

namespace {
int scan_backward_combined(
    int dtype, const void* combined, const int64_t combined_strides[3], const void* inits,
    const int64_t inits_strides[3], const float* logit_bias, const void* hq,
    const int64_t hq_strides[4], const void* hk, const int64_t hk_strides[4], const void* hv,
    const int64_t hv_strides[4], const void* grad_hq, const int64_t grad_hq_strides[4],
    const void* grad_hk, const int64_t grad_hk_strides[4], const void* grad_hv,
    const int64_t grad_hv_strides[4], void* grad_combined, const int64_t grad_combined_strides[3],
    void* grad_inits, const int64_t grad_inits_strides[3], float* grad_logit_bias,
    void* workspace, size_t workspace_bytes, void* chain_ws, size_t chain_ws_bytes, int B, int T,
    int NH, int NKVH, int Da, int r, int P, int Q, int K, int use_sigmoid, void* stream) {
  LTV_REQUIRE(combined_strides && inits_strides && hq_strides && hk_strides && hv_strides &&
                  grad_hq_strides && grad_hk_strides && grad_hv_strides &&
                  grad_combined_strides && grad_inits_strides,
              LTV_ERR_INVALID_ARG, "null stride array");
  const int D = Da * r;
  const int es = dtype == LTV_DTYPE_BF16 ? 2 : 4;
  const void* hp[3] = {hq, hk, hv};
  const int64_t* hs[3] = {hq_strides, hk_strides, hv_strides};
  const void* gp[3] = {grad_hq, grad_hk, grad_hv};
  const int64_t* gs[3] = {grad_hq_strides, grad_hk_strides, grad_hv_strides};
  return scan_backward_impl(
      dtype, values_view(combined, combined_strides, D, Da),
      logits_view(combined, combined_strides, D, Da, es), view3(inits, inits_strides), dtype,
      logit_bias, hp, hs, gp, gs, values_view(grad_combined, grad_combined_strides, D, Da),
      logits_view(grad_combined, grad_combined_strides, D, Da, es), 0,
      view3(grad_inits, grad_inits_strides), grad_logit_bias, workspace, workspace_bytes,
      chain_ws, chain_ws_bytes, B, T, NH, NKVH, Da, r, P, Q, K, use_sigmoid, (hipStream_t)stream);
}
}  // namespace

extern "C" int ltv_hm_look_back_scan_backward(
    int dtype, const void* combined, const int64_t combined_strides[3], const void* inits,
    const int64_t inits_strides[3], const float* logit_bias, const void* hq,
    const int64_t hq_strides[4], const void* hk, const int64_t hk_strides[4], const void* hv,
    const int64_t hv_strides[4], const void* grad_hq, const int64_t grad_hq_strides[4],
    const void* grad_hk, const int64_t grad_hk_strides[4], const void* grad_hv,
    const int64_t grad_hv_strides[4], void* grad_combined, const int64_t grad_combined_strides[3],
    void* grad_inits, const int64_t grad_inits_strides[3], float* grad_logit_bias,
    void* workspace, size_t workspace_bytes, int B, int T, int NH, int NKVH, int Da, int r, int P,
    int Q, int K, int use_sigmoid, void* stream) {
  return scan_backward_combined(
      dtype, combined, combined_strides, inits, inits_strides, logit_bias, hq, hq_strides, hk,
      hk_strides, hv, hv_strides, grad_hq, grad_hq_strides, grad_hk, grad_hk_strides, grad_hv,
      grad_hv_strides, grad_combined, grad_combined_strides, grad_inits, grad_inits_strides,
      grad_logit_bias, workspace, workspace_bytes, nullptr, 0, B, T, NH, NKVH, Da, r, P, Q, K,
      use_sigmoid, stream);
}

extern "C" size_t ltv_hm_scan_backward_chain_workspace_size(int dtype, int B, int T, int NH,
                                                           int NKVH, int Da, int r) {
  if (check_shape(dtype, B, T, NH, NKVH, Da, r) != LTV_OK) return 0;
  return bwd_chain_plan(dtype, B, T, NH + 2 * NKVH, Da, r).bytes;
}

extern "C" int ltv_chain_take_error(void) {
  ltv::ChainHost& h = ltv::chain_host();
  std::lock_guard<std::mutex> lk(h.mu);
  if (h.host == nullptr) return 0;
  return (int)__atomic_exchange_n(h.host, 0u, __ATOMIC_SEQ_CST);
}

extern "C" int ltv_lb_set_windows_per_lane(int wpl) {
  LTV_REQUIRE(wpl >= 0, LTV_ERR_INVALID_ARG, "wpl must be >= 0 (got %d)", wpl);
  ltv::g_lb_wpl.store(wpl, std::memory_order_relaxed);
  return LTV_OK;
}

extern "C" int ltv_chain_set_test_controls(int spin_max, int no_publish) {
  LTV_REQUIRE(spin_max >= 0, LTV_ERR_INVALID_ARG, "spin_max must be >= 0 (got %d)", spin_max);
  ltv::ChainHost& h = ltv::chain_host();
  std::lock_guard<std::mutex> lk(h.mu);
  h.spin_max = spin_max == 0 ? ltv::kChainSpinMax : spin_max;
  h.no_publish = no_publish != 0;
  return LTV_OK;
}

extern "C" int ltv_hm_scan_backward_ws(
    int dtype, const void* combined, const int64_t combined_strides[3], const void* inits,
    const int64_t inits_strides[3], const float* logit_bias, const void* hq,
    const int64_t hq_strides[4], const void* hk, const int64_t hk_strides[4], const void* hv,
    const int64_t hv_strides[4], const void* grad_hq, const int64_t grad_hq_strides[4],
    const void* grad_hk, const int64_t grad_hk_strides[4], const void* grad_hv,
    const int64_t grad_hv_strides[4], void* grad_combined, const int64_t grad_combined_strides[3],
    void* grad_inits, const int64_t grad_inits_strides[3], float* grad_logit_bias,
    void* workspace, size_t workspace_bytes, void* chain_workspace, size_t chain_workspace_bytes,
    int B, int T, int NH, int NKVH, int Da, int r, int use_sigmoid, void* stream) {
  return scan_backward_combined(
      dtype, combined, combined_strides, inits, inits_strides, logit_bias, hq, hq_strides, hk,
      hk_strides, hv, hv_strides, grad_hq, grad_hq_strides, grad_hk, grad_hk_strides, grad_hv,
      grad_hv_strides, grad_combined, grad_combined_strides, grad_inits, grad_inits_strides,
      grad_logit_bias, workspace, workspace_bytes, chain_workspace, chain_workspace_bytes, B, T,
      NH, NKVH, Da, r, kUnboundedP, 1, 1, use_sigmoid, stream);
}

extern "C" int ltv_hm_scan_backward(
    int dtype, const void* combined, const int64_t combined_strides[3], const void* inits,
    const int64_t inits_strides[3], const float* logit_bias, const void* hq,
    const int64_t hq_strides[4], const void* hk, const int64_t hk_strides[4], const void* hv,
    const int64_t hv_strides[4], const void* grad_hq, const int64_t grad_hq_strides[4],
    const void* grad_hk, const int64_t grad_hk_strides[4], const void* grad_hv,
    const int64_t grad_hv_strides[4], void* grad_combined, const int64_t grad_combined_strides[3],
    void* grad_inits, const int64_t grad_inits_strides[3], float* grad_logit_bias,
    void* workspace, size_t workspace_bytes, int B, int T, int NH, int NKVH, int Da, int r,
    int use_sigmoid, void* stream) {
  return ltv_hm_look_back_scan_backward(
      dtype, combined, combined_strides, inits, inits_strides, logit_bias, hq, hq_strides, hk,
      hk_strides, hv, hv_strides, grad_hq, grad_hq_strides, grad_hk, grad_hk_strides, grad_hv,
      grad_hv_strides, grad_combined, grad_combined_strides, grad_inits, grad_inits_strides,
      grad_logit_bias, workspace, workspace_bytes, B, T, NH, NKVH, Da, r, kUnboundedP, 1, 1,
      use_sigmoid, stream);
}

extern "C" int ltv_hm_look_back_scan_backward_split_ws(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    int inits_dtype, const float* logit_bias, const void* hq, const int64_t hq_strides[4],
    const void* hk, const int64_t hk_strides[4], const void* hv, const int64_t hv_strides[4],
    const void* grad_hq, const int64_t grad_hq_strides[4], const void* grad_hk,
    const int64_t grad_hk_strides[4], const void* grad_hv, const int64_t grad_hv_strides[4],
    void* grad_values, const int64_t grad_values_strides[4], void* grad_logits,
    const int64_t grad_logits_strides[4], int grad_logits_pad, void* grad_inits,
    const int64_t grad_inits_strides[3], float* grad_logit_bias, void* workspace,
    size_t workspace_bytes, void* chain_workspace, size_t chain_workspace_bytes, int B, int T,
    int NH, int NKVH, int Da, int r, int P, int Q, int K, int use_sigmoid, void* stream) {
  LTV_REQUIRE(values_strides && logits_strides && inits_strides && hq_strides && hk_strides &&
                  hv_strides && grad_hq_strides && grad_hk_strides && grad_hv_strides &&
                  grad_values_strides && grad_logits_strides && grad_inits_strides,
              LTV_ERR_INVALID_ARG, "null stride array");
  const void* hp[3] = {hq, hk, hv};
  const int64_t* hs[3] = {hq_strides, hk_strides, hv_strides};
  const void* gp[3] = {grad_hq, grad_hk, grad_hv};
  const int64_t* gs[3] = {grad_hq_strides, grad_hk_strides, grad_hv_strides};
  return scan_backward_impl(dtype, view4(values, values_strides), view4(logits, logits_strides),
                            view3(inits, inits_strides), inits_dtype, logit_bias, hp, hs, gp, gs,
                            view4(grad_values, grad_values_strides),
                            view4(grad_logits, grad_logits_strides), grad_logits_pad,
                            view3(grad_inits, grad_inits_strides), grad_logit_bias, workspace,
                            workspace_bytes, chain_workspace, chain_workspace_bytes, B, T, NH,
                            NKVH, Da, r, P, Q, K, use_sigmoid, (hipStream_t)stream);
}

extern "C" int ltv_hm_look_back_scan_backward_split(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    const float* logit_bias, const void* hq, const int64_t hq_strides[4], const void* hk,
    const int64_t hk_strides[4], const void* hv, const int64_t hv_strides[4],
    const void* grad_hq, const int64_t grad_hq_strides[4], const void* grad_hk,
    const int64_t grad_hk_strides[4], const void* grad_hv, const int64_t grad_hv_strides[4],
    void* grad_values, const int64_t grad_values_strides[4], void* grad_logits,
    const int64_t grad_logits_strides[4], void* grad_inits, const int64_t grad_inits_strides[3],
    float* grad_logit_bias, void* workspace, size_t workspace_bytes, int B, int T, int NH,
    int NKVH, int Da, int r, int P, int Q, int K, int use_sigmoid, void* stream) {
  return ltv_hm_look_back_scan_backward_split_ws(
      dtype, values, values_strides, logits, logits_strides, inits, inits_strides, dtype,
      logit_bias,
      hq, hq_strides, hk, hk_strides, hv, hv_strides, grad_hq, grad_hq_strides, grad_hk,
      grad_hk_strides, grad_hv, grad_hv_strides, grad_values, grad_values_strides, grad_logits,
      grad_logits_strides, 0, grad_inits, grad_inits_strides, grad_logit_bias, workspace,
      workspace_bytes, nullptr, 0, B, T, NH, NKVH, Da, r, P, Q, K, use_sigmoid, stream);
}

extern "C" int ltv_hm_scan_backward_split(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    const float* logit_bias, const void* hq, const int64_t hq_strides[4], const void* hk,
    const int64_t hk_strides[4], const void* hv, const int64_t hv_strides[4],
    const void* grad_hq, const int64_t grad_hq_strides[4], const void* grad_hk,
    const int64_t grad_hk_strides[4], const void* grad_hv, const int64_t grad_hv_strides[4],
    void* grad_values, const int64_t grad_values_strides[4], void* grad_logits,
    const int64_t grad_logits_strides[4], void* grad_inits, const int64_t grad_inits_strides[3],
    float* grad_logit_bias, void* workspace, size_t workspace_bytes, int B, int T, int NH,
    int NKVH, int Da, int r, int use_sigmoid, void* stream) {
  return ltv_hm_look_back_scan_backward_split(
      dtype, values, values_strides, logits, logits_strides, inits, inits_strides, logit_bias,
      hq, hq_strides, hk, hk_strides, hv, hv_strides, grad_hq, grad_hq_strides, grad_hk,
      grad_hk_strides, grad_hv, grad_hv_strides, grad_values, grad_values_strides, grad_logits,
      grad_logits_strides, grad_inits, grad_inits_strides, grad_logit_bias, workspace,
      workspace_bytes, B, T, NH, NKVH, Da, r, kUnboundedP, 1, 1, use_sigmoid, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free backward: ltv_hm_scan_backward with its workspace in a
// file-scope device array instead of a caller buffer.
//
// `scratch` exists once per GPU (each device holds its own copy, at its own
// address, from the library's load until the process ends).  In host code the
// array's name is only a host-side stand-in: the device address is looked up
// once per device with hipGetSymbolAddress, with that device current, and
// only that address is ever handed to kernels.  Every call on one GPU shares
// the array, so calls that overlap on one GPU (different streams, or host
// threads) race on it; calls in one stream are ordered.  The backward writes
// every workspace element it later reads, so nothing has to start at zero.
// ---------------------------------------------------------------------------
#include <mutex>

namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
constexpr int kMaxScratchDevices = 64;

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxScratchDevices] = {};

// Device address of the current device's `scratch` (looked up on the first
// call per device).  The stream, when given, must belong to that device.
int scratch_for_current_device(hipStream_t st, void** out) {
  int dev = -1;
  LTV_HIP_CHECK(hipGetDevice(&dev));
  LTV_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, LTV_ERR_UNSUPPORTED,
              "device index %d beyond the %d devices the scratch table holds", dev,
              kMaxScratchDevices);
  if (st != nullptr) {
    hipDevice_t sdev = -1;
    LTV_HIP_CHECK(hipStreamGetDevice(st, &sdev));
    LTV_REQUIRE((int)sdev == dev, LTV_ERR_INVALID_ARG,
                "stream belongs to device %d but device %d is current", (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    LTV_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    LTV_REQUIRE(p != nullptr, LTV_ERR_HIP, "hipGetSymbolAddress returned a null scratch address");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return LTV_OK;
}

}  // namespace

extern "C" size_t ltv_hm_scan_backward_noalloc_max_workspace(void) { return kNoAllocScratchBytes; }

extern "C" int ltv_hm_scan_backward_noalloc(
    int dtype, const void* combined, const int64_t combined_strides[3], const void* inits,
    const int64_t inits_strides[3], const float* logit_bias, const void* hq,
    const int64_t hq_strides[4], const void* hk, const int64_t hk_strides[4], const void* hv,
    const int64_t hv_strides[4], const void* grad_hq, const int64_t grad_hq_strides[4],
    const void* grad_hk, const int64_t grad_hk_strides[4], const void* grad_hv,
    const int64_t grad_hv_strides[4], void* grad_combined, const int64_t grad_combined_strides[3],
    void* grad_inits, const int64_t grad_inits_strides[3], float* grad_logit_bias, int B, int T,
    int NH, int NKVH, int Da, int r, int use_sigmoid, void* stream) {
  int rc = check_shape(dtype, B, T, NH, NKVH, Da, r);
  if (rc) return rc;
  const size_t need = bwd_workspace_bytes(dtype, B, T, NH, NKVH, Da, r, kUnboundedP, 1, 1);
  LTV_REQUIRE(need <= kNoAllocScratchBytes, LTV_ERR_WORKSPACE,
              "this backward needs %zu bytes of workspace; the allocation-free entry point holds "
              "%zu (use ltv_hm_scan_backward with a caller workspace)",
              need, kNoAllocScratchBytes);
  void* ws = nullptr;
  rc = scratch_for_current_device((hipStream_t)stream, &ws);
  if (rc) return rc;
  return ltv_hm_scan_backward(dtype, combined, combined_strides, inits, inits_strides, logit_bias,
                              hq, hq_strides, hk, hk_strides, hv, hv_strides, grad_hq,
                              grad_hq_strides, grad_hk, grad_hk_strides, grad_hv, grad_hv_strides,
                              grad_combined, grad_combined_strides, grad_inits,
                              grad_inits_strides, grad_logit_bias, ws, kNoAllocScratchBytes, B, T,
                              NH, NKVH, Da, r, use_sigmoid, stream);
}
