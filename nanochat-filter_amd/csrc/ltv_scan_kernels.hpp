// LTV head-major gated EWMA scan, forward and backward, for gfx950.
//
// Recurrence (per channel d of head h, gate group j = d / r):
//   alpha_t = sigmoid(logit_t[j] + bias[h, j])          (or the raw sum)
//   h_t     = (1 - alpha_t) * h_{t-1} + alpha_t * u_t,   h_{-1} = inits
// as in nanochat/ops/ltv_reference_ops.py:83-124 and the CUDA kernels
// cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_{forward,backward}.cu.
//
// Work decomposition (all of T for one (b, head, channel slab) per workgroup):
//   * a lane owns V = 16 / sizeof(io) consecutive channels ("a vector") and a
//     run of L consecutive time steps; the V x L block lives in registers;
//   * a 64-lane wavefront is CL channel lanes x TG = 64 / CL time groups, with
//     lane = cl * TG + tg, so the TG time groups of one channel vector are
//     adjacent lanes;
//   * NW wavefronts split time further; one pass ("tile") covers
//     TW = NW * TG * L steps and the workgroup walks T tile by tile, carrying
//     the fp32 state across tiles in registers.
// Each tile is a three-level affine scan of (a, x) pairs, (a1,x1) then (a2,x2)
// = (a1 a2, a2 x1 + x2):
//   1. per lane: sequential fold of its L steps (registers);
//   2. per wavefront: inclusive scan over the TG time-group lanes (shuffles);
//   3. per workgroup: wavefront aggregates through LDS (one barrier per tile),
//      composed in wavefront order onto the running carry.
// The lane then re-runs its L steps sequentially from its exact carry-in and
// writes the outputs, so values are read from HBM once and written once.
//
// The backward runs the same structure in reverse time over
//   g_t = gy_t + (1 - alpha_{t+1}) g_{t+1},   g_T = 0
// and emits du, dlogit, dinit and a per-workgroup dbias partial (reduced by a
// second, single-workgroup kernel in a fixed order: no atomics, deterministic).

#pragma once

#include "ltv_device.hpp"
#include "ltv_abi_internal.hpp"

namespace ltv {

// ---------------------------------------------------------------------------
// Argument blocks (passed by value as kernel arguments)
// ---------------------------------------------------------------------------
struct View4 {
  const void* p;
  int64_t s[4];  // element strides (b, h, t, c)
};

struct OutHeads {
  void* p[3];      // q, k, v
  int64_t s[3][4];  // element strides (b, h_local, t, d)
};

struct ScanShape {
  int B, T, NH, NKVH, Da, r, D, H;
  int nslab;      // channel slabs per head
  int use_sigmoid;
};

struct FwdArgs {
  ScanShape sh;
  View4 u;       // values   (B, H, T, D)
  View4 lg;      // logits   (B, H, T, Da)
  View4 init;    // inits    (B, H, D) -- s[2] unused
  const float* bias;  // (H, Da) contiguous fp32
  OutHeads out;
};

struct BwdArgs {
  ScanShape sh;
  View4 u;
  View4 lg;
  View4 init;
  const float* bias;
  OutHeads h;      // saved forward outputs
  OutHeads gy;     // upstream gradients
  OutHeads du;     // gradient of the value slots (3 "heads" share one view: p[0])
  View4 dlg;       // gradient of the logit slots
  View4 dinit;     // (B, H, D)
  float* dbias_partial;  // (B, H, Da) fp32 workspace
};

__device__ __forceinline__ void head_select(const OutHeads& o, int h, int NH, int NKVH,
                                            int& which, int& hl) {
  if (h < NH) {
    which = 0;
    hl = h;
  } else if (h < NH + NKVH) {
    which = 1;
    hl = h - NH;
  } else {
    which = 2;
    hl = h - NH - NKVH;
  }
}

// Lane-local load / store of V channels at (b, h, t, c0..c0+V-1) of a strided view.
template <typename TIO, bool VEC>
__device__ __forceinline__ void load_vec(const TIO* base, int64_t sc, int nvalid,
                                         float (&o)[io_traits<TIO>::kVec]) {
  constexpr int V = io_traits<TIO>::kVec;
  if (VEC) {
    uint4 q = *reinterpret_cast<const uint4*>(base);
    unpack16(q, o, TIO());
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) o[v] = (v < nvalid) ? io_traits<TIO>::load(base + v * sc) : 0.0f;
  }
}

template <typename TIO, bool VEC>
__device__ __forceinline__ void store_vec(TIO* base, int64_t sc, int nvalid,
                                          const float (&x)[io_traits<TIO>::kVec]) {
  constexpr int V = io_traits<TIO>::kVec;
  if (VEC) {
    *reinterpret_cast<uint4*>(base) = pack16(x, TIO());
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (v < nvalid) io_traits<TIO>::store(base + v * sc, x[v]);
  }
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// LANEGATE: every lane's V channels share one gate (r % V == 0); otherwise each
// channel reads its own gate j = c / r.
template <typename TIO, int CL, int L, int NW, bool VEC, bool LANEGATE>
__global__ void __launch_bounds__(NW * 64)
scan_fwd_kernel(const FwdArgs args) {
  constexpr int V = io_traits<TIO>::kVec;
  constexpr int TG = 64 / CL;
  constexpr int NA = LANEGATE ? 1 : V;  // decay factors per lane
  const ScanShape& S = args.sh;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int cl = lane / TG;
  const int tg = lane % TG;

  int bid = blockIdx.x;
  const int slab = bid % S.nslab;
  bid /= S.nslab;
  const int h = bid % S.H;
  const int b = bid / S.H;

  const int c0 = (slab * CL + cl) * V;
  const int nvalid = min(V, S.D - c0);  // may be <= 0 for padding lanes
  const bool lane_active = nvalid > 0;

  int which, hl;
  head_select(args.out, h, S.NH, S.NKVH, which, hl);
  TIO* outp = reinterpret_cast<TIO*>(args.out.p[which]);
  const int64_t* os = args.out.s[which];
  outp += (int64_t)b * os[0] + (int64_t)hl * os[1] + (int64_t)c0 * os[3];

  const TIO* up = reinterpret_cast<const TIO*>(args.u.p) + (int64_t)b * args.u.s[0] +
                  (int64_t)h * args.u.s[1] + (int64_t)c0 * args.u.s[3];
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1];

  // gate index and bias per decay factor
  int gj[NA];
  float gbias[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    int c = c0 + (LANEGATE ? 0 : i);
    int j = lane_active ? min(c, S.D - 1) / S.r : 0;
    gj[i] = j;
    gbias[i] = args.bias[h * S.Da + j];
  }

  // running state (exact carry at the start of the current tile)
  float carry[V];
  {
    const TIO* ip = reinterpret_cast<const TIO*>(args.init.p) + (int64_t)b * args.init.s[0] +
                    (int64_t)h * args.init.s[1] + (int64_t)c0 * args.init.s[3];
    if (lane_active)
      load_vec<TIO, VEC>(ip, args.init.s[3], nvalid, carry);
    else
#pragma unroll
      for (int v = 0; v < V; ++v) carry[v] = 0.0f;
  }

  __shared__ float lds_a[2][NW][CL][NA];
  __shared__ float lds_x[2][NW][CL][V];

  constexpr int TW = NW * TG * L;
  const int ntiles = (S.T + TW - 1) / TW;
  const bool use_sig = S.use_sigmoid != 0;

  for (int it = 0; it < ntiles; ++it) {
    const int t0 = it * TW + (w * TG + tg) * L;

    // ---- loads (all L steps issued before any use)
    float uv[L][V];
    float al[L][NA];
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const int t = t0 + s;
      const bool ok = lane_active && t < S.T;
      if (ok) {
        load_vec<TIO, VEC>(up + (int64_t)t * args.u.s[2], args.u.s[3], nvalid, uv[s]);
#pragma unroll
        for (int i = 0; i < NA; ++i)
          al[s][i] = io_traits<TIO>::load(lp + (int64_t)t * args.lg.s[2] +
                                          (int64_t)gj[i] * args.lg.s[3]);
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) uv[s][v] = 0.0f;
#pragma unroll
        for (int i = 0; i < NA; ++i) al[s][i] = 0.0f;
      }
    }
    // ---- gates; padded steps become the identity (alpha = 0 -> a = 1, x = 0)
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const bool ok = lane_active && (t0 + s) < S.T;
#pragma unroll
      for (int i = 0; i < NA; ++i)
        al[s][i] = ok ? gate_alpha(al[s][i] + gbias[i], use_sig) : 0.0f;
    }

    // ---- level 1: lane-local fold
    float A[NA], X[V];
#pragma unroll
    for (int i = 0; i < NA; ++i) A[i] = 1.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) X[v] = 0.0f;
#pragma unroll
    for (int s = 0; s < L; ++s) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float a = al[s][LANEGATE ? 0 : v];
        X[v] = (1.0f - a) * X[v] + a * uv[s][v];
      }
#pragma unroll
      for (int i = 0; i < NA; ++i) A[i] *= (1.0f - al[s][i]);
    }

    // ---- level 2: inclusive scan over the TG time-group lanes
#pragma unroll
    for (int off = 1; off < TG; off <<= 1) {
      float Ap[NA], Xp[V];
#pragma unroll
      for (int i = 0; i < NA; ++i) Ap[i] = __shfl_up(A[i], off, TG);
#pragma unroll
      for (int v = 0; v < V; ++v) Xp[v] = __shfl_up(X[v], off, TG);
      if (tg >= off) {
#pragma unroll
        for (int v = 0; v < V; ++v) X[v] = A[LANEGATE ? 0 : v] * Xp[v] + X[v];
#pragma unroll
        for (int i = 0; i < NA; ++i) A[i] *= Ap[i];
      }
    }
    // exclusive prefix of this lane inside its wavefront
    float Ae[NA], Xe[V];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      float t = __shfl_up(A[i], 1, TG);
      Ae[i] = (tg == 0) ? 1.0f : t;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float t = __shfl_up(X[v], 1, TG);
      Xe[v] = (tg == 0) ? 0.0f : t;
    }

    // ---- level 3: wavefront aggregates through LDS
    float hin[V];
    if (NW > 1) {
      const int buf = it & 1;
      if (tg == TG - 1) {
#pragma unroll
        for (int i = 0; i < NA; ++i) lds_a[buf][w][cl][i] = A[i];
#pragma unroll
        for (int v = 0; v < V; ++v) lds_x[buf][w][cl][v] = X[v];
      }
      __syncthreads();
      // carry into this wavefront, then on to the end of the tile
      float cw[V];
#pragma unroll
      for (int v = 0; v < V; ++v) cw[v] = carry[v];
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        if (ww == w) {
#pragma unroll
          for (int v = 0; v < V; ++v) hin[v] = cw[v];
        }
#pragma unroll
        for (int v = 0; v < V; ++v)
          cw[v] = lds_a[buf][ww][cl][LANEGATE ? 0 : v] * cw[v] + lds_x[buf][ww][cl][v];
      }
#pragma unroll
      for (int v = 0; v < V; ++v) carry[v] = cw[v];
    } else {
      float Aw[NA], Xw[V];
#pragma unroll
      for (int i = 0; i < NA; ++i) Aw[i] = __shfl(A[i], TG - 1, TG);
#pragma unroll
      for (int v = 0; v < V; ++v) Xw[v] = __shfl(X[v], TG - 1, TG);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        hin[v] = carry[v];
        carry[v] = Aw[LANEGATE ? 0 : v] * carry[v] + Xw[v];
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) hin[v] = Ae[LANEGATE ? 0 : v] * hin[v] + Xe[v];

    // ---- re-run the lane's steps from the exact carry-in and store
#pragma unroll
    for (int s = 0; s < L; ++s) {
      float hv[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float a = al[s][LANEGATE ? 0 : v];
        hin[v] = (1.0f - a) * hin[v] + a * uv[s][v];
        hv[v] = hin[v];
      }
      const int t = t0 + s;
      if (lane_active && t < S.T) store_vec<TIO, VEC>(outp + (int64_t)t * os[2], os[3], nvalid, hv);
    }
  }
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
// GROUP_LANES (runtime, power of two): number of channel lanes that share one
// gate when LANEGATE (= r / V); 1 otherwise.  When !LANEGATE, r divides V and
// each lane owns V / r complete gate groups.
template <typename TIO, int CL, int L, int NW, bool VEC, bool LANEGATE>
__global__ void __launch_bounds__(NW * 64)
scan_bwd_kernel(const BwdArgs args) {
  constexpr int V = io_traits<TIO>::kVec;
  constexpr int TG = 64 / CL;
  constexpr int NA = LANEGATE ? 1 : V;
  const ScanShape& S = args.sh;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int cl = lane / TG;
  const int tg = lane % TG;

  int bid = blockIdx.x;  // nslab == 1 for the backward: the workgroup owns the head
  const int h = bid % S.H;
  const int b = bid / S.H;

  const int c0 = cl * V;
  const int nvalid = min(V, S.D - c0);
  const bool lane_active = nvalid > 0;
  const int group_lanes = LANEGATE ? (S.r / V) : 1;   // lanes per gate group
  const int groups_per_lane = LANEGATE ? 1 : (V / S.r);

  int which, hl;
  head_select(args.h, h, S.NH, S.NKVH, which, hl);
  const TIO* hp = reinterpret_cast<const TIO*>(args.h.p[which]);
  const int64_t* hs = args.h.s[which];
  hp += (int64_t)b * hs[0] + (int64_t)hl * hs[1] + (int64_t)c0 * hs[3];
  const TIO* gp = reinterpret_cast<const TIO*>(args.gy.p[which]);
  const int64_t* gs = args.gy.s[which];
  gp += (int64_t)b * gs[0] + (int64_t)hl * gs[1] + (int64_t)c0 * gs[3];

  const TIO* up = reinterpret_cast<const TIO*>(args.u.p) + (int64_t)b * args.u.s[0] +
                  (int64_t)h * args.u.s[1] + (int64_t)c0 * args.u.s[3];
  TIO* dup = reinterpret_cast<TIO*>(args.du.p[0]) + (int64_t)b * args.du.s[0][0] +
             (int64_t)h * args.du.s[0][1] + (int64_t)c0 * args.du.s[0][3];
  const int64_t dus_t = args.du.s[0][2], dus_c = args.du.s[0][3];
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1];
  TIO* dlp = reinterpret_cast<TIO*>(const_cast<void*>(args.dlg.p)) + (int64_t)b * args.dlg.s[0] +
             (int64_t)h * args.dlg.s[1];
  const TIO* ip = reinterpret_cast<const TIO*>(args.init.p) + (int64_t)b * args.init.s[0] +
                  (int64_t)h * args.init.s[1] + (int64_t)c0 * args.init.s[3];
  TIO* dip = reinterpret_cast<TIO*>(const_cast<void*>(args.dinit.p)) + (int64_t)b * args.dinit.s[0] +
             (int64_t)h * args.dinit.s[1] + (int64_t)c0 * args.dinit.s[3];

  int gj[NA];
  float gbias[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    int c = c0 + (LANEGATE ? 0 : i);
    int j = lane_active ? min(c, S.D - 1) / S.r : 0;
    gj[i] = j;
    gbias[i] = args.bias[h * S.Da + j];
  }
  // this lane writes dlogit for group i when it leads it
  const bool leader = LANEGATE ? ((cl % group_lanes) == 0) : true;

  float carry[V];  // g at the first step after the current tile (g_T = 0)
#pragma unroll
  for (int v = 0; v < V; ++v) carry[v] = 0.0f;
  float dbias_acc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) dbias_acc[i] = 0.0f;

  __shared__ float lds_a[2][NW][CL][NA];
  __shared__ float lds_x[2][NW][CL][V];
  __shared__ float lds_db[NW * TG][CL][NA];

  constexpr int TW = NW * TG * L;
  const int ntiles = (S.T + TW - 1) / TW;
  const bool use_sig = S.use_sigmoid != 0;

  for (int it = ntiles - 1; it >= 0; --it) {
    const int t0 = it * TW + (w * TG + tg) * L;

    float gyv[L][V];
    float uv[L][V];
    float hpv[L][V];
    float al[L + 1][NA];
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const int t = t0 + s;
      const bool ok = lane_active && t < S.T;
      if (ok) {
        load_vec<TIO, VEC>(gp + (int64_t)t * gs[2], gs[3], nvalid, gyv[s]);
        load_vec<TIO, VEC>(up + (int64_t)t * args.u.s[2], args.u.s[3], nvalid, uv[s]);
        if (t == 0)
          load_vec<TIO, VEC>(ip, args.init.s[3], nvalid, hpv[s]);
        else
          load_vec<TIO, VEC>(hp + (int64_t)(t - 1) * hs[2], hs[3], nvalid, hpv[s]);
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          gyv[s][v] = 0.0f;
          uv[s][v] = 0.0f;
          hpv[s][v] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int s = 0; s <= L; ++s) {
      const int t = t0 + s;
      const bool ok = lane_active && t < S.T;
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        float raw = ok ? io_traits<TIO>::load(lp + (int64_t)t * args.lg.s[2] +
                                              (int64_t)gj[i] * args.lg.s[3])
                       : 0.0f;
        al[s][i] = ok ? gate_alpha(raw + gbias[i], use_sig) : 0.0f;
      }
    }
    // decay factor that carries g_{t+1} into g_t: a_{t+1} = 1 - alpha_{t+1};
    // zero past the end of the sequence (g_T = 0) and for padded steps.
    // level 1: lane-local reverse fold, (A, G): g_{t0} = A g_{t0+L} + G
    float A[NA], G[V];
#pragma unroll
    for (int i = 0; i < NA; ++i) A[i] = 1.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) G[v] = 0.0f;
#pragma unroll
    for (int s = L - 1; s >= 0; --s) {
      const bool ok = lane_active && (t0 + s) < S.T;
      const bool has_next = (t0 + s + 1) < S.T;
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const float an = (ok && has_next) ? (1.0f - al[s + 1][i]) : (ok ? 0.0f : 1.0f);
        // padded steps are the identity (A, G unchanged)
        if (ok) A[i] *= an;
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float an = has_next ? (1.0f - al[s + 1][LANEGATE ? 0 : v]) : 0.0f;
        if (ok) G[v] = gyv[s][v] + an * G[v];
      }
    }

    // level 2: inclusive suffix scan over the TG time-group lanes
#pragma unroll
    for (int off = 1; off < TG; off <<= 1) {
      float An[NA], Gn[V];
#pragma unroll
      for (int i = 0; i < NA; ++i) An[i] = __shfl_down(A[i], off, TG);
#pragma unroll
      for (int v = 0; v < V; ++v) Gn[v] = __shfl_down(G[v], off, TG);
      if (tg + off < TG) {
#pragma unroll
        for (int v = 0; v < V; ++v) G[v] = A[LANEGATE ? 0 : v] * Gn[v] + G[v];
#pragma unroll
        for (int i = 0; i < NA; ++i) A[i] *= An[i];
      }
    }
    float Ae[NA], Ge[V];  // exclusive suffix (lanes after this one)
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      float t = __shfl_down(A[i], 1, TG);
      Ae[i] = (tg == TG - 1) ? 1.0f : t;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float t = __shfl_down(G[v], 1, TG);
      Ge[v] = (tg == TG - 1) ? 0.0f : t;
    }

    // level 3: wavefront aggregates, composed from the last wavefront back
    float gin[V];
    if (NW > 1) {
      const int buf = it & 1;
      if (tg == 0) {
#pragma unroll
        for (int i = 0; i < NA; ++i) lds_a[buf][w][cl][i] = A[i];
#pragma unroll
        for (int v = 0; v < V; ++v) lds_x[buf][w][cl][v] = G[v];
      }
      __syncthreads();
      float cw[V];
#pragma unroll
      for (int v = 0; v < V; ++v) cw[v] = carry[v];
#pragma unroll
      for (int ww = NW - 1; ww >= 0; --ww) {
        if (ww == w) {
#pragma unroll
          for (int v = 0; v < V; ++v) gin[v] = cw[v];
        }
#pragma unroll
        for (int v = 0; v < V; ++v)
          cw[v] = lds_a[buf][ww][cl][LANEGATE ? 0 : v] * cw[v] + lds_x[buf][ww][cl][v];
      }
#pragma unroll
      for (int v = 0; v < V; ++v) carry[v] = cw[v];
    } else {
      float Aw[NA], Gw[V];
#pragma unroll
      for (int i = 0; i < NA; ++i) Aw[i] = __shfl(A[i], 0, TG);
#pragma unroll
      for (int v = 0; v < V; ++v) Gw[v] = __shfl(G[v], 0, TG);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        gin[v] = carry[v];
        carry[v] = Aw[LANEGATE ? 0 : v] * carry[v] + Gw[v];
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) gin[v] = Ae[LANEGATE ? 0 : v] * gin[v] + Ge[v];

    // re-run the lane's steps backwards from the exact carry-in
    float dl[L][NA];
#pragma unroll
    for (int s = L - 1; s >= 0; --s) {
      const int t = t0 + s;
      const bool ok = lane_active && t < S.T;
      const bool has_next = (t + 1) < S.T;
      float duv[V], dav[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int gi = LANEGATE ? 0 : v;
        const float an = has_next ? (1.0f - al[s + 1][gi]) : 0.0f;
        const float g = gyv[s][v] + an * gin[v];
        gin[v] = ok ? g : gin[v];
        const float alpha = al[s][gi];
        duv[v] = alpha * g;
        dav[v] = (uv[s][v] - hpv[s][v]) * g;
      }
      if (ok) {
        store_vec<TIO, VEC>(dup + (int64_t)t * dus_t, dus_c, nvalid, duv);
        if (t == 0) {
          float di[V];
#pragma unroll
          for (int v = 0; v < V; ++v) di[v] = (1.0f - al[s][LANEGATE ? 0 : v]) * gin[v];
          store_vec<TIO, VEC>(dip, args.dinit.s[3], nvalid, di);
        }
      }
      // per-group partial sums of dalpha over this lane's channels
      if (LANEGATE) {
        float p = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) p += (v < nvalid) ? dav[v] : 0.0f;
        dl[s][0] = ok ? p : 0.0f;
      } else {
#pragma unroll
        for (int i = 0; i < NA; ++i) dl[s][i] = 0.0f;
        // V / r groups of r channels each: group k holds channels k*r .. k*r+r-1
        for (int k = 0; k < groups_per_lane; ++k) {
          float p = 0.0f;
          for (int q = 0; q < S.r; ++q) {
            const int v = k * S.r + q;
#pragma unroll
            for (int vv = 0; vv < V; ++vv)
              if (vv == v) p += (vv < nvalid) ? dav[vv] : 0.0f;
          }
#pragma unroll
          for (int i = 0; i < NA; ++i)
            if (i == k) dl[s][i] = ok ? p : 0.0f;
        }
      }
    }
    // cross-lane reduction for groups that span lanes (butterfly over the
    // channel-lane bits inside the group: bitwise identical in every lane)
    if (LANEGATE) {
      for (int m = 1; m < group_lanes; m <<= 1) {
#pragma unroll
        for (int s = 0; s < L; ++s) dl[s][0] += __shfl_xor(dl[s][0], m * TG);
      }
    }
    // finish: sigmoid multiplier, store dlogit, accumulate dbias
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const int t = t0 + s;
      const bool ok = lane_active && t < S.T;
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        // a group exists when its first channel is a real channel of the head
        if (LANEGATE || (i < groups_per_lane && c0 + i * S.r < S.D)) {
          const int gi = LANEGATE ? 0 : i * S.r;  // decay slot of the group's first channel
          const float alpha = al[s][gi];
          const float d = use_sig ? dl[s][i] * (alpha * (1.0f - alpha)) : dl[s][i];
          if (ok && leader) {
            const int j = gj[gi];
            io_traits<TIO>::store(dlp + (int64_t)t * args.dlg.s[2] + (int64_t)j * args.dlg.s[3], d);
            dbias_acc[i] += d;
          }
        }
      }
    }
  }

  // dbias partial for (b, h): sum the leaders' accumulators in a fixed order
  const int tgw = w * TG + tg;
#pragma unroll
  for (int i = 0; i < NA; ++i) lds_db[tgw][cl][i] = (lane_active && leader) ? dbias_acc[i] : 0.0f;
  __syncthreads();
  for (int j = threadIdx.x; j < S.Da; j += NW * 64) {
    // gate j is led by channel lane (j * r) / V, decay slot (j * r) % V
    const int c = j * S.r;
    const int lcl = c / V;
    const int slot = LANEGATE ? 0 : (c % V) / S.r;
    float acc = 0.0f;
    for (int q = 0; q < NW * TG; ++q) acc += lds_db[q][lcl][slot];
    args.dbias_partial[((int64_t)b * S.H + h) * S.Da + j] = acc;
  }
}

// ---------------------------------------------------------------------------
// Generic backward for gate groups the main kernel cannot reduce in lanes
// (r neither divides V nor is V times a power of two).  One thread per
// (b, h, channel) walks T backwards; the per-channel dalpha terms go to an fp32
// workspace and a second kernel reduces each group in channel order.
// ---------------------------------------------------------------------------
template <typename TIO>
__global__ void scan_bwd_channel_kernel(const BwdArgs args, float* __restrict__ dalpha_ws) {
  const ScanShape& S = args.sh;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * S.D) return;
  const int c = (int)(idx % S.D);
  const int h = (int)((idx / S.D) % S.H);
  const int b = (int)(idx / ((int64_t)S.D * S.H));
  int which, hl;
  head_select(args.h, h, S.NH, S.NKVH, which, hl);
  const TIO* hp = reinterpret_cast<const TIO*>(args.h.p[which]) + (int64_t)b * args.h.s[which][0] +
                  (int64_t)hl * args.h.s[which][1] + (int64_t)c * args.h.s[which][3];
  const TIO* gp = reinterpret_cast<const TIO*>(args.gy.p[which]) + (int64_t)b * args.gy.s[which][0] +
                  (int64_t)hl * args.gy.s[which][1] + (int64_t)c * args.gy.s[which][3];
  const TIO* up = reinterpret_cast<const TIO*>(args.u.p) + (int64_t)b * args.u.s[0] +
                  (int64_t)h * args.u.s[1] + (int64_t)c * args.u.s[3];
  TIO* dup = reinterpret_cast<TIO*>(args.du.p[0]) + (int64_t)b * args.du.s[0][0] +
             (int64_t)h * args.du.s[0][1] + (int64_t)c * args.du.s[0][3];
  const int j = c / S.r;
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1] + (int64_t)j * args.lg.s[3];
  const float bias = args.bias[h * S.Da + j];
  const bool use_sig = S.use_sigmoid != 0;
  float g = 0.0f, a_next = 0.0f;
  for (int t = S.T - 1; t >= 0; --t) {
    const float alpha = gate_alpha(io_traits<TIO>::load(lp + (int64_t)t * args.lg.s[2]) + bias, use_sig);
    g = io_traits<TIO>::load(gp + (int64_t)t * args.gy.s[which][2]) + a_next * g;
    io_traits<TIO>::store(dup + (int64_t)t * args.du.s[0][2], alpha * g);
    float hprev;
    if (t == 0) {
      const TIO* ip = reinterpret_cast<const TIO*>(args.init.p) + (int64_t)b * args.init.s[0] +
                      (int64_t)h * args.init.s[1] + (int64_t)c * args.init.s[3];
      hprev = io_traits<TIO>::load(ip);
      TIO* dip = reinterpret_cast<TIO*>(const_cast<void*>(args.dinit.p)) + (int64_t)b * args.dinit.s[0] +
                 (int64_t)h * args.dinit.s[1] + (int64_t)c * args.dinit.s[3];
      io_traits<TIO>::store(dip, (1.0f - alpha) * g);
    } else {
      hprev = io_traits<TIO>::load(hp + (int64_t)(t - 1) * args.h.s[which][2]);
    }
    const float da = (io_traits<TIO>::load(up + (int64_t)t * args.u.s[2]) - hprev) * g;
    dalpha_ws[(((int64_t)b * S.H + h) * S.T + t) * S.D + c] = da;
    a_next = 1.0f - alpha;
  }
}

template <typename TIO>
__global__ void scan_bwd_group_reduce_kernel(const BwdArgs args, const float* __restrict__ dalpha_ws) {
  const ScanShape& S = args.sh;
  // one thread per (b, h, j) over all t, so dbias partials need no extra pass
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * S.Da) return;
  const int j = (int)(idx % S.Da);
  const int h = (int)((idx / S.Da) % S.H);
  const int b = (int)(idx / ((int64_t)S.Da * S.H));
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1] + (int64_t)j * args.lg.s[3];
  TIO* dlp = reinterpret_cast<TIO*>(const_cast<void*>(args.dlg.p)) + (int64_t)b * args.dlg.s[0] +
             (int64_t)h * args.dlg.s[1] + (int64_t)j * args.dlg.s[3];
  const float bias = args.bias[h * S.Da + j];
  const bool use_sig = S.use_sigmoid != 0;
  float acc_b = 0.0f;
  for (int t = 0; t < S.T; ++t) {
    const float* row = dalpha_ws + (((int64_t)b * S.H + h) * S.T + t) * S.D + (int64_t)j * S.r;
    float p = 0.0f;
    for (int q = 0; q < S.r; ++q) p += row[q];
    const float alpha = gate_alpha(io_traits<TIO>::load(lp + (int64_t)t * args.lg.s[2]) + bias, use_sig);
    const float d = use_sig ? p * (alpha * (1.0f - alpha)) : p;
    io_traits<TIO>::store(dlp + (int64_t)t * args.dlg.s[2], d);
    acc_b += d;
  }
  args.dbias_partial[idx] = acc_b;
}

// ---------------------------------------------------------------------------
// Host launchers (ltv_scan_fwd.hip / ltv_scan_bwd.hip)
// ---------------------------------------------------------------------------
constexpr int kScanL = 8;   // steps per lane per tile
constexpr int kScanNW = 4;  // wavefronts per workgroup

// Forward: grid = B * H * nslab workgroups of kScanNW * 64 threads.
int scan_launch_fwd(bool bf16, const FwdArgs& a, int CL, int grid, bool vec, bool lanegate,
                    hipStream_t st);
// Backward main kernel: grid = B * H, CL channel lanes cover the whole head.
int scan_launch_bwd(bool bf16, const BwdArgs& a, int CL, int grid, bool vec, bool lanegate,
                    hipStream_t st);
// Backward for gate groups outside the main kernel's reduction patterns.
int scan_launch_bwd_channel(bool bf16, const BwdArgs& a, float* dalpha_ws, hipStream_t st);
// dbias[h, j] = sum_b partial[b, h, j]
int scan_launch_dbias_reduce(const float* partial, float* dbias, int B, int HDa, hipStream_t st);

}  // namespace ltv

