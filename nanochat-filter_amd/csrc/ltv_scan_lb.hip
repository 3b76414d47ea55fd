// Look-back scan for short chunk windows: one lane per (b, head, window,
// channel vector), walking its window sequentially in registers.
//
// With chunks of Q steps and a K - 1 step warm-up (the reference's production
// layer spec is P = Q = 16, K = 9) a window spans Q + K - 1 steps: far less
// than a tile of the full-recurrence kernels, whose cross-lane scan levels and
// per-workgroup setup would then dominate.  Here the lanes of a wavefront are
// the channel vectors (fastest, so a step's loads are contiguous 16-byte
// vectors across lanes) of consecutive windows; a window's steps are walked
// by its lanes one after another, loads issued a batch at a time.
//
// Forward: each window runs h_t = h + alpha_t (u_t - h) from the inits over
// [lo, hi) and stores the outputs of [st, hi).
//
// Backward (the exact gradient; requires K - 1 <= Q, so a step is read by its
// own window and at most the next one's warm-up): the lane of window o owns
// the gradients of its steps [st, hi) and gathers both contributions:
//   g1 -- its own chain, g1_t = gy_t + (1 - alpha_{t+1}) g1_{t+1}, g1_hi = 0,
//         with the states h_{t-1}: the saved outputs inside the window, the
//         recomputed warm-up end state at t = st;
//   g2 -- window o + 1's chain on its warm-up [lo', st') = the tail of o:
//         g2_t = (1 - alpha_{t+1}) g2_{t+1} from g2_st' = G, the value of
//         o + 1's own chain at its first step (recomputed here from o + 1's
//         gy and gates), with o + 1's warm-up states recomputed from the inits.
//   du_t = alpha_t (g1_t + g2_t),  dalpha_t = (u_t - h_{t-1}) g1_t + (u_t - h'_{t-1}) g2_t
// and window o's own share of grad_inits, prod_{j=lo}^{st} (1 - alpha_j) g1_st,
// goes to a per-window fp32 slot (summed by scan_lb_dinit_kernel), dbias per
// (b, h, window) to the partial buffer (summed by dbias_reduce_kernel).  Every
// output element has exactly one writer: no atomics, no fold pass.
#include "ltv_scan_kernels.hpp"

namespace ltv {
namespace {

// Steps whose loads are issued together: per-channel gates load V logits per
// step, so their batches are shorter (register budget).
template <int GM>
constexpr int fwd_batch() {
  return GM == GATE_LANE ? 8 : 4;
}
template <int GM>
constexpr int bwd_batch() {
  return GM == GATE_LANE ? 4 : 2;
}

// Raw gate logits of step t (GATE_LANE: one value; per-channel modes: V values).
template <typename TIO, int GM>
struct GateRaw {
  static constexpr int V = Pack<TIO>::V;
  static constexpr int NA = GM == GATE_LANE ? 1 : V;
  float x[NA];
  __device__ __forceinline__ void load(const TIO* lp_t, const GateIdx<GM, V>& gi, bool ok,
                                       int nvalid) {
    if (GM == GATE_CHANVEC) {
      const uint4 q = ok ? *reinterpret_cast<const uint4*>(lp_t) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int v = 0; v < NA; ++v) x[v] = Pack<TIO>::get(q, v);
    } else {
#pragma unroll
      for (int i = 0; i < NA; ++i)
        x[i] = ok && (GM == GATE_LANE || i < nvalid) ? Pack<TIO>::load1(lp_t + gi.off[i]) : 0.0f;
    }
  }
  __device__ __forceinline__ void alpha(const GateIdx<GM, V>& gi, bool use_sig,
                                        float (&a)[NA]) const {
#pragma unroll
    for (int i = 0; i < NA; ++i) a[i] = gate_alpha(x[i] + gi.bias[i], use_sig);
  }
};

struct LaneMap {
  int cv, win;
  int64_t bh;
};

__device__ __forceinline__ LaneMap lane_map(int lanes, int nwin) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  LaneMap m;
  m.cv = (int)(gid % lanes);
  const int64_t rest = gid / lanes;
  m.win = (int)(rest % nwin);
  m.bh = rest / nwin;
  return m;
}

// Lanes per (b, h) in the buffer-addressed kernels: nwin x lanes rounded up to
// whole wavefronts, so that a wavefront never spans two (b, h) (lanes is a
// power of two: below 64 it divides 64, and a window never straddles
// wavefronts either); the padding lanes get win >= nwin.
__host__ __device__ inline int64_t lanes_per_bh(int lanes, int nwin) {
  return ((int64_t)nwin * lanes + 63) / 64 * 64;
}
__device__ __forceinline__ LaneMap lane_map_bh(int lanes, int nwin) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per = lanes_per_bh(lanes, nwin);
  const int64_t rest = gid % per;
  LaneMap m;
  m.bh = gid / per;
  m.win = (int)(rest / lanes);
  m.cv = (int)(rest % lanes);
  return m;
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <typename TIO, int GM, bool VEC>
__global__ void __launch_bounds__(256) scan_lb_short_fwd_kernel(const FwdArgs args) {
  constexpr int V = Pack<TIO>::V;
  constexpr int NA = GM == GATE_LANE ? 1 : V;
  constexpr bool GL = GM == GATE_LANE;
  constexpr int NB = fwd_batch<GM>();
  const ScanShape& S = args.sh;
  const LaneMap m = lane_map(args.lanes, args.nwin);
  if (m.bh >= (int64_t)S.B * S.H) return;
  const int h = (int)(m.bh % S.H), b = (int)(m.bh / S.H);
  const int c0 = m.cv * V;
  const int nvalid = min(V, S.D - c0);
  if (nvalid <= 0) return;
  const Window wd = look_back_window(m.win, S.T, args.P, args.Q, args.K);

  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView ov = head_view(args.out, which);
  TIO* outp = reinterpret_cast<TIO*>(ov.p) + (int64_t)b * ov.s[0] + (int64_t)hl * ov.s[1] +
              (int64_t)c0 * ov.s[3];
  const TIO* up = reinterpret_cast<const TIO*>(args.u.p) + (int64_t)b * args.u.s[0] +
                  (int64_t)h * args.u.s[1] + (int64_t)c0 * args.u.s[3];
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1];
  if (GM == GATE_CHANVEC) lp += (int64_t)c0;
  GateIdx<GM, V> gi;
  gi.init(args.bias + h * S.Da, c0, nvalid, S.D, S.r, args.lg.s[3]);
  const bool use_sig = S.use_sigmoid != 0;
  const int64_t ust = args.u.s[2], usc = args.u.s[3], lst = args.lg.s[2];

  float hv[V];
  {
    const TIO* ip = reinterpret_cast<const TIO*>(args.init.p) + (int64_t)b * args.init.s[0] +
                    (int64_t)h * args.init.s[1] + (int64_t)c0 * args.init.s[3];
    const uint4 q = ld_vec<TIO, VEC>(ip, args.init.s[3], nvalid);
#pragma unroll
    for (int v = 0; v < V; ++v) hv[v] = Pack<TIO>::get(q, v);
  }
  for (int t0 = wd.lo; t0 < wd.hi; t0 += NB) {
    uint4 uq[NB];
    GateRaw<TIO, GM> gr[NB];
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int t = t0 + s;
      const bool ok = t < wd.hi;
      uq[s] = ok ? ld_vec<TIO, VEC>(up + (int64_t)t * ust, usc, nvalid) : make_uint4(0u, 0u, 0u, 0u);
      gr[s].load(lp + (int64_t)t * lst, gi, ok, nvalid);
    }
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int t = t0 + s;
      if (t < wd.hi) {
        float a[NA];
        gr[s].alpha(gi, use_sig, a);
#pragma unroll
        for (int v = 0; v < V; ++v) hv[v] = fmaf(a[GL ? 0 : v], Pack<TIO>::get(uq[s], v) - hv[v], hv[v]);
        if (t >= wd.st) st_vec<TIO, VEC>(outp + (int64_t)t * ov.s[2], ov.s[3], nvalid, hv);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
// Sum of x over the aligned groups of `gl` adjacent lanes (gl a power of two).
__device__ __forceinline__ float group_sum(float x, int gl) {
  for (int m = 1; m < gl; m <<= 1) x += __shfl_xor(x, m, 64);
  return x;
}

template <typename TIO, int GM, bool VEC, int KW>
__global__ void __launch_bounds__(256) scan_lb_short_bwd_kernel(const BwdArgs args) {
  constexpr int V = Pack<TIO>::V;
  constexpr int NA = GM == GATE_LANE ? 1 : V;
  constexpr bool GL = GM == GATE_LANE;
  constexpr int NB = bwd_batch<GM>();
  const ScanShape& S = args.sh;
  const int nwin = args.nchunk;
  const LaneMap m = lane_map(args.lanes, nwin);
  // a window's lanes are consecutive and share bh: whole gate groups leave together
  if (m.bh >= (int64_t)S.B * S.H) return;
  const int h = (int)(m.bh % S.H), b = (int)(m.bh / S.H);
  const int c0 = m.cv * V;
  const int nvalid = min(V, S.D - c0);
  const bool active = nvalid > 0;
  const int gl = GL ? S.r / V : 1;  // lanes per gate group (GATE_LANE)

  const Window wd = look_back_window(m.win, S.T, args.P, args.Q, args.K);
  const bool has_next = m.win + 1 < nwin;
  Window wn;
  if (has_next) {
    wn = look_back_window(m.win + 1, S.T, args.P, args.Q, args.K);
  } else {
    wn.lo = wn.st = wn.hi = wd.hi;
  }

  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView hvw = head_view(args.h, which), gvw = head_view(args.gy, which);
  const TIO* hp = reinterpret_cast<const TIO*>(hvw.p) + (int64_t)b * hvw.s[0] +
                  (int64_t)hl * hvw.s[1] + (int64_t)c0 * hvw.s[3];
  const TIO* gp = reinterpret_cast<const TIO*>(gvw.p) + (int64_t)b * gvw.s[0] +
                  (int64_t)hl * gvw.s[1] + (int64_t)c0 * gvw.s[3];
  const TIO* up = reinterpret_cast<const TIO*>(args.u.p) + (int64_t)b * args.u.s[0] +
                  (int64_t)h * args.u.s[1] + (int64_t)c0 * args.u.s[3];
  TIO* dup = reinterpret_cast<TIO*>(const_cast<void*>(args.du.p)) + (int64_t)b * args.du.s[0] +
             (int64_t)h * args.du.s[1] + (int64_t)c0 * args.du.s[3];
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1];
  TIO* dlp = reinterpret_cast<TIO*>(const_cast<void*>(args.dlg.p)) + (int64_t)b * args.dlg.s[0] +
             (int64_t)h * args.dlg.s[1];
  if (GM == GATE_CHANVEC) lp += (int64_t)c0;
  GateIdx<GM, V> gi;
  gi.init(args.bias + h * S.Da, c0, nvalid, S.D, S.r, args.lg.s[3]);
  const bool use_sig = S.use_sigmoid != 0;
  const int64_t ust = args.u.s[2], usc = args.u.s[3], lst = args.lg.s[2];
  const int64_t hst = hvw.s[2], hsc = hvw.s[3], gst = gvw.s[2], gsc = gvw.s[3];
  const int64_t dust = args.du.s[2], dusc = args.du.s[3];
  const int64_t dlst = args.dlg.s[2], dlsc = args.dlg.s[3];

  float ini[V];
  {
    const TIO* ip = reinterpret_cast<const TIO*>(args.init.p) + (int64_t)b * args.init.s[0] +
                    (int64_t)h * args.init.s[1] + (int64_t)c0 * args.init.s[3];
    const uint4 q = active ? ld_vec<TIO, VEC>(ip, args.init.s[3], nvalid) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int v = 0; v < V; ++v) ini[v] = Pack<TIO>::get(q, v);
  }

  // ---- (A1) own warm-up [lo, st): the state entering st and prod (1 - alpha)
  float h1[V], prodw[NA];
#pragma unroll
  for (int v = 0; v < V; ++v) h1[v] = ini[v];
#pragma unroll
  for (int i = 0; i < NA; ++i) prodw[i] = 1.0f;
  for (int t0 = wd.lo; t0 < wd.st; t0 += NB) {
    uint4 uq[NB];
    GateRaw<TIO, GM> gr[NB];
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int t = t0 + s;
      const bool ok = active && t < wd.st;
      uq[s] = ok ? ld_vec<TIO, VEC>(up + (int64_t)t * ust, usc, nvalid) : make_uint4(0u, 0u, 0u, 0u);
      gr[s].load(lp + (int64_t)t * lst, gi, ok, nvalid);
    }
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      if (t0 + s < wd.st) {
        float a[NA];
        gr[s].alpha(gi, use_sig, a);
#pragma unroll
        for (int v = 0; v < V; ++v) h1[v] = fmaf(a[GL ? 0 : v], Pack<TIO>::get(uq[s], v) - h1[v], h1[v]);
#pragma unroll
        for (int i = 0; i < NA; ++i) prodw[i] *= 1.0f - a[i];
      }
    }
  }
  const uint4 h_st = Pack<TIO>::pack(h1);  // I/O-rounded, as the saved outputs

  // ---- (A2) the next window's warm-up states: HN[s] enters step wn.lo + s
  const int nt = wn.st - wn.lo;  // tail steps of this window read by the next (<= KW)
  uint4 HN[KW];
  {
    float hn[V];
#pragma unroll
    for (int v = 0; v < V; ++v) hn[v] = ini[v];
    uint4 uq[KW];
    GateRaw<TIO, GM> gr[KW];
#pragma unroll
    for (int s = 0; s < KW; ++s) {
      const int t = wn.lo + s;
      const bool ok = active && s < nt;
      uq[s] = ok ? ld_vec<TIO, VEC>(up + (int64_t)t * ust, usc, nvalid) : make_uint4(0u, 0u, 0u, 0u);
      gr[s].load(lp + (int64_t)t * lst, gi, ok, nvalid);
    }
#pragma unroll
    for (int s = 0; s < KW; ++s) {
      HN[s] = Pack<TIO>::pack(hn);
      if (s < nt) {
        float a[NA];
        gr[s].alpha(gi, use_sig, a);
#pragma unroll
        for (int v = 0; v < V; ++v) hn[v] = fmaf(a[GL ? 0 : v], Pack<TIO>::get(uq[s], v) - hn[v], hn[v]);
      }
    }
  }

  // ---- (G) the next window's own chain at its first step, and 1 - alpha there
  float G[V], a_hi[NA];
#pragma unroll
  for (int v = 0; v < V; ++v) G[v] = 0.0f;
#pragma unroll
  for (int i = 0; i < NA; ++i) a_hi[i] = 0.0f;
  for (int tb = wn.hi; tb > wn.st; tb -= NB) {
    uint4 gq[NB];
    GateRaw<TIO, GM> gr[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int t = tb - 1 - k;
      const bool ok = active && t >= wn.st;
      gq[k] = ok ? ld_vec<TIO, VEC>(gp + (int64_t)t * gst, gsc, nvalid) : make_uint4(0u, 0u, 0u, 0u);
      gr[k].load(lp + (int64_t)t * lst, gi, ok, nvalid);
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      if (tb - 1 - k >= wn.st) {
        // a_hi holds 1 - alpha_{t+1} (0 past the window's last step)
#pragma unroll
        for (int v = 0; v < V; ++v) G[v] = fmaf(a_hi[GL ? 0 : v], G[v], Pack<TIO>::get(gq[k], v));
        float a[NA];
        gr[k].alpha(gi, use_sig, a);
#pragma unroll
        for (int i = 0; i < NA; ++i) a_hi[i] = 1.0f - a[i];
      }
    }
  }

  // ---- (B) own steps in reverse: g1 (own chain) and g2 (next window's warm-up)
  float g1[V], g2[V], an[NA];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    g1[v] = 0.0f;
    g2[v] = G[v];
  }
#pragma unroll
  for (int i = 0; i < NA; ++i) an[i] = a_hi[i];
  float dacc[GL ? 1 : V];
#pragma unroll
  for (int k = 0; k < (GL ? 1 : V); ++k) dacc[k] = 0.0f;

  // one reverse step at t; with_g2: t lies in the next window's warm-up, hn its state
  auto step = [&](int t, const uint4& gq, const uint4& uq, const uint4& hq, const GateRaw<TIO, GM>& gr,
                  bool with_g2, const uint4& hn) {
    float a[NA];
    gr.alpha(gi, use_sig, a);
    float duv[V], dav[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int ia = GL ? 0 : v;
      g1[v] = fmaf(an[ia], g1[v], Pack<TIO>::get(gq, v));
      g2[v] = with_g2 ? an[ia] * g2[v] : 0.0f;
      const float u = Pack<TIO>::get(uq, v);
      duv[v] = a[ia] * (g1[v] + g2[v]);
      dav[v] = (u - Pack<TIO>::get(hq, v)) * g1[v];
      if (with_g2) dav[v] = fmaf(u - Pack<TIO>::get(hn, v), g2[v], dav[v]);
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) an[i] = 1.0f - a[i];
    if (active) st_vec<TIO, VEC>(dup + (int64_t)t * dust, dusc, nvalid, duv);
    if (GL) {
      float p = 0.0f;
#pragma unroll
      for (int v = 0; v < V; ++v) p += v < nvalid ? dav[v] : 0.0f;
      p = group_sum(p, gl);
      const float d = use_sig ? p * (a[0] * (1.0f - a[0])) : p;
      if (active && (m.cv % gl) == 0) {
        dacc[0] += d;
        Pack<TIO>::store1(dlp + (int64_t)t * dlst + (int64_t)(c0 / S.r) * dlsc, d);
      }
    } else {
      // whole groups of r channels inside the lane (r | V)
#pragma unroll
      for (int mm = 1; mm < V; mm <<= 1) {
        if (mm < S.r) {
          float tsum[V];
#pragma unroll
          for (int v = 0; v < V; ++v) tsum[v] = dav[v] + dav[v ^ mm];
#pragma unroll
          for (int v = 0; v < V; ++v) dav[v] = tsum[v];
        }
      }
      float dl[V];
#pragma unroll
      for (int v = 0; v < V; ++v) dl[v] = use_sig ? dav[v] * (a[v] * (1.0f - a[v])) : dav[v];
      if (active) {
        if (GM == GATE_CHANVEC) {
          st_vec<TIO, true>(dlp + (int64_t)t * dlst + c0, 1, V, dl);
#pragma unroll
          for (int v = 0; v < V; ++v) dacc[v] += dl[v];
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if ((v & (S.r - 1)) == 0 && v < nvalid) {
              dacc[v] += dl[v];
              Pack<TIO>::store1(dlp + (int64_t)t * dlst + (int64_t)((c0 + v) / S.r) * dlsc, dl[v]);
            }
          }
        }
      }
    }
  };
  // state entering step t of this window: the saved output of t - 1, or at st
  // the recomputed warm-up end state
  auto load_h = [&](int t, bool ok) -> uint4 {
    if (!ok) return make_uint4(0u, 0u, 0u, 0u);
    return t == wd.st ? h_st : ld_vec<TIO, VEC>(hp + (int64_t)(t - 1) * hst, hsc, nvalid);
  };

  // (B1) the tail [wn.lo, wn.st), read by the next window: compile-time rows of
  // HN, in batches of NB steps whose loads are issued together
#pragma unroll
  for (int s0 = KW - NB; s0 >= 0; s0 -= NB) {
    uint4 gq[NB], uq[NB], hq[NB];
    GateRaw<TIO, GM> gr[NB];
#pragma unroll
    for (int k = NB - 1; k >= 0; --k) {
      const int t = wn.lo + s0 + k;
      const bool ok = active && s0 + k < nt;
      gq[k] = ok ? ld_vec<TIO, VEC>(gp + (int64_t)t * gst, gsc, nvalid) : make_uint4(0u, 0u, 0u, 0u);
      uq[k] = ok ? ld_vec<TIO, VEC>(up + (int64_t)t * ust, usc, nvalid) : make_uint4(0u, 0u, 0u, 0u);
      hq[k] = load_h(t, ok);
      gr[k].load(lp + (int64_t)t * lst, gi, ok, nvalid);
    }
#pragma unroll
    for (int k = NB - 1; k >= 0; --k)
      if (s0 + k < nt) step(wn.lo + s0 + k, gq[k], uq[k], hq[k], gr[k], true, HN[s0 + k]);
  }
  // (B2) the rest [st, wn.lo), batches in reverse
  const int b2_hi = has_next ? wn.lo : wd.hi;
  for (int tb = b2_hi; tb > wd.st; tb -= NB) {
    uint4 gq[NB], uq[NB], hq[NB];
    GateRaw<TIO, GM> gr[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int t = tb - 1 - k;
      const bool ok = active && t >= wd.st;
      gq[k] = ok ? ld_vec<TIO, VEC>(gp + (int64_t)t * gst, gsc, nvalid) : make_uint4(0u, 0u, 0u, 0u);
      uq[k] = ok ? ld_vec<TIO, VEC>(up + (int64_t)t * ust, usc, nvalid) : make_uint4(0u, 0u, 0u, 0u);
      hq[k] = load_h(t, ok);
      gr[k].load(lp + (int64_t)t * lst, gi, ok, nvalid);
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int t = tb - 1 - k;
      if (t >= wd.st) step(t, gq[k], uq[k], hq[k], gr[k], false, h_st);
    }
  }

  // ---- this window's share of grad_inits: prod_{j=lo}^{st} (1 - alpha_j) g1_st
  // (an = 1 - alpha_st after the last step; an empty window leaves g1 = 0)
  if (active) {
    float di[V];
#pragma unroll
    for (int v = 0; v < V; ++v) di[v] = prodw[GL ? 0 : v] * an[GL ? 0 : v] * g1[v];
    st_f32<VEC, V>(args.wdi + ((int64_t)m.bh * nwin + m.win) * S.D + c0, nvalid, di);
  }
  // ---- dbias partial of (b, h, window)
  float* pp = args.dbias_partial + ((int64_t)m.bh * nwin + m.win) * S.Da;
  if (GL) {
    if (active && (m.cv % gl) == 0) pp[c0 / S.r] = dacc[0];
  } else if (active) {
#pragma unroll
    for (int v = 0; v < V; ++v)
      if ((GM == GATE_CHANVEC || (v & (S.r - 1)) == 0) && v < nvalid) pp[(c0 + v) / S.r] = dacc[v];
  }
}

// ---------------------------------------------------------------------------
// Buffer-addressed versions (used when every view spans less than 2^31 bytes):
// each access is a buffer instruction on the tensor's base with a 32-bit lane
// offset, masked lanes pass kOob, the steps are branch-free (a masked step
// leaves the carried state unchanged) and the step loops run a wave-uniform
// number of batches with the next batch's loads in flight.  With loads and
// stores under branches, or loops with per-lane trip counts, the compiler waits
// for every outstanding memory operation at each use: these kernels spent
// three quarters of their time waiting.
// ---------------------------------------------------------------------------

// Buffer resource over a view's (b, h) slice (wave-uniform: the launcher uses
// these kernels only when every wavefront lies in one (b, h)), and a lane's
// byte offset of channel c at t = 0 in it.
template <class VW>
__device__ __forceinline__ Rsrc slice_rsrc(const VW& v, int b, int h, int esize) {
  return make_rsrc(reinterpret_cast<const char*>(v.p) +
                   ((int64_t)b * v.s[0] + (int64_t)h * v.s[1]) * esize);
}
template <class VW>
__device__ __forceinline__ uint32_t chan_off(const VW& v, int c, int esize) {
  return (uint32_t)((int64_t)c * v.s[3] * esize);
}

// maximum over the wavefront (every lane active)
__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = max(x, __shfl_xor(x, m, 64));
  return __builtin_amdgcn_readfirstlane(x);
}

// sum over aligned groups of gl adjacent lanes (gl a power of two <= 64), with
// fixed levels and masked adds (no loop or branch around the shuffles)
__device__ __forceinline__ float group_sum_fixed(float x, int gl) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float y = __shfl_xor(x, m, 64);
    x += m < gl ? y : 0.0f;
  }
  return x;
}

template <typename TIO, int GM, bool VEC>
__global__ void __launch_bounds__(256) scan_lb_buf_fwd_kernel(const FwdArgs args) {
  constexpr int V = Pack<TIO>::V;
  constexpr int NA = GM == GATE_LANE ? 1 : V;
  constexpr bool GL = GM == GATE_LANE;
  constexpr int NB = fwd_batch<GM>();
  constexpr int E = sizeof(TIO);
  const ScanShape& S = args.sh;
  const LaneMap m = lane_map_bh(args.lanes, args.nwin);
  const int bhu = __builtin_amdgcn_readfirstlane(
      (int)(m.bh < (int64_t)S.B * S.H ? m.bh : (int64_t)S.B * S.H));
  const bool in_grid = bhu < S.B * S.H;
  const int bhc = in_grid ? bhu : 0;
  const int h = bhc % S.H, b = bhc / S.H;
  const int c0 = m.cv * V;
  const int nvalid = min(V, S.D - c0);
  const bool active = in_grid && m.win < args.nwin && nvalid > 0;
  const Window wd = look_back_window(m.win, S.T, args.P, args.Q, args.K);
  const int nbatch = (wave_max(active ? wd.hi - wd.lo : 0) + NB - 1) / NB;

  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView ov = head_view(args.out, which);
  const Rsrc ur = slice_rsrc(args.u, b, h, E), lr = slice_rsrc(args.lg, b, h, E),
             orr = slice_rsrc(ov, b, hl, E);
  const uint32_t ustb = (uint32_t)(args.u.s[2] * E), uscb = (uint32_t)(args.u.s[3] * E);
  const uint32_t lstb = (uint32_t)(args.lg.s[2] * E);
  const uint32_t ostb = (uint32_t)(ov.s[2] * E), oscb = (uint32_t)(ov.s[3] * E);
  const uint32_t ub = chan_off(args.u, c0, E);
  const uint32_t lb = GM == GATE_CHANVEC ? chan_off(args.lg, c0, E) : 0u;
  const uint32_t ob = chan_off(ov, c0, E);
  GateIdx<GM, V> gi;
  gi.init(args.bias + h * S.Da, c0, nvalid, S.D, S.r, args.lg.s[3]);
  const bool use_sig = S.use_sigmoid != 0;

  float hv[V];
  {
    // fp32 inits (with bf16 values) are rounded to bf16 as they are read
    const int EI = args.init_f32 ? 4 : E;
    const uint4 q = bld_init<TIO, VEC>(slice_rsrc(args.init, b, h, EI), chan_off(args.init, c0, EI),
                                       (uint32_t)(args.init.s[3] * EI), nvalid, active,
                                       args.init_f32 != 0);
#pragma unroll
    for (int v = 0; v < V; ++v) hv[v] = Pack<TIO>::get(q, v);
  }
  uint4 nu[2][NB];
  LogitRaw<TIO, GM, NB> nl[2];
  auto load = [&](int k, auto bufc) __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value;
    const int t0 = wd.lo + k * NB;
#pragma unroll
    for (int s = 0; s < NB; ++s)
      nu[buf][s] = bld_vec<TIO, VEC>(ur, ub + (uint32_t)(t0 + s) * ustb, uscb, nvalid,
                                     active && t0 + s < wd.hi);
    nl[buf].template load<true>(lr, lb + (uint32_t)t0 * lstb, lstb, gi, t0, wd.hi, active, nvalid);
  };
  auto process = [&](int k, auto bufc) __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value;
    const int t0 = wd.lo + k * NB;
    uint4 uq[NB];
#pragma unroll
    for (int s = 0; s < NB; ++s) uq[s] = nu[buf][s];
    float al[NB][NA];
    nl[buf].gates(gi, t0, wd.hi, active, use_sig, al);  // 0 (the identity) when masked
    load(k + 1, std::integral_constant<int, 1 - buf>{});
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int t = t0 + s;
#pragma unroll
      for (int v = 0; v < V; ++v)
        hv[v] = fmaf(al[s][GL ? 0 : v], Pack<TIO>::get(uq[s], v) - hv[v], hv[v]);
      bst_vec<TIO, VEC>(orr, ob + (uint32_t)t * ostb, oscb, nvalid,
                        active && t >= wd.st && t < wd.hi, hv);
    }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  load(0, B0{});
  for (int k = 0; k < nbatch; k += 2) {
    process(k, B0{});
    if (k + 1 < nbatch) process(k + 1, B1{});
  }
}

template <typename TIO, int GM, bool VEC, int KW>
__global__ void __launch_bounds__(256) scan_lb_buf_bwd_kernel(const BwdArgs args) {
  constexpr int V = Pack<TIO>::V;
  constexpr int NA = GM == GATE_LANE ? 1 : V;
  constexpr bool GL = GM == GATE_LANE;
  constexpr int NB = bwd_batch<GM>();
  constexpr int E = sizeof(TIO);
  static_assert(KW % NB == 0, "warm-up rows in whole batches");
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  const ScanShape& S = args.sh;
  const int nwin = args.nchunk;
  const LaneMap m = lane_map_bh(args.lanes, nwin);
  const int bhu = __builtin_amdgcn_readfirstlane(
      (int)(m.bh < (int64_t)S.B * S.H ? m.bh : (int64_t)S.B * S.H));
  const bool in_grid = bhu < S.B * S.H;
  const int bhc = in_grid ? bhu : 0;
  const int h = bhc % S.H, b = bhc / S.H;
  const int c0 = m.cv * V;
  const int nvalid = min(V, S.D - c0);
  const bool active = in_grid && m.win < nwin && nvalid > 0;
  const int gl = GL ? S.r / V : 1;  // lanes per gate group (GATE_LANE)

  const Window wd = look_back_window(m.win, S.T, args.P, args.Q, args.K);
  const bool has_next = m.win + 1 < nwin;
  // the last window has an empty successor at wd.hi; selected without a branch
  // and kept opaque, so the compiler does not specialise the loads on it
  Window wn;
  {
    const Window wr = look_back_window(m.win + 1, S.T, args.P, args.Q, args.K);
    wn.lo = (int)opaque((uint32_t)(has_next ? wr.lo : wd.hi));
    wn.st = (int)opaque((uint32_t)(has_next ? wr.st : wd.hi));
    wn.hi = (int)opaque((uint32_t)(has_next ? wr.hi : wd.hi));
  }
  const int nt = wn.st - wn.lo;  // tail steps of this window read by the next (<= KW)
  const int b2_hi = has_next ? wn.lo : wd.hi;
  // wave-uniform batch counts of the runtime-length phases
  const int nb_g = (wave_max(active ? wn.hi - wn.st : 0) + NB - 1) / NB;
  const int nb_b2 = (wave_max(active ? b2_hi - wd.st : 0) + NB - 1) / NB;

  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView hvw = head_view(args.h, which), gvw = head_view(args.gy, which);
  const Rsrc ur = slice_rsrc(args.u, b, h, E), lr = slice_rsrc(args.lg, b, h, E),
             hr = slice_rsrc(hvw, b, hl, E), gr = slice_rsrc(gvw, b, hl, E),
             dur = slice_rsrc(args.du, b, h, E), dlr = slice_rsrc(args.dlg, b, h, E);
  const uint32_t ustb = (uint32_t)(args.u.s[2] * E), uscb = (uint32_t)(args.u.s[3] * E);
  const uint32_t lstb = (uint32_t)(args.lg.s[2] * E);
  const uint32_t hstb = (uint32_t)(hvw.s[2] * E), hscb = (uint32_t)(hvw.s[3] * E);
  const uint32_t gstb = (uint32_t)(gvw.s[2] * E), gscb = (uint32_t)(gvw.s[3] * E);
  const uint32_t dustb = (uint32_t)(args.du.s[2] * E), duscb = (uint32_t)(args.du.s[3] * E);
  const uint32_t dlstb = (uint32_t)(args.dlg.s[2] * E), dlscb = (uint32_t)(args.dlg.s[3] * E);
  const uint32_t ub = chan_off(args.u, c0, E);
  const uint32_t lb = GM == GATE_CHANVEC ? chan_off(args.lg, c0, E) : 0u;
  const uint32_t hb = chan_off(hvw, c0, E), gb = chan_off(gvw, c0, E);
  const uint32_t dub = chan_off(args.du, c0, E);
  const uint32_t dlb = 0u;
  GateIdx<GM, V> gi;
  gi.init(args.bias + h * S.Da, c0, nvalid, S.D, S.r, args.lg.s[3]);
  const bool use_sig = S.use_sigmoid != 0;

  float ini[V];
  {
    // fp32 inits (with bf16 values) are rounded to bf16 as they are read
    const int EI = args.init_f32 ? 4 : E;
    const uint4 q = bld_init<TIO, VEC>(slice_rsrc(args.init, b, h, EI), chan_off(args.init, c0, EI),
                                       (uint32_t)(args.init.s[3] * EI), nvalid, active,
                                       args.init_f32 != 0);
#pragma unroll
    for (int v = 0; v < V; ++v) ini[v] = Pack<TIO>::get(q, v);
  }

  // ---- (A1) own warm-up [lo, st) (at most KW steps): the state entering st
  // and prod (1 - alpha); (A2) the next window's warm-up states: HN[s] enters
  // step wn.lo + s.  Batches of NB steps, the next batch's loads in flight.
  float h1[V], prodw[NA];
#pragma unroll
  for (int v = 0; v < V; ++v) h1[v] = ini[v];
#pragma unroll
  for (int i = 0; i < NA; ++i) prodw[i] = 1.0f;
  uint4 HN[KW];
  {
    float hn[V];
#pragma unroll
    for (int v = 0; v < V; ++v) hn[v] = ini[v];
    // the two warm-ups as one sequence of 2 KW / NB batches: batches [0, KW / NB)
    // walk [lo, lo + KW), the rest [wn.lo, wn.lo + KW)
    constexpr int NBW = KW / NB;
    uint4 wu[2][NB];
    LogitRaw<TIO, GM, NB> wl[2];
    auto wload = [&](int k, auto bufc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      const bool own = k < NBW;
      const int t0 = own ? wd.lo + k * NB : wn.lo + (k - NBW) * NB;
      const int tend = own ? wd.st : wn.st;
#pragma unroll
      for (int s = 0; s < NB; ++s)
        wu[buf][s] = bld_vec<TIO, VEC>(ur, ub + (uint32_t)(t0 + s) * ustb, uscb, nvalid,
                                       active && k < 2 * NBW && t0 + s < tend);
      wl[buf].template load<true>(lr, lb + (uint32_t)t0 * lstb, lstb, gi, t0, tend, active && k < 2 * NBW, nvalid);
    };
    auto wstep = [&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      constexpr int buf = k & 1;
      constexpr bool own = k < NBW;
      const int t0 = own ? wd.lo + k * NB : wn.lo + (k - NBW) * NB;
      const int tend = own ? wd.st : wn.st;
      uint4 uq[NB];
#pragma unroll
      for (int s = 0; s < NB; ++s) uq[s] = wu[buf][s];
      float al[NB][NA];
      wl[buf].gates(gi, t0, tend, active, use_sig, al);  // 0 when masked: the identity step
      wload(k + 1, std::integral_constant<int, 1 - buf>{});
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        if constexpr (own) {
#pragma unroll
          for (int v = 0; v < V; ++v)
            h1[v] = fmaf(al[s][GL ? 0 : v], Pack<TIO>::get(uq[s], v) - h1[v], h1[v]);
#pragma unroll
          for (int i = 0; i < NA; ++i) prodw[i] *= 1.0f - al[s][i];
        } else {
          HN[(k - NBW) * NB + s] = Pack<TIO>::pack(hn);
#pragma unroll
          for (int v = 0; v < V; ++v)
            hn[v] = fmaf(al[s][GL ? 0 : v], Pack<TIO>::get(uq[s], v) - hn[v], hn[v]);
        }
      }
    };
    wload(0, B0{});
    static_loop<0, 2 * NBW>(wstep);
  }
  const uint4 h_st = Pack<TIO>::pack(h1);  // I/O-rounded, as the saved outputs

  // ---- (G) the next window's own chain at its first step, and 1 - alpha there,
  // walking [wn.st, wn.hi) in reverse; a_hi holds 1 - alpha_{t+1} (0 past the
  // window's last step), masked steps leave both unchanged
  float G[V], a_hi[NA];
#pragma unroll
  for (int v = 0; v < V; ++v) G[v] = 0.0f;
#pragma unroll
  for (int i = 0; i < NA; ++i) a_hi[i] = 0.0f;
  {
    uint4 ng[2][NB];
    LogitRaw<TIO, GM, NB> nl[2];
    // batch k covers t = wn.hi - 1 - (k NB + j), j = 0..NB-1 (loads ascending in t)
    auto gload = [&](int k, auto bufc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      const int tl = wn.hi - (k + 1) * NB;  // lowest step of the batch
#pragma unroll
      for (int s = 0; s < NB; ++s)
        ng[buf][s] = bld_vec<TIO, VEC>(gr, gb + (uint32_t)(tl + s) * gstb, gscb, nvalid,
                                       active && k < nb_g && tl + s >= wn.st);
      nl[buf].template load<true>(lr, lb + (uint32_t)tl * lstb, lstb, gi, tl, wn.hi,
                   active && k < nb_g, nvalid, wn.st);
    };
    auto gstep = [&](int k, auto bufc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      const int tl = wn.hi - (k + 1) * NB;
      uint4 gq[NB];
#pragma unroll
      for (int s = 0; s < NB; ++s) gq[s] = ng[buf][s];
      float al[NB][NA];
      nl[buf].gates(gi, tl, wn.hi, active, use_sig, al);
      gload(k + 1, std::integral_constant<int, 1 - buf>{});
#pragma unroll
      for (int s = NB - 1; s >= 0; --s) {
        const bool ok = active && tl + s >= wn.st;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float gn = fmaf(a_hi[GL ? 0 : v], G[v], Pack<TIO>::get(gq[s], v));
          G[v] = ok ? gn : G[v];
        }
#pragma unroll
        for (int i = 0; i < NA; ++i) a_hi[i] = ok ? 1.0f - al[s][i] : a_hi[i];
      }
    };
    gload(0, B0{});
    for (int k = 0; k < nb_g; k += 2) {
      gstep(k, B0{});
      if (k + 1 < nb_g) gstep(k + 1, B1{});
    }
  }

  // ---- (B) own steps in reverse: g1 (own chain) and g2 (next window's warm-up)
  float g1[V], g2[V], an[NA];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    g1[v] = 0.0f;
    g2[v] = G[v];
  }
#pragma unroll
  for (int i = 0; i < NA; ++i) an[i] = a_hi[i];
  float dacc[GL ? 1 : V];
#pragma unroll
  for (int k = 0; k < (GL ? 1 : V); ++k) dacc[k] = 0.0f;
  const int gjl = GL ? c0 / S.r : 0;  // gate group of this lane (GATE_LANE)
  const bool glead = GL && active && (m.cv % gl) == 0;

  // one reverse step at t (branch-free; a masked step changes nothing); with_g2:
  // t lies in the next window's warm-up, hn its state
  auto step = [&](int t, bool ok, const uint4& gq, const uint4& uq, const uint4& hq,
                  const float (&a)[NA], bool with_g2, const uint4& hn) {
    float duv[V], dav[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int ia = GL ? 0 : v;
      const float g1n = fmaf(an[ia], g1[v], Pack<TIO>::get(gq, v));
      const float g2n = with_g2 ? an[ia] * g2[v] : 0.0f;
      g1[v] = ok ? g1n : g1[v];
      g2[v] = ok ? g2n : g2[v];
      const float u = Pack<TIO>::get(uq, v);
      duv[v] = a[ia] * (g1n + g2n);
      dav[v] = (u - Pack<TIO>::get(hq, v)) * g1n;
      if (with_g2) dav[v] = fmaf(u - Pack<TIO>::get(hn, v), g2n, dav[v]);
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) an[i] = ok ? 1.0f - a[i] : an[i];
    bst_vec<TIO, VEC>(dur, dub + (uint32_t)t * dustb, duscb, nvalid, ok, duv);
    if (GL) {
      float p = 0.0f;
#pragma unroll
      for (int v = 0; v < V; ++v) p += v < nvalid ? dav[v] : 0.0f;
      p = group_sum_fixed(ok ? p : 0.0f, gl);
      const float d = use_sig ? p * (a[0] * (1.0f - a[0])) : p;
      const bool st = ok && glead;
      dacc[0] += st ? d : 0.0f;
      bst1<TIO>(dlr, st ? dlb + (uint32_t)t * dlstb + (uint32_t)gjl * dlscb : kOob, d);
    } else {
      // whole groups of r channels inside the lane (r | V)
#pragma unroll
      for (int mm = 1; mm < V; mm <<= 1) {
        if (mm < S.r) {
          float tsum[V];
#pragma unroll
          for (int v = 0; v < V; ++v) tsum[v] = dav[v] + dav[v ^ mm];
#pragma unroll
          for (int v = 0; v < V; ++v) dav[v] = tsum[v];
        }
      }
      float dl[V];
#pragma unroll
      for (int v = 0; v < V; ++v) dl[v] = use_sig ? dav[v] * (a[v] * (1.0f - a[v])) : dav[v];
      if (GM == GATE_CHANVEC) {
        bst_vec<TIO, true>(dlr, dlb + (uint32_t)t * dlstb + (uint32_t)c0 * E, E, V, ok, dl);
#pragma unroll
        for (int v = 0; v < V; ++v) dacc[v] += ok ? dl[v] : 0.0f;
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const bool lead = ok && (v & (S.r - 1)) == 0 && v < nvalid;
          dacc[v] += lead ? dl[v] : 0.0f;
          bst1<TIO>(dlr, lead ? dlb + (uint32_t)t * dlstb +
                                    (uint32_t)((c0 + v) / S.r) * dlscb
                              : kOob,
                    dl[v]);
        }
      }
    }
  };

  // loads of one reverse step: gy, u, logits at t and the state entering t (the
  // saved output of t - 1, or at st the recomputed warm-up end state)
  uint4 bg[2][NB], bu[2][NB], bh[2][NB];
  LogitRaw<TIO, GM, NB> bl[2];
  auto bload = [&](int tlow, int tlim_lo, int tlim_hi, bool any, auto bufc) __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value;
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int t = tlow + s;
      const bool ok = active && any && t >= tlim_lo && t < tlim_hi;
      bg[buf][s] = bld_vec<TIO, VEC>(gr, gb + (uint32_t)t * gstb, gscb, nvalid, ok);
      bu[buf][s] = bld_vec<TIO, VEC>(ur, ub + (uint32_t)t * ustb, uscb, nvalid, ok);
      bh[buf][s] = bld_vec<TIO, VEC>(hr, hb + (uint32_t)(t - 1) * hstb, hscb, nvalid,
                                     ok && t != wd.st);
    }
    bl[buf].template load<true>(lr, lb + (uint32_t)tlow * lstb, lstb, gi, tlow, tlim_hi, active && any, nvalid,
                 tlim_lo);
  };

  // (B1) the tail [wn.lo, wn.st), read by the next window: compile-time rows of
  // HN, batches from the last
  {
    constexpr int NBW = KW / NB;
    auto b1step = [&](int q, auto bufc) __attribute__((always_inline)) {  // q-th batch from the last: rows s0 .. s0 + NB - 1
      constexpr int buf = decltype(bufc)::value;
      const int s0 = KW - (q + 1) * NB;
      const int tlow = wn.lo + s0;
      uint4 gq[NB], uq[NB], hq[NB];
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        gq[s] = bg[buf][s];
        uq[s] = bu[buf][s];
        hq[s] = tlow + s == wd.st ? h_st : bh[buf][s];
      }
      float al[NB][NA];
      bl[buf].gates(gi, tlow, wn.st, active, use_sig, al);
      if (q + 1 < NBW)
        bload(wn.lo + KW - (q + 2) * NB, wn.lo, wn.st, true, std::integral_constant<int, 1 - buf>{});
      else  // the first batch of (B2)
        bload(b2_hi - NB, wd.st, b2_hi, nb_b2 > 0, std::integral_constant<int, 1 - buf>{});
#pragma unroll
      for (int s = NB - 1; s >= 0; --s) {
        const int t = tlow + s;
        step(t, active && s0 + s < nt, gq[s], uq[s], hq[s], al[s], true, HN[s0 + s]);
      }
    };
    bload(wn.lo + KW - NB, wn.lo, wn.st, true, B0{});
    static_loop<0, NBW>([&](auto qc) __attribute__((always_inline)) {
      constexpr int q = decltype(qc)::value;
      b1step(q, std::integral_constant<int, q & 1>{});
    });
  }
  // (B2) the rest [st, b2_hi) in reverse; its first batch was loaded into the
  // buffer after the last (B1) batch
  {
    constexpr int NBW = KW / NB;
    constexpr int first = NBW % 2;  // buffer holding the first (B2) batch
    auto b2step = [&](int k, auto bufc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      const int tlow = b2_hi - (k + 1) * NB;
      uint4 gq[NB], uq[NB], hq[NB];
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        gq[s] = bg[buf][s];
        uq[s] = bu[buf][s];
        hq[s] = tlow + s == wd.st ? h_st : bh[buf][s];
      }
      float al[NB][NA];
      bl[buf].gates(gi, tlow, b2_hi, active, use_sig, al);
      bload(tlow - NB, wd.st, b2_hi, k + 1 < nb_b2, std::integral_constant<int, 1 - buf>{});
#pragma unroll
      for (int s = NB - 1; s >= 0; --s) {
        const int t = tlow + s;
        step(t, active && t >= wd.st && t < b2_hi, gq[s], uq[s], hq[s], al[s], false, h_st);
      }
    };
    for (int k = 0; k < nb_b2; k += 2) {
      b2step(k, std::integral_constant<int, first>{});
      if (k + 1 < nb_b2) b2step(k + 1, std::integral_constant<int, 1 - first>{});
    }
  }

  // ---- this window's share of grad_inits: prod_{j=lo}^{st} (1 - alpha_j) g1_st
  // (an = 1 - alpha_st after the last step; an empty window leaves g1 = 0)
  if (active) {
    float di[V];
#pragma unroll
    for (int v = 0; v < V; ++v) di[v] = prodw[GL ? 0 : v] * an[GL ? 0 : v] * g1[v];
    st_f32<VEC, V>(args.wdi + ((int64_t)bhc * nwin + m.win) * S.D + c0, nvalid, di);
  }
  // ---- dbias partial of (b, h, window)
  float* pp = args.dbias_partial + ((int64_t)bhc * nwin + m.win) * S.Da;
  if (GL) {
    if (glead) pp[gjl] = dacc[0];
  } else if (active) {
#pragma unroll
    for (int v = 0; v < V; ++v)
      if ((GM == GATE_CHANVEC || (v & (S.r - 1)) == 0) && v < nvalid) pp[(c0 + v) / S.r] = dacc[v];
  }
}

// Several consecutive windows per lane (args.wpl), walked last to first.  The
// window a lane processes before window o is o + 1, so what o needs from its
// successor is already in the lane instead of being recomputed from memory:
//   G, a_hi -- o + 1's own chain at its first step and 1 - alpha there: o + 1's
//              g1 and an when its walk ends;
//   HN, u   -- o + 1's warm-up states and inputs on [lo', st') = o's tail,
//              formed by o + 1's own warm-up pass and kept in this lane's LDS
//              slot until o's tail pass reads them.
// So u and gy are read once per step; only a lane's first window (the last of
// its group) recomputes its successor's G and warm-up from memory, as the
// one-window kernel does for every window.  Per window:
//   (B1) the tail [lo', st') in reverse, u and HN from the slot;
//   (A)  the own warm-up [lo, st): the state entering st, prod (1 - alpha), and
//        the states and u the next window in the lane needs (into the slot);
//   (B2) [st, lo') in reverse.
// The outputs are those of scan_lb_buf_bwd_kernel, element for element (the
// same operations in the same order).  Requires K - 1 < min(P, Q), so a tail
// never holds st, and KW <= 8 (the slot).
template <typename TIO, int GM, bool VEC, int KW>
__global__ void __launch_bounds__(256, 2) scan_lb_buf_bwd_multi_kernel(const BwdArgs args) {
  constexpr int V = Pack<TIO>::V;
  constexpr int NA = GM == GATE_LANE ? 1 : V;
  constexpr bool GL = GM == GATE_LANE;
  constexpr int NB = bwd_batch<GM>();
  constexpr int NBW = KW / NB;
  constexpr int E = sizeof(TIO);
  static_assert(KW % NB == 0 && KW <= 8, "warm-up rows in whole batches, at most 8");
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  const ScanShape& S = args.sh;
  const int nwin = args.nchunk;
  const int wpl = args.wpl;
  const int ngrp = (nwin + wpl - 1) / wpl;
  const LaneMap m = lane_map_bh(args.lanes, ngrp);  // m.win: the lane's group of windows
  const int bhu = __builtin_amdgcn_readfirstlane(
      (int)(m.bh < (int64_t)S.B * S.H ? m.bh : (int64_t)S.B * S.H));
  const bool in_grid = bhu < S.B * S.H;
  const int bhc = in_grid ? bhu : 0;
  const int h = bhc % S.H, b = bhc / S.H;
  const int c0 = m.cv * V;
  const int nvalid = min(V, S.D - c0);
  const bool lane_ok = in_grid && m.win < ngrp && nvalid > 0;
  const int gl = GL ? S.r / V : 1;  // lanes per gate group (GATE_LANE)
  const int g_lo = m.win * wpl;                    // the group's first window
  const int o_top = min(nwin, g_lo + wpl) - 1;     // its last: processed first

  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView hvw = head_view(args.h, which), gvw = head_view(args.gy, which);
  const Rsrc ur = slice_rsrc(args.u, b, h, E), lr = slice_rsrc(args.lg, b, h, E),
             hr = slice_rsrc(hvw, b, hl, E), gr = slice_rsrc(gvw, b, hl, E),
             dur = slice_rsrc(args.du, b, h, E), dlr = slice_rsrc(args.dlg, b, h, E);
  const uint32_t ustb = (uint32_t)(args.u.s[2] * E), uscb = (uint32_t)(args.u.s[3] * E);
  const uint32_t lstb = (uint32_t)(args.lg.s[2] * E);
  const uint32_t hstb = (uint32_t)(hvw.s[2] * E), hscb = (uint32_t)(hvw.s[3] * E);
  const uint32_t gstb = (uint32_t)(gvw.s[2] * E), gscb = (uint32_t)(gvw.s[3] * E);
  const uint32_t dustb = (uint32_t)(args.du.s[2] * E), duscb = (uint32_t)(args.du.s[3] * E);
  const uint32_t dlstb = (uint32_t)(args.dlg.s[2] * E), dlscb = (uint32_t)(args.dlg.s[3] * E);
  const uint32_t ub = chan_off(args.u, c0, E);
  const uint32_t lb = GM == GATE_CHANVEC ? chan_off(args.lg, c0, E) : 0u;
  const uint32_t hb = chan_off(hvw, c0, E), gb = chan_off(gvw, c0, E);
  const uint32_t dub = chan_off(args.du, c0, E);
  const uint32_t dlb = 0u;
  GateIdx<GM, V> gi;
  gi.init(args.bias + h * S.Da, c0, nvalid, S.D, S.r, args.lg.s[3]);
  const bool use_sig = S.use_sigmoid != 0;
  const int gjl = GL ? c0 / S.r : 0;  // gate group of this lane (GATE_LANE)
  const bool glead0 = GL && (m.cv % gl) == 0;

  // the inits, read again by every window's warm-up pass (registers are short)
  const int EI = args.init_f32 ? 4 : E;  // fp32 inits: rounded to bf16 as they are read
  const Rsrc irs = slice_rsrc(args.init, b, h, EI);
  const uint32_t ioff = chan_off(args.init, c0, EI), iscb = (uint32_t)(args.init.s[3] * EI);

  // this lane's slot: row s holds the state entering step lo' + s of the
  // successor's warm-up and the input u there (one 16-byte vector each)
  __shared__ uint4 slot_h[KW][256], slot_u[KW][256];
  const int tid = threadIdx.x;

  // ---- the successor of the lane's first window: its warm-up over that
  // window's tail (states and u into the slot), and its own chain's G
  float G[V], a_hi[NA];
#pragma unroll
  for (int v = 0; v < V; ++v) G[v] = 0.0f;
#pragma unroll
  for (int i = 0; i < NA; ++i) a_hi[i] = 0.0f;
  {
    const Window wd = look_back_window(o_top, S.T, args.P, args.Q, args.K);
    const bool has_next = o_top + 1 < nwin;
    Window wn;
    {
      const Window wr = look_back_window(o_top + 1, S.T, args.P, args.Q, args.K);
      wn.lo = (int)opaque((uint32_t)(has_next ? wr.lo : wd.hi));
      wn.st = (int)opaque((uint32_t)(has_next ? wr.st : wd.hi));
      wn.hi = (int)opaque((uint32_t)(has_next ? wr.hi : wd.hi));
    }
    const int nb_g = (wave_max(lane_ok ? wn.hi - wn.st : 0) + NB - 1) / NB;
    {
      float hn[V];
      {
        const uint4 q = bld_init<TIO, VEC>(irs, ioff, iscb, nvalid, lane_ok, args.init_f32 != 0);
#pragma unroll
        for (int v = 0; v < V; ++v) hn[v] = Pack<TIO>::get(q, v);
      }
      uint4 wu[2][NB];
      LogitRaw<TIO, GM, NB> wl[2];
      auto wload = [&](int k, auto bufc) __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        const int t0 = wn.lo + k * NB;
#pragma unroll
        for (int s = 0; s < NB; ++s)
          wu[buf][s] = bld_vec<TIO, VEC>(ur, ub + (uint32_t)(t0 + s) * ustb, uscb, nvalid,
                                         lane_ok && k < NBW && t0 + s < wn.st);
        wl[buf].template load<true>(lr, lb + (uint32_t)t0 * lstb, lstb, gi, t0, wn.st,
                                    lane_ok && k < NBW, nvalid);
      };
      auto wstep = [&](auto kc) __attribute__((always_inline)) {
        constexpr int k = decltype(kc)::value;
        constexpr int buf = k & 1;
        const int t0 = wn.lo + k * NB;
        uint4 uq[NB];
#pragma unroll
        for (int s = 0; s < NB; ++s) uq[s] = wu[buf][s];
        float al[NB][NA];
        wl[buf].gates(gi, t0, wn.st, lane_ok, use_sig, al);
        wload(k + 1, std::integral_constant<int, 1 - buf>{});
#pragma unroll
        for (int s = 0; s < NB; ++s) {
          slot_h[k * NB + s][tid] = Pack<TIO>::pack(hn);
          slot_u[k * NB + s][tid] = uq[s];
#pragma unroll
          for (int v = 0; v < V; ++v)
            hn[v] = fmaf(al[s][GL ? 0 : v], Pack<TIO>::get(uq[s], v) - hn[v], hn[v]);
        }
      };
      wload(0, B0{});
      static_loop<0, NBW>(wstep);
    }
    {
      uint4 ng[2][NB];
      LogitRaw<TIO, GM, NB> nl[2];
      auto gload = [&](int k, auto bufc) __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        const int tl = wn.hi - (k + 1) * NB;
#pragma unroll
        for (int s = 0; s < NB; ++s)
          ng[buf][s] = bld_vec<TIO, VEC>(gr, gb + (uint32_t)(tl + s) * gstb, gscb, nvalid,
                                         lane_ok && k < nb_g && tl + s >= wn.st);
        nl[buf].template load<true>(lr, lb + (uint32_t)tl * lstb, lstb, gi, tl, wn.hi,
                                    lane_ok && k < nb_g, nvalid, wn.st);
      };
      auto gstep = [&](int k, auto bufc) __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        const int tl = wn.hi - (k + 1) * NB;
        uint4 gq[NB];
#pragma unroll
        for (int s = 0; s < NB; ++s) gq[s] = ng[buf][s];
        float al[NB][NA];
        nl[buf].gates(gi, tl, wn.hi, lane_ok, use_sig, al);
        gload(k + 1, std::integral_constant<int, 1 - buf>{});
#pragma unroll
        for (int s = NB - 1; s >= 0; --s) {
          const bool ok = lane_ok && tl + s >= wn.st;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const float gn = fmaf(a_hi[GL ? 0 : v], G[v], Pack<TIO>::get(gq[s], v));
            G[v] = ok ? gn : G[v];
          }
#pragma unroll
          for (int i = 0; i < NA; ++i) a_hi[i] = ok ? 1.0f - al[s][i] : a_hi[i];
        }
      };
      gload(0, B0{});
      for (int k = 0; k < nb_g; k += 2) {
        gstep(k, B0{});
        if (k + 1 < nb_g) gstep(k + 1, B1{});
      }
    }
  }

  for (int it = 0; it < wpl; ++it) {
    const int o = o_top - it;
    const bool active = lane_ok && o >= g_lo;
    const Window wd = look_back_window(active ? o : 0, S.T, args.P, args.Q, args.K);
    const bool has_next = o + 1 < nwin;
    Window wn;
    {
      const Window wr = look_back_window(o + 1, S.T, args.P, args.Q, args.K);
      wn.lo = (int)opaque((uint32_t)(has_next ? wr.lo : wd.hi));
      wn.st = (int)opaque((uint32_t)(has_next ? wr.st : wd.hi));
      wn.hi = (int)opaque((uint32_t)(has_next ? wr.hi : wd.hi));
    }
    const int nt = wn.st - wn.lo;  // tail steps of this window (<= KW)
    const int b2_hi = has_next ? wn.lo : wd.hi;
    const int nb_b2 = (wave_max(active ? b2_hi - wd.st : 0) + NB - 1) / NB;
    const bool glead = glead0 && active;

    float g1[V], g2[V], an[NA];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      g1[v] = 0.0f;
      g2[v] = G[v];
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) an[i] = a_hi[i];
    float dacc[GL ? 1 : V];
#pragma unroll
    for (int k = 0; k < (GL ? 1 : V); ++k) dacc[k] = 0.0f;

    // one reverse step at t (branch-free; a masked step changes nothing); with_g2:
    // t lies in the next window's warm-up, hn its state
    auto step = [&](int t, bool ok, const uint4& gq, const uint4& uq, const uint4& hq,
                    const float (&a)[NA], bool with_g2, const uint4& hn) {
      float duv[V], dav[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int ia = GL ? 0 : v;
        const float g1n = fmaf(an[ia], g1[v], Pack<TIO>::get(gq, v));
        const float g2n = with_g2 ? an[ia] * g2[v] : 0.0f;
        g1[v] = ok ? g1n : g1[v];
        g2[v] = ok ? g2n : g2[v];
        const float u = Pack<TIO>::get(uq, v);
        duv[v] = a[ia] * (g1n + g2n);
        dav[v] = (u - Pack<TIO>::get(hq, v)) * g1n;
        if (with_g2) dav[v] = fmaf(u - Pack<TIO>::get(hn, v), g2n, dav[v]);
      }
#pragma unroll
      for (int i = 0; i < NA; ++i) an[i] = ok ? 1.0f - a[i] : an[i];
      bst_vec<TIO, VEC>(dur, dub + (uint32_t)t * dustb, duscb, nvalid, ok, duv);
      if (GL) {
        float p = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) p += v < nvalid ? dav[v] : 0.0f;
        p = group_sum_fixed(ok ? p : 0.0f, gl);
        const float d = use_sig ? p * (a[0] * (1.0f - a[0])) : p;
        const bool stl = ok && glead;
        dacc[0] += stl ? d : 0.0f;
        bst1<TIO>(dlr, stl ? dlb + (uint32_t)t * dlstb + (uint32_t)gjl * dlscb : kOob, d);
      } else {
#pragma unroll
        for (int mm = 1; mm < V; mm <<= 1) {
          if (mm < S.r) {
            float tsum[V];
#pragma unroll
            for (int v = 0; v < V; ++v) tsum[v] = dav[v] + dav[v ^ mm];
#pragma unroll
            for (int v = 0; v < V; ++v) dav[v] = tsum[v];
          }
        }
        float dl[V];
#pragma unroll
        for (int v = 0; v < V; ++v) dl[v] = use_sig ? dav[v] * (a[v] * (1.0f - a[v])) : dav[v];
        if (GM == GATE_CHANVEC) {
          bst_vec<TIO, true>(dlr, dlb + (uint32_t)t * dlstb + (uint32_t)c0 * E, E, V, ok, dl);
#pragma unroll
          for (int v = 0; v < V; ++v) dacc[v] += ok ? dl[v] : 0.0f;
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const bool lead = ok && (v & (S.r - 1)) == 0 && v < nvalid;
            dacc[v] += lead ? dl[v] : 0.0f;
            bst1<TIO>(dlr, lead ? dlb + (uint32_t)t * dlstb + (uint32_t)((c0 + v) / S.r) * dlscb
                                : kOob,
                      dl[v]);
          }
        }
      }
    };

    // The three passes' loads are chained: the last batch of (B1) issues the
    // first of (A), the last of (A) the first of (B2), so only the first batch
    // of a window waits for a full load round trip.
    float h1[V], prodw[NA];
    {
      const uint4 q = bld_init<TIO, VEC>(irs, ioff, iscb, nvalid, lane_ok, args.init_f32 != 0);
#pragma unroll
      for (int v = 0; v < V; ++v) h1[v] = Pack<TIO>::get(q, v);
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) prodw[i] = 1.0f;
    uint4 wu[2][NB];
    LogitRaw<TIO, GM, NB> wl[2];
    auto wload = [&](int kk, auto bufc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      const int t0 = wd.lo + kk * NB;
#pragma unroll
      for (int s = 0; s < NB; ++s)
        wu[buf][s] = bld_vec<TIO, VEC>(ur, ub + (uint32_t)(t0 + s) * ustb, uscb, nvalid,
                                       active && kk < NBW && t0 + s < wd.st);
      wl[buf].template load<true>(lr, lb + (uint32_t)t0 * lstb, lstb, gi, t0, wd.st,
                                  active && kk < NBW, nvalid);
    };
    uint4 cg[2][NB], cu[2][NB], ch[2][NB];
    LogitRaw<TIO, GM, NB> cl[2];
    auto bload = [&](int tlow, bool any, auto bufc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        const int t = tlow + s;
        const bool ok = active && any && t >= wd.st && t < b2_hi;
        cg[buf][s] = bld_vec<TIO, VEC>(gr, gb + (uint32_t)t * gstb, gscb, nvalid, ok);
        cu[buf][s] = bld_vec<TIO, VEC>(ur, ub + (uint32_t)t * ustb, uscb, nvalid, ok);
        ch[buf][s] = bld_vec<TIO, VEC>(hr, hb + (uint32_t)(t - 1) * hstb, hscb, nvalid,
                                       ok && t != wd.st);
      }
      cl[buf].template load<true>(lr, lb + (uint32_t)tlow * lstb, lstb, gi, tlow, b2_hi,
                                  active && any, nvalid, wd.st);
    };

    // (B1) the tail [wn.lo, wn.st) in reverse: gy, the saved states and the
    // logits from memory, u and the successor's warm-up states from the slot
    {
      uint4 bg[2][NB], bh[2][NB];
      LogitRaw<TIO, GM, NB> bl[2];
      auto tload = [&](int q, auto bufc) __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        const int tlow = wn.lo + KW - (q + 1) * NB;
#pragma unroll
        for (int s = 0; s < NB; ++s) {
          const int t = tlow + s;
          const bool ok = active && q < NBW && t >= wn.lo && t < wn.st;
          bg[buf][s] = bld_vec<TIO, VEC>(gr, gb + (uint32_t)t * gstb, gscb, nvalid, ok);
          bh[buf][s] = bld_vec<TIO, VEC>(hr, hb + (uint32_t)(t - 1) * hstb, hscb, nvalid, ok);
        }
        bl[buf].template load<true>(lr, lb + (uint32_t)tlow * lstb, lstb, gi, tlow, wn.st,
                                    active && q < NBW, nvalid, wn.lo);
      };
      auto tstep = [&](auto qc) __attribute__((always_inline)) {
        constexpr int q = decltype(qc)::value;
        constexpr int buf = q & 1;
        const int s0 = KW - (q + 1) * NB;
        const int tlow = wn.lo + s0;
        uint4 gq[NB], hq[NB];
#pragma unroll
        for (int s = 0; s < NB; ++s) {
          gq[s] = bg[buf][s];
          hq[s] = bh[buf][s];
        }
        float al[NB][NA];
        bl[buf].gates(gi, tlow, wn.st, active, use_sig, al);
        if constexpr (q + 1 < NBW)
          tload(q + 1, std::integral_constant<int, 1 - buf>{});
        else
          wload(0, B0{});  // the first batch of (A)
#pragma unroll
        for (int s = NB - 1; s >= 0; --s) {
          const int t = tlow + s;
          step(t, active && s0 + s < nt, gq[s], slot_u[s0 + s][tid], hq[s], al[s], true,
               slot_h[s0 + s][tid]);
        }
      };
      tload(0, B0{});
      static_loop<0, NBW>(tstep);
    }

    // (A) the own warm-up [lo, st): the state entering st and prod (1 - alpha);
    // its states and u are the slot of the next window in the lane (o - 1,
    // whose tail this is), written after (B1) has read this window's
    {
      auto wstep = [&](auto kc) __attribute__((always_inline)) {
        constexpr int kk = decltype(kc)::value;
        constexpr int buf = kk & 1;
        const int t0 = wd.lo + kk * NB;
        uint4 uq[NB];
#pragma unroll
        for (int s = 0; s < NB; ++s) uq[s] = wu[buf][s];
        float al[NB][NA];
        wl[buf].gates(gi, t0, wd.st, active, use_sig, al);  // 0 when masked: the identity step
        if constexpr (kk + 1 < NBW)
          wload(kk + 1, std::integral_constant<int, 1 - buf>{});
        else
          bload(b2_hi - NB, nb_b2 > 0, B0{});  // the first batch of (B2)
#pragma unroll
        for (int s = 0; s < NB; ++s) {
          slot_h[kk * NB + s][tid] = Pack<TIO>::pack(h1);
          slot_u[kk * NB + s][tid] = uq[s];
#pragma unroll
          for (int v = 0; v < V; ++v)
            h1[v] = fmaf(al[s][GL ? 0 : v], Pack<TIO>::get(uq[s], v) - h1[v], h1[v]);
#pragma unroll
          for (int i = 0; i < NA; ++i) prodw[i] *= 1.0f - al[s][i];
        }
      };
      static_loop<0, NBW>(wstep);
    }
    const uint4 h_st = Pack<TIO>::pack(h1);  // I/O-rounded, as the saved outputs

    // (B2) [st, b2_hi) in reverse (its first batch was issued by (A))
    {
      auto b2step = [&](int kk, auto bufc) __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        const int tlow = b2_hi - (kk + 1) * NB;
        uint4 gq[NB], uq[NB], hq[NB];
#pragma unroll
        for (int s = 0; s < NB; ++s) {
          gq[s] = cg[buf][s];
          uq[s] = cu[buf][s];
          hq[s] = tlow + s == wd.st ? h_st : ch[buf][s];
        }
        float al[NB][NA];
        cl[buf].gates(gi, tlow, b2_hi, active, use_sig, al);
        bload(tlow - NB, kk + 1 < nb_b2, std::integral_constant<int, 1 - buf>{});
#pragma unroll
        for (int s = NB - 1; s >= 0; --s) {
          const int t = tlow + s;
          step(t, active && t >= wd.st && t < b2_hi, gq[s], uq[s], hq[s], al[s], false, h_st);
        }
      };
      for (int kk = 0; kk < nb_b2; kk += 2) {
        b2step(kk, B0{});
        if (kk + 1 < nb_b2) b2step(kk + 1, B1{});
      }
    }

    // ---- this window's share of grad_inits and its dbias partial
    if (active) {
      float di[V];
#pragma unroll
      for (int v = 0; v < V; ++v) di[v] = prodw[GL ? 0 : v] * an[GL ? 0 : v] * g1[v];
      st_f32<VEC, V>(args.wdi + ((int64_t)bhc * nwin + o) * S.D + c0, nvalid, di);
      float* pp = args.dbias_partial + ((int64_t)bhc * nwin + o) * S.Da;
      if (GL) {
        if (glead) pp[gjl] = dacc[0];
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v)
          if ((GM == GATE_CHANVEC || (v & (S.r - 1)) == 0) && v < nvalid) pp[(c0 + v) / S.r] = dacc[v];
      }
    }
    // the window before this one in the lane starts from this one's chain
#pragma unroll
    for (int v = 0; v < V; ++v) G[v] = g1[v];
#pragma unroll
    for (int i = 0; i < NA; ++i) a_hi[i] = an[i];
  }
}

template <typename TIO, int GM, bool VEC>
void launch_fwd(const FwdArgs& a, int grid, bool buf, hipStream_t st) {
  if (buf)
    hipLaunchKernelGGL((scan_lb_buf_fwd_kernel<TIO, GM, VEC>), dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((scan_lb_short_fwd_kernel<TIO, GM, VEC>), dim3(grid), dim3(256), 0, st, a);
}

template <typename TIO, int GM, bool VEC>
constexpr bool lb_multi_ok() {
  return sizeof(TIO) == 4 || (GM == GATE_LANE && VEC);
}
inline bool lb_multi_ok_rt(bool f32, int gm, bool vec) {
  return f32 || (gm == GATE_LANE && vec);
}

template <typename TIO, int GM, bool VEC>
void launch_bwd(const BwdArgs& a, int grid, int kw_max, bool buf, bool multi, hipStream_t st) {
  // the several-windows kernel is built where it fits two wavefronts per SIMD
  // without spilling in its loops
  if constexpr (lb_multi_ok<TIO, GM, VEC>()) {
    if (multi) {
      hipLaunchKernelGGL((scan_lb_buf_bwd_multi_kernel<TIO, GM, VEC, 8>), dim3(grid), dim3(256),
                         0, st, a);
      return;
    }
  }
  if (buf) {
    if (kw_max <= 8)
      hipLaunchKernelGGL((scan_lb_buf_bwd_kernel<TIO, GM, VEC, 8>), dim3(grid), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((scan_lb_buf_bwd_kernel<TIO, GM, VEC, 16>), dim3(grid), dim3(256), 0, st, a);
  } else if (kw_max <= 8) {
    hipLaunchKernelGGL((scan_lb_short_bwd_kernel<TIO, GM, VEC, 8>), dim3(grid), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((scan_lb_short_bwd_kernel<TIO, GM, VEC, 16>), dim3(grid), dim3(256), 0, st, a);
  }
}

template <typename TIO>
int fwd_t(const FwdArgs& a, bool vec, int gm, bool buf, hipStream_t st) {
  const int64_t lanes =
      (int64_t)a.sh.B * a.sh.H * (buf ? lanes_per_bh(a.lanes, a.nwin) : (int64_t)a.nwin * a.lanes);
  const int64_t grid = (lanes + 255) / 256;
  LTV_REQUIRE(grid < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
  if (vec) {
    if (gm == GATE_LANE) launch_fwd<TIO, GATE_LANE, true>(a, (int)grid, buf, st);
    else if (gm == GATE_CHANVEC) launch_fwd<TIO, GATE_CHANVEC, true>(a, (int)grid, buf, st);
    else launch_fwd<TIO, GATE_CHAN, true>(a, (int)grid, buf, st);
  } else {
    if (gm == GATE_LANE) launch_fwd<TIO, GATE_LANE, false>(a, (int)grid, buf, st);
    else launch_fwd<TIO, GATE_CHAN, false>(a, (int)grid, buf, st);
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

template <typename TIO>
int bwd_t(const BwdArgs& a, bool vec, int gm, int kw_max, bool buf, hipStream_t st) {
  // several windows per lane (a.wpl) only with buffer addressing, a warm-up of
  // at most 8 steps and an instantiation that has the kernel
  const bool multi = buf && a.wpl > 1 && kw_max <= 8 && lb_multi_ok_rt(sizeof(TIO) == 4, gm, vec);
  const int ngrp = multi ? (a.nchunk + a.wpl - 1) / a.wpl : a.nchunk;
  const int64_t lanes = (int64_t)a.sh.B * a.sh.H *
                        (buf ? lanes_per_bh(a.lanes, ngrp) : (int64_t)a.nchunk * a.lanes);
  const int64_t grid = (lanes + 255) / 256;
  LTV_REQUIRE(grid < (1ll << 31), LTV_ERR_UNSUPPORTED, "grid too large");
  LTV_REQUIRE(kw_max <= 16, LTV_ERR_UNSUPPORTED, "warm-up of %d steps too long", kw_max);
  if (vec) {
    if (gm == GATE_LANE) launch_bwd<TIO, GATE_LANE, true>(a, (int)grid, kw_max, buf, multi, st);
    else if (gm == GATE_CHANVEC) launch_bwd<TIO, GATE_CHANVEC, true>(a, (int)grid, kw_max, buf, multi, st);
    else launch_bwd<TIO, GATE_CHAN, true>(a, (int)grid, kw_max, buf, multi, st);
  } else {
    if (gm == GATE_LANE) launch_bwd<TIO, GATE_LANE, false>(a, (int)grid, kw_max, buf, multi, st);
    else launch_bwd<TIO, GATE_CHAN, false>(a, (int)grid, kw_max, buf, multi, st);
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

}  // namespace

int scan_launch_lb_short_fwd(bool bf16, const FwdArgs& a, bool vec, int gm, bool buf,
                             hipStream_t st) {
  return bf16 ? fwd_t<bf16_t>(a, vec, gm, buf, st) : fwd_t<float>(a, vec, gm, buf, st);
}

int scan_launch_lb_short_bwd(bool bf16, const BwdArgs& a, bool vec, int gm, int kw_max, bool buf,
                             hipStream_t st) {
  return bf16 ? bwd_t<bf16_t>(a, vec, gm, kw_max, buf, st)
              : bwd_t<float>(a, vec, gm, kw_max, buf, st);
}

}  // namespace ltv
