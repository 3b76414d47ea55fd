// fp32-accumulating MFMA GEMM over strided operands (gfx950
// v_mfma_f32_32x32x2_f32), the engine of the reference-layout
// fused_linear_transpose op in fp32, and in bf16 for the layouts the
// direct-to-LDS bf16 kernels do not take:
//
//   C(m, n) = sum_kk A(m, kk) B(n, kk),   kk = ko * kin + ki
//   A(m, kk) at A + m sam + ko sako + ki saki (+ z sab for batch z), B alike
//
// The products are exact in fp32 for bf16 operands and rounded once for fp32
// ones, as in an fp32 FMA; the sums run in fp32.
//
// 128 x 128 output tiles, 8 wavefronts of 64 x 32 (2 blocks of 32 x 32),
// 32-wide k-steps through two LDS stages: the global loads of step s + 1 sit
// in registers while step s runs its MFMAs, then go to the other stage; one
// barrier per step.  Two workgroups share a CU (at most 72 KB of LDS each).
// Each operand is staged in one of three ways, chosen per launch from its
// strides:
//   kF32KQ  k-contiguous quads (saki = 1): 4 consecutive k of one row per
//           load, LDS [row][k] (rows padded to 36 floats);
//   kF32MQ  row-contiguous quads (sam = 1): 4 consecutive rows at one k,
//           LDS [k][row] (k-rows padded to 136 floats);
//   kF32SC  any strides: one element per load, LDS [k][row].
// Reduction order inside a k-step: the MFMA takes, per lane, one element of a
// 2-deep reduction (lanes 0..31 the first, lanes 32..63 the second).  The p-th
// MFMA of 8-k group g gives lanes 0..31 k = 8 g + p and lanes 32..63
// k = 8 g + 4 + p, so a KQ lane fetches its four k with one ds_read_b128; both
// operands use the same assignment, so every product pairs matching k.
//
// Split-K: blockIdx.z = batch * splits + split; split s sums
// kk in [s k_split, min(K, (s + 1) k_split)) into C + s scs (k_split a
// multiple of the 32-wide k-step).
#pragma once

#include <utility>

#include "ltv_device.hpp"

namespace ltv {

enum F32Stage { kF32KQ = 0, kF32MQ = 1, kF32SC = 2 };

constexpr int kF32B = 128;  // tile rows of A and of B
constexpr int kF32BK = 32;  // reduction indices per k-step
constexpr int kF32RowKQ = kF32BK + 4;  // floats per LDS row, KQ staging
constexpr int kF32RowMQ = kF32B + 8;   // floats per LDS k-row, MQ / SC staging
// 8 wavefronts (2 along the rows x 4 along the columns) of 64 x 32: four per
// SIMD with two workgroups per CU, so one wavefront's barrier or load wait
// leaves three to feed the SIMD's matrix core
constexpr int kF32Threads = 512;
constexpr int kF32Quads = kF32B * kF32BK / 4 / kF32Threads;  // quads per thread per operand
constexpr int kF32BlocksN = 1;  // 32-column blocks per wavefront

template <int L>
struct F32LdsTile {
  static constexpr int kFloats = L == kF32KQ ? kF32B * kF32RowKQ : kF32BK * kF32RowMQ;
};

struct F32mArgs {
  const void* A;
  int64_t sam, sako, saki, sab;
  const void* B;
  int64_t sbn, sbko, sbki, sbb;
  void* C;
  int64_t scm, scn, scb, scs;  // output strides: row, column, batch, split
  int M, N, K, kin;
  int k_split, splits;
};

// One operand of one workgroup: its rows [row0, row0 + 128) and the
// reduction range [kb, ke) of its split.
template <typename TI>
struct F32Operand {
  const TI* p;  // at the workgroup's batch
  int64_t sr, sko, ski;
  int rows, kin, row0, ke;
  bool outer;  // the reduction index has an outer part (kin < K)

  __device__ __forceinline__ int64_t koff(int kk) const {
    if (!outer) return (int64_t)kk * ski;
    const int ko = kk / kin;
    return (int64_t)ko * sko + (int64_t)(kk - ko * kin) * ski;
  }
};

// 4 consecutive elements (aligned) -> floats
__device__ __forceinline__ float4 ld_quad(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ float4 ld_quad(const bf16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                     __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
}

// Global -> registers -> LDS staging of one 128-row x 32-k operand tile.
// A k-step inside the reduction range whose 32 indices share one outer index
// (kin a multiple of 32, or no outer part) takes the fast load: each quad at
// a per-thread pointer fixed for the tile plus a per-step scalar offset, rows
// past the operand masked (KQ and MQ; an MQ tile whose last quad is partial
// takes the general load).  Other steps check every element.
template <typename TI, int L>
struct F32Stager {
  float4 r[kF32Quads];  // KQ / MQ: kF32Quads quads per thread; SC: 4 kF32Quads elements
  const TI* rp[kF32Quads];  // KQ / MQ: quad c at the tile's rows and this thread's k, k0 = 0
  uint32_t ok;      // bit c: quad c lies inside the operand's rows
  uint32_t keep;    // bit c: quad c of the last load is stored as loaded (else zeros)
  bool fast_ok;     // the fast load applies to this tile (uniform)

  __device__ __forceinline__ void setup(const F32Operand<TI>& op) {
    const int t = threadIdx.x;
    ok = 0;
    fast_ok = L != kF32SC && (!op.outer || op.kin % kF32BK == 0) &&
              !(L == kF32MQ && op.rows % 4 != 0 && op.row0 + kF32B > op.rows);
#pragma unroll
    for (int c = 0; c < kF32Quads; ++c) {
      const int q = t + kF32Threads * c;
      if (L == kF32KQ) {
        const int row = op.row0 + (q >> 3);
        rp[c] = op.p + (int64_t)(row < op.rows ? row : 0) * op.sr + 4 * (q & 7);
        if (row < op.rows) ok |= 1u << c;
      } else {
        const int row = op.row0 + 4 * (q & 31);
        rp[c] = op.p + (row < op.rows ? row : 0) + (int64_t)(q >> 5) * op.ski;
        if (row < op.rows) ok |= 1u << c;
      }
    }
  }

  // the fast load applies to the step at k0 (uniform)
  __device__ __forceinline__ bool fast_at(const F32Operand<TI>& op, int k0) const {
    return fast_ok && k0 + kF32BK <= op.ke;
  }

  // Rows past the operand load row 0 of the operand (clamped pointers: no
  // branch, so the loads of both operands stay in flight together) and are
  // replaced by zeros when stored, after the step's MFMAs.
  __device__ __forceinline__ void load_fast(const F32Operand<TI>& op, int k0) {
    // offset of reduction index k0; the step's 32 indices share its outer index
    const int64_t ks = op.outer ? (int64_t)(k0 / op.kin) * op.sko + (int64_t)(k0 % op.kin) * op.ski
                                : (int64_t)k0 * op.ski;
#pragma unroll
    for (int c = 0; c < kF32Quads; ++c) r[c] = ld_quad(rp[c] + ks);
    keep = ok;
  }

  __device__ __forceinline__ void load_checked(const F32Operand<TI>& op, int k0) {
    const int t = threadIdx.x;
    keep = (1u << kF32Quads) - 1;
#pragma unroll
    for (int c = 0; c < kF32Quads; ++c) {
      const int q = t + kF32Threads * c;
      float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (L == kF32KQ) {
        const int row = op.row0 + (q >> 3), kk = k0 + 4 * (q & 7);
        if (row < op.rows && kk < op.ke) {
          const TI* p = op.p + (int64_t)row * op.sr + op.koff(kk);
          if (kk + 4 <= op.ke) {
            const float4 f = ld_quad(p);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (kk + e < op.ke) v[e] = io_traits<TI>::load(p + e);
          }
        }
      } else if (L == kF32MQ) {
        const int row = op.row0 + 4 * (q & 31), kk = k0 + (q >> 5);
        if (row < op.rows && kk < op.ke) {
          const TI* p = op.p + row + op.koff(kk);
          if (row + 4 <= op.rows) {
            const float4 f = ld_quad(p);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (row + e < op.rows) v[e] = io_traits<TI>::load(p + e);
          }
        }
      } else {
        // element e of this thread: row (t & 127), k-row (t >> 7) + 4 (4 c + e)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = op.row0 + (t & 127), kk = k0 + (t >> 7) + (kF32Threads / kF32B) * (4 * c + e);
          if (row < op.rows && kk < op.ke)
            v[e] = io_traits<TI>::load(op.p + (int64_t)row * op.sr + op.koff(kk));
        }
      }
      r[c] = make_float4(v[0], v[1], v[2], v[3]);
    }
  }

  __device__ __forceinline__ void store(float* lds) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int c = 0; c < kF32Quads; ++c) {
      const int q = t + kF32Threads * c;
      const bool in = (keep >> c) & 1u;
      const float4 v = in ? r[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (L == kF32KQ) {
        *reinterpret_cast<float4*>(lds + (q >> 3) * kF32RowKQ + 4 * (q & 7)) = v;
      } else if (L == kF32MQ) {
        *reinterpret_cast<float4*>(lds + (q >> 5) * kF32RowMQ + 4 * (q & 31)) = v;
      } else {
        const float v[4] = {r[c].x, r[c].y, r[c].z, r[c].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          lds[((t >> 7) + (kF32Threads / kF32B) * (4 * c + e)) * kF32RowMQ + (t & 127)] = v[e];
      }
    }
  }
};

// The four MFMA operands (p = 0..3) of 8-k group g for block rows
// [rb, rb + 32): lane l's row rb + l % 32, k = 8 g + 4 (l / 32) + p.
template <int L>
__device__ __forceinline__ float4 f32_frag(const float* lds, int rb, int g, int lane) {
  const int row = rb + (lane & 31), k = 8 * g + 4 * (lane >> 5);
  if (L == kF32KQ) return *reinterpret_cast<const float4*>(lds + row * kF32RowKQ + k);
  const float* p = lds + k * kF32RowMQ + row;
  return make_float4(p[0], p[kF32RowMQ], p[2 * kF32RowMQ], p[3 * kF32RowMQ]);
}

template <typename TI, typename TO, int LA, int LB>
__global__ void __launch_bounds__(kF32Threads, 2) gemm_f32m_kernel(const F32mArgs g) {
  __shared__ __attribute__((aligned(16))) float lds_a[2][F32LdsTile<LA>::kFloats];
  __shared__ __attribute__((aligned(16))) float lds_b[2][F32LdsTile<LB>::kFloats];

  // workgroup w (dispatch order) runs on XCD w % 8: deal the tiles to the XCDs
  // in contiguous ranges (n-tiles fastest), so tiles sharing an operand tile
  // share that XCD's L2.  XCD x holds the workgroups x, x + 8, ... < total:
  // q + (x < r) of them (q, r = total / 8, total % 8), tiles from x q + min(x, r).
  const int gx = gridDim.x, gy = gridDim.y;
  const int64_t total = (int64_t)gx * gy * gridDim.z;
  const int64_t w = blockIdx.x + (int64_t)gx * (blockIdx.y + (int64_t)gy * blockIdx.z);
  const int64_t xcd = w % 8, q = total / 8, r = total % 8;
  const int64_t u = xcd * q + (xcd < r ? xcd : r) + w / 8;
  const int tx = (int)(u % gx), ty = (int)((u / gx) % gy), z = (int)(u / ((int64_t)gx * gy));
  const int batch = z / g.splits, split = z - batch * g.splits;
  const int kb = split * g.k_split;
  const int ke = min(g.K, kb + g.k_split);
  const int m0 = ty * kF32B, n0 = tx * kF32B;
  const bool outer = g.kin < g.K;

  F32Operand<TI> oa{reinterpret_cast<const TI*>(g.A) + (int64_t)batch * g.sab, g.sam, g.sako,
                    g.saki, g.M, g.kin, m0, ke, outer};
  F32Operand<TI> ob{reinterpret_cast<const TI*>(g.B) + (int64_t)batch * g.sbb, g.sbn, g.sbko,
                    g.sbki, g.N, g.kin, n0, ke, outer};

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave & 1) * 64, wn = (wave >> 1) * (32 * kF32BlocksN);

  f32x16_t acc[2][kF32BlocksN];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < kF32BlocksN; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

  F32Stager<TI, LA> sa;
  F32Stager<TI, LB> sb;
  sa.setup(oa);
  sb.setup(ob);
  auto load_step = [&](int k0) {
    if (sa.fast_at(oa, k0) && sb.fast_at(ob, k0)) {
      sa.load_fast(oa, k0);
      sb.load_fast(ob, k0);
    } else {
      sa.load_checked(oa, k0);
      sb.load_checked(ob, k0);
    }
  };
  const int nsteps = ke > kb ? (ke - kb + kF32BK - 1) / kF32BK : 0;
  if (nsteps > 0) {
    load_step(kb);
    sa.store(lds_a[0]);
    sb.store(lds_b[0]);
  }
  __syncthreads();
  // Fragments of 8-k group g go to register set g & 1, read one group ahead
  // of their MFMAs.  The last group's MFMAs of a step run after the barrier
  // that ends it, covering the first reads of the next step.
  float4 fa[2][2], fb[2][kF32BlocksN];
  auto read_group = [&](auto setc, int stage, int gi) {
    constexpr int set = decltype(setc)::value;
#pragma unroll
    for (int a = 0; a < 2; ++a) fa[set][a] = f32_frag<LA>(lds_a[stage], wm + 32 * a, gi, lane);
#pragma unroll
    for (int b = 0; b < kF32BlocksN; ++b) fb[set][b] = f32_frag<LB>(lds_b[stage], wn + 32 * b, gi, lane);
  };
  auto mfma_group = [&](auto setc) {
    constexpr int set = decltype(setc)::value;
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < kF32BlocksN; ++b) {
          const float4& A = fa[set][a];
          const float4& Bf = fb[set][b];
          const float av = p == 0 ? A.x : p == 1 ? A.y : p == 2 ? A.z : A.w;
          const float bv = p == 0 ? Bf.x : p == 1 ? Bf.y : p == 2 ? Bf.z : Bf.w;
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[a][b], 0, 0, 0);
        }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  static_assert(kF32BK / 8 == 4, "four 8-k groups per step");
  if (nsteps > 0) read_group(S0{}, 0, 0);
  for (int s = 0; s < nsteps; ++s) {
    const int cur = s & 1;
    const bool more = s + 1 < nsteps;
    if (more) load_step(kb + (s + 1) * kF32BK);
    read_group(S1{}, cur, 1);
    mfma_group(S0{});
    read_group(S0{}, cur, 2);
    mfma_group(S1{});
    read_group(S1{}, cur, 3);
    mfma_group(S0{});
    if (more) {
      // the other stage was last read in step s - 1, before the barrier that ended it
      sa.store(lds_a[cur ^ 1]);
      sb.store(lds_b[cur ^ 1]);
    }
    __syncthreads();
    if (more) read_group(S0{}, cur ^ 1, 0);
    mfma_group(S1{});
  }

  // lane l of block (a, b) holds column n = 32 b + l % 32 and rows
  // m = 32 a + 8 (v / 4) + 4 (l / 32) + v % 4
  TO* C = reinterpret_cast<TO*>(g.C) + (int64_t)batch * g.scb + (int64_t)split * g.scs;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < kF32BlocksN; ++b) {
      const int n = n0 + wn + 32 * b + (lane & 31);
      if (n >= g.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm + 32 * a + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (m < g.M) io_traits<TO>::store(C + (int64_t)m * g.scm + (int64_t)n * g.scn, acc[a][b][v]);
      }
    }
}

}  // namespace ltv
