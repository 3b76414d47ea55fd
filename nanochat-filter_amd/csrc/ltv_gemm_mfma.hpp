// bf16 MFMA GEMM core for gfx950 (fp32 accumulation).
//
//   Out(i, j) = sum_k P(i, k) * Q(j, k)
//
// i is the output axis that is contiguous in memory (each lane of a
// v_mfma_f32_32x32x16_bf16 result holds four consecutive i), j the other one.
// Each operand is stored either K-contiguous (KC: (row, k) at row * ld + k) or
// row-contiguous (RC: (row, k) at k * ld + row).  Tiles are staged through LDS
// in the operand's own orientation; KC fragments are read with ds_read_b128,
// RC fragments with ds_read_b64_tr_b16, whose lane layout (pinned on MI355X):
// within each 16-lane group, lane i receives element i % 4 of the 8-byte chunks
// addressed by lanes i / 4, i / 4 + 4, i / 4 + 8, i / 4 + 12.  Addressing lane s
// at row kb + s / 4, columns 4 (s % 4) .. + 3 of a [k][row] tile therefore hands
// lane i the column-i values of rows kb .. kb + 3: an MFMA operand fragment.
//
// Block tile BI x BJ x 64, WGI x WGJ wavefronts each owning (BI / WGI) x
// (BJ / WGJ) as 32 x 32 MFMA blocks.  Two LDS stages and one register stage:
// global loads run a k-tile ahead of the MFMAs, one barrier per k-tile.  The
// reduction range can be split (split-K); the kernel is persistent over all
// (tile, split) work items.
#pragma once

#include <utility>

#include "ltv_device.hpp"

namespace ltv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

enum OpLayout { OP_KC = 0, OP_RC = 1 };

// Every operand must span fewer than 2^31 elements (the kernels keep 32-bit
// element offsets); the host entry points check this.
struct GemmOperand {
  const bf16_t* p;
  int64_t ld;
  int rows;     // rows >= this read as zero
  int k_valid;  // k >= this reads as zero
  // Batched layout (blen > 0, direct-to-LDS kernel only): the batched index --
  // the rows of an RC operand, the reduction index of a KC one -- runs in
  // batches of blen whose storage lies bstride elements apart: index n sits
  // at (n / blen) bstride + n % blen.  A tile's rows (RC) or a k-step (KC)
  // must not straddle two batches.
  int64_t bstride = 0;
  int blen = 0;
};

struct GemmArgs {
  GemmOperand P, Q;
  int K;        // total reduction length
  int k_split;  // reduction length per split (multiple of 64)
  int splits;   // number of splits of the reduction
  int tiles_i, tiles_j;
};

constexpr int kGemmBK = 64;
constexpr int kPadKC = 8;   // bf16 of padding per KC row in LDS (bank spread)
// bf16 of padding per RC row in LDS: with a 64-byte row offset modulo 256
// bytes, the four rows one 16-lane group of ds_read_b64_tr_b16 touches land in
// four disjoint 16-bank windows
constexpr int kPadRC = 32;

template <int R, int L>
struct LdsTile {
  static constexpr int kElems = L == OP_KC ? R * (kGemmBK + kPadKC) : kGemmBK * (R + kPadRC);
};

// zero the bf16 elements of a 16-byte chunk whose index k0 + e >= k_valid
__device__ __forceinline__ uint4 mask_k_tail(uint4 q, int k0, int k_valid) {
  if (k0 + 8 <= k_valid) return q;
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t keep = 0;
    if (k0 + 2 * p < k_valid) keep |= 0x0000ffffu;
    if (k0 + 2 * p + 1 < k_valid) keep |= 0xffff0000u;
    w[p] &= keep;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Global -> registers -> LDS staging of one operand tile (R rows x 64 k).
// setup() fixes the tile's rows (per-chunk base pointers and row validity);
// load() then only offsets by k0, with per-chunk k checks only in the k-tile
// that crosses k_valid / k_end.
template <int R, int L, int NT>
struct TileStage {
  static constexpr int CH = R * 8 / NT;  // 16-byte chunks per thread
  static_assert(CH >= 1 && R * 8 % NT == 0, "tile too small for the thread count");
  uint4 q[CH];
  const bf16_t* p;
  uint32_t off[CH];  // chunk element offset from p at k = 0 (operands span < 2^31 elements)
  uint32_t row_ok;   // bit c: chunk c's row is inside the operand
  int64_t ld;

  __device__ __forceinline__ void setup(const GemmOperand& op, int row0) {
    p = op.p;
    ld = op.ld;
    row_ok = 0;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int idx = threadIdx.x + c * NT;
      if (L == OP_KC) {
        const int row = idx >> 3, kc = (idx & 7) * 8;
        const bool ok = row0 + row < op.rows;
        off[c] = ok ? (uint32_t)((int64_t)(row0 + row) * op.ld + kc) : 0u;
        if (ok) row_ok |= 1u << c;
      } else {
        const int kk = idx / (R / 8), rc = (idx % (R / 8)) * 8;
        const bool ok = row0 + rc < op.rows;
        off[c] = ok ? (uint32_t)((int64_t)kk * op.ld + row0 + rc) : 0u;
        if (ok) row_ok |= 1u << c;
      }
    }
  }

  __device__ __forceinline__ void load(int k0, int kv) {
    const bool full = k0 + kGemmBK <= kv;  // uniform across the workgroup
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int idx = threadIdx.x + c * NT;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      const bool rok = (row_ok >> c) & 1u;
      if (L == OP_KC) {
        const bf16_t* ptr = p + off[c] + k0;
        if (full) {
          if (rok) v = *reinterpret_cast<const uint4*>(ptr);
        } else {
          const int gk = k0 + (idx & 7) * 8;
          if (rok && gk < kv) v = mask_k_tail(*reinterpret_cast<const uint4*>(ptr), gk, kv);
        }
      } else {
        const bf16_t* ptr = p + off[c] + (int64_t)k0 * ld;
        if (full) {
          if (rok) v = *reinterpret_cast<const uint4*>(ptr);
        } else {
          const int gk = k0 + idx / (R / 8);
          if (rok && gk < kv) v = *reinterpret_cast<const uint4*>(ptr);
        }
      }
      q[c] = v;
    }
  }

  __device__ __forceinline__ void store(bf16_t* lds) const {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int idx = threadIdx.x + c * NT;
      if (L == OP_KC) {
        const int row = idx >> 3, kc = (idx & 7) * 8;
        *reinterpret_cast<uint4*>(lds + row * (kGemmBK + kPadKC) + kc) = q[c];
      } else {
        const int kk = idx / (R / 8), rc = (idx % (R / 8)) * 8;
        *reinterpret_cast<uint4*>(lds + kk * (R + kPadRC) + rc) = q[c];
      }
    }
  }
};

// MFMA operand fragment (8 consecutive k of one row) for k-step ks.
template <int R, int L>
__device__ __forceinline__ bf16x8_t read_frag(const bf16_t* lds, int row_base, int ks, int lane) {
  if (L == OP_KC) {
    const bf16_t* p = lds + (row_base + (lane & 31)) * (kGemmBK + kPadKC) + ks * 16 + 8 * (lane >> 5);
    return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
  } else {
    const int g = lane >> 4, s = lane & 15;
    const int row = row_base + (g & 1) * 16 + 4 * (s & 3);
    const int k = ks * 16 + (g >> 1) * 8 + (s >> 2);
    typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
    const bf16_t* p0 = lds + k * (R + kPadRC) + row;
    const bf16_t* p1 = p0 + 4 * (R + kPadRC);
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p0);
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p1);
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    const i16x8_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8_t, v);
  }
}

template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{})
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Scheduling pattern for one k-step: N times {one MFMA, RD LDS reads, WR LDS
// writes, VM global loads}.  Instructions beyond the pattern are placed freely.
template <int N, int RD, int WR, int VM>
__device__ __forceinline__ void sched_interleave() {
  if constexpr (N > 0) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // MFMA
    if constexpr (RD > 0) __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);  // DS read
    if constexpr (WR > 0) __builtin_amdgcn_sched_group_barrier(0x200, WR, 0);  // DS write
    if constexpr (VM > 0) __builtin_amdgcn_sched_group_barrier(0x020, VM, 0);  // VMEM read
    sched_interleave<N - 1, RD, WR, VM>();
  }
}

// Position in a workgroup's stream of (output tile, split, k-tile) steps.
// Workgroup w takes work items w, w + G, w + 2G, ... (G = gridDim.x); when the
// item count and G are multiples of 8, item u is remapped so that all items of
// one XCD (w % 8) form a contiguous range, i fastest: tiles that share a j
// block then share that XCD's L2.
struct GemmCursor {
  int k, kt, nk;  // item ordinal of this workgroup, k-tile within the item, k-tiles in it
  int i0, j0, kb, ke, split;
  bool valid;
};

template <int BI, int BJ>
__device__ __forceinline__ void gemm_decode(const GemmArgs& g, GemmCursor& c) {
  const int ntiles = g.tiles_i * g.tiles_j;
  const int total = ntiles * g.splits;
  int u = blockIdx.x + c.k * gridDim.x;
  c.valid = u < total;
  if (!c.valid) return;
  if (total % 8 == 0 && gridDim.x % 8 == 0) u = (u % 8) * (total / 8) + u / 8;
  const int split = u / ntiles;
  const int tile = u - split * ntiles;
  const int ti = tile % g.tiles_i, tj = tile / g.tiles_i;
  c.i0 = ti * BI;
  c.j0 = tj * BJ;
  c.split = split;
  c.kb = split * g.k_split;
  c.ke = min(c.kb + g.k_split, g.K);
  c.nk = (c.ke - c.kb + kGemmBK - 1) / kGemmBK;
  c.kt = 0;
}

template <int BI, int BJ>
__device__ __forceinline__ void gemm_advance(const GemmArgs& g, GemmCursor& c) {
  if (++c.kt >= c.nk) {
    ++c.k;
    gemm_decode<BI, BJ>(g, c);
  }
}

// Persistent: gridDim.x workgroups walk all (tile, split) items as one
// continuous stream of k-tiles, so the loads of the next tile are in flight
// while the current tile's epilogue stores drain.  Every item needs >= 1 k-tile.
template <int BI, int BJ, int WGI, int WGJ, int PL, int QL, class Epi>
__global__ void __launch_bounds__(WGI * WGJ * 64)
gemm_bf16_kernel(const GemmArgs g, const Epi epi) {
  constexpr int NT = WGI * WGJ * 64;
  constexpr int WI = BI / WGI, WJ = BJ / WGJ;
  constexpr int MI = WI / 32, MJ = WJ / 32;
  static_assert(MI >= 1 && MJ >= 1 && WI % 32 == 0 && WJ % 32 == 0, "bad wave tile");
  constexpr int PE = LdsTile<BI, PL>::kElems, QE = LdsTile<BJ, QL>::kElems;

  __shared__ __attribute__((aligned(16))) bf16_t lds_p[2][PE];
  __shared__ __attribute__((aligned(16))) bf16_t lds_q[2][QE];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wi = wave % WGI, wj = wave / WGI;

  f32x16_t acc[MI][MJ];
#pragma unroll
  for (int a = 0; a < MI; ++a)
#pragma unroll
    for (int b = 0; b < MJ; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

  TileStage<BI, PL, NT> sp;
  TileStage<BJ, QL, NT> sq;

  // One k-tile of MFMAs from LDS.  Operand fragments are double-buffered in
  // registers (the next k-step's reads issue between this step's MFMAs).  The
  // staging of the next k-tile overlaps the MFMAs too: during k-step 1 the
  // registers loaded one k-tile ago go to the other LDS stage (free since the
  // barrier that ended the previous k-tile), during k-step 2 the loads of the
  // k-tile after next are issued into the freed registers.  sched_group_barrier
  // interleaves MFMAs with those memory instructions.
  constexpr int NMF = MI * MJ;  // MFMAs per k-step
  constexpr int NRD = (PL == OP_RC ? 2 : 1) * MI + (QL == OP_RC ? 2 : 1) * MJ;  // LDS reads
  constexpr int RD_PER_MF = (NRD + NMF - 1) / NMF;
  auto ktile = [&](const bf16_t* lp, const bf16_t* lq, bf16_t* wp, bf16_t* wq, bool do_store,
                   auto&& issue_loads) {
    bf16x8_t pf[2][MI], qf[2][MJ];
#pragma unroll
    for (int a = 0; a < MI; ++a) pf[0][a] = read_frag<BI, PL>(lp, wi * WI + a * 32, 0, lane);
#pragma unroll
    for (int b = 0; b < MJ; ++b) qf[0][b] = read_frag<BJ, QL>(lq, wj * WJ + b * 32, 0, lane);
    __builtin_amdgcn_sched_barrier(0);
    static_for<kGemmBK / 16>([&](auto ksc) {
      constexpr int ks = decltype(ksc)::value;
      constexpr int cur = ks & 1;
      if constexpr (ks + 1 < kGemmBK / 16) {
#pragma unroll
        for (int a = 0; a < MI; ++a)
          pf[cur ^ 1][a] = read_frag<BI, PL>(lp, wi * WI + a * 32, ks + 1, lane);
#pragma unroll
        for (int b = 0; b < MJ; ++b)
          qf[cur ^ 1][b] = read_frag<BJ, QL>(lq, wj * WJ + b * 32, ks + 1, lane);
      }
      if constexpr (ks == 1) {
        if (do_store) {
          sp.store(wp);
          sq.store(wq);
        }
      }
      if constexpr (ks == 2) issue_loads();
#pragma unroll
      for (int a = 0; a < MI; ++a)
#pragma unroll
        for (int b = 0; b < MJ; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf[cur][a], qf[cur][b], acc[a][b], 0,
                                                              0, 0);
      sched_interleave<NMF, (ks + 1 < kGemmBK / 16) ? RD_PER_MF : 0, ks == 1 ? 1 : 0,
                       ks == 2 ? 1 : 0>();
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  auto load = [&](const GemmCursor& c) {
    if (c.kt == 0) {
      sp.setup(g.P, c.i0);
      sq.setup(g.Q, c.j0);
    }
    const int k0 = c.kb + c.kt * kGemmBK;
    sp.load(k0, min(c.ke, g.P.k_valid));
    sq.load(k0, min(c.ke, g.Q.k_valid));
  };

  // Two LDS stages, one register stage: the step after next waits in
  // registers while the current step is multiplied.
  GemmCursor lc, cc;
  lc.k = 0;
  gemm_decode<BI, BJ>(g, lc);
  cc = lc;
  if (lc.valid) {
    load(lc);
    sp.store(lds_p[0]);
    sq.store(lds_q[0]);
    gemm_advance<BI, BJ>(g, lc);
    if (lc.valid) load(lc);
  }
  __syncthreads();
  int stage = 0;
  while (cc.valid) {
    // registers hold the step after cc (when lc is valid): it goes to the other
    // LDS stage during this k-tile, then the step after that is loaded
    const bool have_next = lc.valid;
    ktile(lds_p[stage], lds_q[stage], lds_p[stage ^ 1], lds_q[stage ^ 1], have_next, [&] {
      if (have_next) {
        gemm_advance<BI, BJ>(g, lc);
        if (lc.valid) load(lc);
      }
    });
    if (cc.kt == cc.nk - 1) {
      // epilogue: lane holds column j = lane % 32 of each 32 x 32 block and rows
      // 8 (v / 4) + 4 (lane / 32) + v % 4 of it
#pragma unroll
      for (int a = 0; a < MI; ++a)
#pragma unroll
        for (int b = 0; b < MJ; ++b) {
          const int j = cc.j0 + wj * WJ + b * 32 + (lane & 31);
          const int i = cc.i0 + wi * WI + a * 32;
          epi.store_block(i, j, cc.split, lane, acc[a][b]);
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
        }
    }
    gemm_advance<BI, BJ>(g, cc);
    __syncthreads();
    stage ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Epilogues.  store_block(i, j, split, lane, v): v holds Out(i + 8 q + 4 (lane / 32)
// + e, j) at v[4 q + e], q, e = 0..3 (one lane's share of a 32-row block).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint2 pack4_bf16(const f32x16_t& v, int q) {
  return make_uint2(cvt_pk_bf16(v[4 * q], v[4 * q + 1]), cvt_pk_bf16(v[4 * q + 2], v[4 * q + 3]));
}

// Row-major bf16 output C[j][i] (i contiguous), rows j < j_valid, i < i_valid
// (i_valid a multiple of 4).
struct EpiRowBF16 {
  bf16_t* c;
  int64_t ldc;
  int i_valid, j_valid;
  // Batched output (blen > 0, direct-to-LDS kernel only): element (i, j) at
  // (i / blen) bstride + j ldc + i % blen; a tile's i range must lie in one batch.
  int64_t bstride = 0;
  int blen = 0;
  __device__ __forceinline__ void store_block(int i, int j, int, int lane,
                                              const f32x16_t& v) const {
    if (j >= j_valid) return;
    bf16_t* row = c + (int64_t)j * ldc + i + 4 * (lane >> 5);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (i + 8 * q + 4 * (lane >> 5) < i_valid)
        *reinterpret_cast<uint2*>(row + 8 * q) = pack4_bf16(v, q);
  }
};

// Row-major fp32 split-K partials C[split][j][i].
struct EpiRowF32Split {
  float* c;
  int64_t ldc, split_stride;
  int i_valid, j_valid;
  __device__ __forceinline__ void store_block(int i, int j, int split, int lane,
                                              const f32x16_t& v) const {
    if (j >= j_valid) return;
    float* row = c + (int64_t)split * split_stride + (int64_t)j * ldc + i + 4 * (lane >> 5);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (i + 8 * q + 4 * (lane >> 5) < i_valid)
        *reinterpret_cast<float4*>(row + 8 * q) =
            make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
  }
};

// Projection output, i = packed feature n, j = token m = b T + t:
//   n <  H D : value channel d = n % D of head h = n / D ->
//              values[((b H + h) T + t) D + d]           (head-major, bf16)
//   n >= H D : logit column n - H D ->  logits[m Lp + n - H D] (row-major, bf16)
// D and Lp are multiples of 4, so four consecutive n stay in one head / row;
// when D is a multiple of 32 the whole 32-row block is one head.
struct EpiProjectHM {
  bf16_t* values;
  bf16_t* logits;
  int H, D, T, Lp, n_logit_end, m_valid;
  __device__ __forceinline__ void store_block(int n, int m, int, int lane,
                                              const f32x16_t& v) const {
    if (m >= m_valid) return;
    const int HD = H * D;
    const int b = m / T, t = m - b * T;
    const int nl = n + 4 * (lane >> 5);
    if (D % 32 == 0 && n + 32 <= HD) {
      const int h = n / D, d = nl - h * D;
      bf16_t* dst = values + (((int64_t)b * H + h) * T + t) * D + d;
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<uint2*>(dst + 8 * q) = pack4_bf16(v, q);
      return;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nq = nl + 8 * q;
      if (nq < HD) {
        const int h = nq / D, d = nq - h * D;
        *reinterpret_cast<uint2*>(values + (((int64_t)b * H + h) * T + t) * D + d) =
            pack4_bf16(v, q);
      } else if (nq < n_logit_end) {
        *reinterpret_cast<uint2*>(logits + (int64_t)m * Lp + (nq - HD)) = pack4_bf16(v, q);
      }
    }
  }
};

}  // namespace ltv
