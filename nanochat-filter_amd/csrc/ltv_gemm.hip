// Fused QKV projection for gfx950: bf16 MFMA GEMMs (fp32 accumulate) for the
// filter module's fast path, and a strided SIMT GEMM for the reference-layout
// fused_linear_transpose op (fp32 or bf16 I/O).
//
// Reference: cpp_ewma/src/fused_linear_transpose_forward.cu:23-58 (one
// strided-batched GEMM, out[b] = W x[b]^T written (B, F, T)) and
// cpp_ewma/src/fused_linear_transpose_backward.cu:22-132 (B GEMMs for dX and B
// accumulating GEMMs for dW).  Here:
//   forward   C[M, Fp]  = X[M, C] . Wp^T           (A, B both K-contiguous)
//   backward  dX[M, C]  = dC[M, Fp] . Wp           (B operand N-contiguous)
//             dW[Fp, C] = dC^T . X  over all M     (both operands reduction-strided),
//             split over M into fp32 partials and reduced in a fixed order.
// Wp is the parameter with its rows regrouped [values, head-major | logits | 0].

#include "ltv_device.hpp"
#include "ltv_abi_internal.hpp"

#include <algorithm>

namespace ltv {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef float floatx16_v __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// MFMA GEMM: C[m, n] = sum_k A(m, k) B(n, k)
//   A_TRANS = false: A(m, k) at A[m * lda + k]   (K-contiguous)
//   A_TRANS = true : A(m, k) at A[k * lda + m]   (M-contiguous)
//   B likewise with n.
// Tile 128 x 128 x 64, 256 threads = 4 wavefronts in 2 x 2, each 64 x 64 made
// of 2 x 2 v_mfma_f32_32x32x16_bf16.  Operands staged K-contiguous in LDS
// (M/N-contiguous operands are transposed in registers on the way in),
// double-buffered with register prefetch: one barrier per K tile.
// ---------------------------------------------------------------------------
constexpr int GBM = 128, GBN = 128, GBK = 64;
constexpr int GPAD = 8;                 // bf16 elements of row padding in LDS
constexpr int GLDK = GBK + GPAD;        // LDS row pitch (elements)

enum { EPI_BF16 = 0, EPI_F32 = 1 };

struct MfmaArgs {
  const bf16_t* A;
  int64_t lda;
  const bf16_t* B;
  int64_t ldb;
  void* C;
  int64_t ldc;
  int64_t c_split_stride;  // elements between split-K partial outputs
  int M, N;
  int k_begin, k_len;      // this launch's reduction range (per split: k_len)
  int k_valid;             // A/B elements with k >= k_valid read as zero
  int m_valid, n_valid;    // stores limited to these
  int tiles_m, tiles_n;
};

// 4 (k) x 8 (row) block of bf16 -> 8 rows x 4 k (each uint2)
__device__ __forceinline__ void transpose4x8(const uint4 (&in)[4], uint2 (&out)[8]) {
  const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&in[0]);
  const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&in[1]);
  const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&in[2]);
  const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&in[3]);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // rows 2p (low halves) and 2p+1 (high halves)
    out[2 * p].x = __builtin_amdgcn_perm(w1[p], w0[p], 0x05040100u);
    out[2 * p].y = __builtin_amdgcn_perm(w3[p], w2[p], 0x05040100u);
    out[2 * p + 1].x = __builtin_amdgcn_perm(w1[p], w0[p], 0x07060302u);
    out[2 * p + 1].y = __builtin_amdgcn_perm(w3[p], w2[p], 0x07060302u);
  }
}

// zero the bf16 elements of a 16-byte chunk whose index k0 + e >= k_valid
__device__ __forceinline__ uint4 mask_tail(uint4 q, int k0, int k_valid) {
  if (k0 + 8 <= k_valid) return q;
  uint32_t* w = reinterpret_cast<uint32_t*>(&q);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t keep = 0;
    if (k0 + 2 * p < k_valid) keep |= 0x0000ffffu;
    if (k0 + 2 * p + 1 < k_valid) keep |= 0xffff0000u;
    w[p] &= keep;
  }
  return q;
}

// Per-thread staging registers for one operand tile.
struct TileRegs {
  uint4 q[4];
};

// K-contiguous operand: 128 rows x 64 k; thread loads rows (tid/8) + 32 i, k chunk (tid%8)*8
__device__ __forceinline__ void load_tile_k(const bf16_t* P, int64_t ld, int row0, int rows,
                                            int k0, int k_end, int k_valid, TileRegs& r) {
  const int tid = threadIdx.x;
  const int kc = (tid & 7) * 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (tid >> 3) + 32 * i;
    const int gr = row0 + row;
    const int gk = k0 + kc;
    uint4 q = make_uint4(0, 0, 0, 0);
    if (gr < rows && gk < k_end) {
      q = *reinterpret_cast<const uint4*>(P + (int64_t)gr * ld + gk);
      q = mask_tail(q, gk, min(k_valid, k_end));
    }
    r.q[i] = q;
  }
}

__device__ __forceinline__ void store_tile_k(bf16_t* lds, const TileRegs& r) {
  const int tid = threadIdx.x;
  const int kc = (tid & 7) * 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (tid >> 3) + 32 * i;
    *reinterpret_cast<uint4*>(lds + row * GLDK + kc) = r.q[i];
  }
}

// Row-contiguous operand: element (row, k) at P[k * ld + row]; thread loads k rows
// (tid/16)*4 .. +4, row chunk (tid%16)*8 .. +8.
__device__ __forceinline__ void load_tile_t(const bf16_t* P, int64_t ld, int row0, int rows,
                                            int k0, int k_end, int k_valid, TileRegs& r) {
  const int tid = threadIdx.x;
  const int rc = (tid & 15) * 8;
  const int kg = (tid >> 4) * 4;
  const int kmax = min(k_end, k_valid);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gk = k0 + kg + i;
    const int gr = row0 + rc;
    uint4 q = make_uint4(0, 0, 0, 0);
    if (gk < kmax && gr < rows) q = *reinterpret_cast<const uint4*>(P + (int64_t)gk * ld + gr);
    r.q[i] = q;
  }
}

__device__ __forceinline__ void store_tile_t(bf16_t* lds, const TileRegs& r) {
  const int tid = threadIdx.x;
  const int rc = (tid & 15) * 8;
  const int kg = (tid >> 4) * 4;
  uint2 o[8];
  transpose4x8(r.q, o);
#pragma unroll
  for (int e = 0; e < 8; ++e) *reinterpret_cast<uint2*>(lds + (rc + e) * GLDK + kg) = o[e];
}

template <bool A_TRANS, bool B_TRANS, int EPI>
__global__ void __launch_bounds__(256, 2) gemm_mfma_kernel(const MfmaArgs g) {
  __shared__ __attribute__((aligned(16))) bf16_t lds_a[2][GBM * GLDK];
  __shared__ __attribute__((aligned(16))) bf16_t lds_b[2][GBN * GLDK];

  // XCD-aware tile order: hardware hands workgroup i to XCD i % 8; give each
  // XCD a contiguous run of tiles (all N tiles of an M block in a row) so the
  // shared A rows stay in that XCD's L2.
  const int ntiles = g.tiles_m * g.tiles_n;
  int tile = blockIdx.x;
  {
    const int per = (ntiles + 7) / 8;
    const int xcd = tile % 8, idx = tile / 8;
    const int cand = xcd * per + idx;
    // fall back to identity order for the ragged remainder
    if (ntiles % 8 == 0) tile = cand;
  }
  const int tm = tile / g.tiles_n;
  const int tn = tile % g.tiles_n;
  const int m0 = tm * GBM, n0 = tn * GBN;
  const int split = blockIdx.y;
  const int kb = g.k_begin + split * g.k_len;
  const int ke = kb + g.k_len;

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int wm = wv >> 1, wn = wv & 1;

  floatx16_v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  TileRegs ra, rb;
  auto load = [&](int k0) {
    if (A_TRANS) load_tile_t(g.A, g.lda, m0, g.M, k0, ke, g.k_valid, ra);
    else load_tile_k(g.A, g.lda, m0, g.M, k0, ke, g.k_valid, ra);
    if (B_TRANS) load_tile_t(g.B, g.ldb, n0, g.N, k0, ke, g.k_valid, rb);
    else load_tile_k(g.B, g.ldb, n0, g.N, k0, ke, g.k_valid, rb);
  };
  auto stash = [&](int buf) {
    if (A_TRANS) store_tile_t(lds_a[buf], ra);
    else store_tile_k(lds_a[buf], ra);
    if (B_TRANS) store_tile_t(lds_b[buf], rb);
    else store_tile_k(lds_b[buf], rb);
  };

  const int nk = (ke - kb + GBK - 1) / GBK;
  if (nk > 0) {
    load(kb);
    stash(0);
  }
  __syncthreads();

  const int frow = lane & 31;
  const int fk = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load(kb + (kt + 1) * GBK);
    const bf16_t* la = lds_a[cur] + (wm * 64 + frow) * GLDK + fk;
    const bf16_t* lb = lds_b[cur] + (wn * 64 + frow) * GLDK + fk;
#pragma unroll
    for (int ks = 0; ks < GBK; ks += 16) {
      bf16x8_v af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        uint4 qa = *reinterpret_cast<const uint4*>(la + i * 32 * GLDK + ks);
        uint4 qb = *reinterpret_cast<const uint4*>(lb + i * 32 * GLDK + ks);
        af[i] = __builtin_bit_cast(bf16x8_v, qa);
        bfr[i] = __builtin_bit_cast(bf16x8_v, qb);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) stash(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds column (lane % 32) of each 32 x 32 block, rows
  // 8 * (v / 4) + 4 * (lane / 32) + v % 4
  const int col = lane & 31;
  const int rbase = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 64 + j * 32 + col;
      if (n >= g.n_valid) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + rbase + (v & 3);
        if (m >= g.m_valid) continue;
        if (EPI == EPI_BF16) {
          reinterpret_cast<bf16_t*>(g.C)[(int64_t)m * g.ldc + n] =
              (bf16_t)f32_to_bf16_bits(acc[i][j][v]);
        } else {
          reinterpret_cast<float*>(g.C)[(int64_t)split * g.c_split_stride + (int64_t)m * g.ldc + n] =
              acc[i][j][v];
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Weight packing: parameter rows (per head: D values then Da logits) ->
// wpack rows [h*D + d | H*D + h*Da + j | zero padding up to Fp], cast to bf16.
// ---------------------------------------------------------------------------
template <typename TW>
__global__ void pack_weight_kernel(const TW* __restrict__ w, bf16_t* __restrict__ wp, int H,
                                   int D, int Da, int C, int Fp) {
  const int64_t total = (int64_t)Fp * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int fpk = (int)(i / C);
    const int c = (int)(i % C);
    float v = 0.0f;
    if (fpk < H * D) {
      const int h = fpk / D, d = fpk % D;
      v = io_traits<TW>::load(w + (int64_t)(h * (D + Da) + d) * C + c);
    } else if (fpk < H * D + H * Da) {
      const int q = fpk - H * D;
      const int h = q / Da, j = q % Da;
      v = io_traits<TW>::load(w + (int64_t)(h * (D + Da) + D + j) * C + c);
    }
    wp[i] = (bf16_t)f32_to_bf16_bits(v);
  }
}

// grad_weight[param row, c] = sum_s partial[s][packed row, c]  (fixed order)
__global__ void dw_reduce_kernel(const float* __restrict__ part, float* __restrict__ gw, int S,
                                 int64_t split_stride, int H, int D, int Da, int C) {
  const int F = H * (D + Da);
  const int64_t total = (int64_t)F * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int f = (int)(i / C);
    const int c = (int)(i % C);
    const int h = f / (D + Da), e = f % (D + Da);
    const int fpk = e < D ? h * D + e : H * D + h * Da + (e - D);
    float acc = 0.0f;
    for (int s = 0; s < S; ++s) acc += part[(int64_t)s * split_stride + (int64_t)fpk * C + c];
    gw[i] = acc;
  }
}

// ---------------------------------------------------------------------------
// Strided SIMT GEMM (any layout, fp32 or bf16 in, fp32 accumulate):
//   C(m, n) = sum_kk A(m, kk) B(n, kk)
// where the reduction index kk = ko * kin + ki addresses
//   A + m*sam + ko*sako + ki*saki,  B + n*sbn + ko*sbko + ki*sbki,
// and blockIdx.z selects a batch (a/b/c batch strides).  64 x 64 tiles,
// 256 threads with 4 x 4 outputs each.
// ---------------------------------------------------------------------------
struct SimtArgs {
  const void* A;
  int64_t sam, sako, saki, sab;
  const void* B;
  int64_t sbn, sbko, sbki, sbb;
  void* C;
  int64_t scm, scn, scb;
  int M, N, K, kin;
};

template <typename TI, typename TO>
__global__ void __launch_bounds__(256) gemm_simt_kernel(const SimtArgs g) {
  constexpr int BM = 64, BN = 64, BK = 16;
  __shared__ float sa[BK][BM + 1];
  __shared__ float sb[BK][BN + 1];
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int z = blockIdx.z;
  const TI* A = reinterpret_cast<const TI*>(g.A) + (int64_t)z * g.sab;
  const TI* B = reinterpret_cast<const TI*>(g.B) + (int64_t)z * g.sbb;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < g.K; k0 += BK) {
    for (int e = threadIdx.x; e < BK * BM; e += 256) {
      const int kk = e / BM, mm = e % BM;
      const int m = m0 + mm, k = k0 + kk;
      float v = 0.0f;
      if (m < g.M && k < g.K) {
        const int ko = k / g.kin, ki = k % g.kin;
        v = io_traits<TI>::load(A + (int64_t)m * g.sam + (int64_t)ko * g.sako + (int64_t)ki * g.saki);
      }
      sa[kk][mm] = v;
    }
    for (int e = threadIdx.x; e < BK * BN; e += 256) {
      const int kk = e / BN, nn = e % BN;
      const int n = n0 + nn, k = k0 + kk;
      float v = 0.0f;
      if (n < g.N && k < g.K) {
        const int ko = k / g.kin, ki = k % g.kin;
        v = io_traits<TI>::load(B + (int64_t)n * g.sbn + (int64_t)ko * g.sbko + (int64_t)ki * g.sbki);
      }
      sb[kk][nn] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = sa[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = sb[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
  TO* C = reinterpret_cast<TO*>(g.C) + (int64_t)z * g.scb;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty + 16 * i, n = n0 + tx + 16 * j;
      if (m < g.M && n < g.N) io_traits<TO>::store(C + (int64_t)m * g.scm + (int64_t)n * g.scn, acc[i][j]);
    }
}

}  // namespace ltv

// ===========================================================================
// Host side
// ===========================================================================
using namespace ltv;

namespace {

int launch_simt(int dtype_in, int dtype_out, const SimtArgs& a, int batches, hipStream_t st) {
  if (a.M == 0 || a.N == 0 || batches == 0) return LTV_OK;
  dim3 grid((a.N + 63) / 64, (a.M + 63) / 64, batches);
  if (dtype_in == LTV_DTYPE_F32 && dtype_out == LTV_DTYPE_F32)
    hipLaunchKernelGGL((gemm_simt_kernel<float, float>), grid, dim3(256), 0, st, a);
  else if (dtype_in == LTV_DTYPE_BF16 && dtype_out == LTV_DTYPE_BF16)
    hipLaunchKernelGGL((gemm_simt_kernel<bf16_t, bf16_t>), grid, dim3(256), 0, st, a);
  else if (dtype_in == LTV_DTYPE_BF16 && dtype_out == LTV_DTYPE_F32)
    hipLaunchKernelGGL((gemm_simt_kernel<bf16_t, float>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_simt_kernel<float, bf16_t>), grid, dim3(256), 0, st, a);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

template <bool AT, bool BT, int EPI>
int launch_mfma(const MfmaArgs& a, int splits, hipStream_t st) {
  dim3 grid(a.tiles_m * a.tiles_n, splits);
  hipLaunchKernelGGL((gemm_mfma_kernel<AT, BT, EPI>), grid, dim3(256), 0, st, a);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

inline int dsize(int dtype) { return dtype == LTV_DTYPE_BF16 ? 2 : 4; }

}  // namespace

extern "C" int ltv_linear_transpose_forward(int dtype, const void* x, const void* weight,
                                            void* out, int B, int T, int K, int F,
                                            void* stream) {
  LTV_REQUIRE(dtype == LTV_DTYPE_F32 || dtype == LTV_DTYPE_BF16, LTV_ERR_INVALID_ARG,
              "dtype must be LTV_DTYPE_F32 or LTV_DTYPE_BF16, got %d", dtype);
  LTV_REQUIRE(B >= 0 && T >= 0 && K >= 0 && F >= 0, LTV_ERR_INVALID_ARG, "negative size");
  if ((int64_t)B * T * F == 0) return LTV_OK;
  LTV_REQUIRE(x && weight && out, LTV_ERR_INVALID_ARG, "null tensor pointer");
  // per batch: out_b (F x T) = W (F x K) . x_b^T
  SimtArgs a;
  a.A = weight; a.sam = K; a.sako = 0; a.saki = 1; a.sab = 0;
  a.B = x; a.sbn = K; a.sbko = 0; a.sbki = 1; a.sbb = (int64_t)T * K;
  a.C = out; a.scm = T; a.scn = 1; a.scb = (int64_t)F * T;
  a.M = F; a.N = T; a.K = K; a.kin = K > 0 ? K : 1;
  return launch_simt(dtype, dtype, a, B, (hipStream_t)stream);
}

extern "C" int ltv_linear_transpose_backward(int dtype, const void* x, const void* weight,
                                             const void* grad_out, int grad_out_is_btf,
                                             void* grad_x, void* grad_weight, int B, int T,
                                             int K, int F, void* stream) {
  LTV_REQUIRE(dtype == LTV_DTYPE_F32 || dtype == LTV_DTYPE_BF16, LTV_ERR_INVALID_ARG,
              "dtype must be LTV_DTYPE_F32 or LTV_DTYPE_BF16, got %d", dtype);
  LTV_REQUIRE(B >= 0 && T >= 0 && K >= 0 && F >= 0, LTV_ERR_INVALID_ARG, "negative size");
  LTV_REQUIRE(x && weight && grad_out && grad_x && grad_weight, LTV_ERR_INVALID_ARG,
              "null tensor pointer");
  hipStream_t st = (hipStream_t)stream;
  // grad_out element (b, f, t): (B,F,T) -> b*F*T + f*T + t ; (B,T,F) -> b*T*F + t*F + f
  const int64_t go_f = grad_out_is_btf ? 1 : T;
  const int64_t go_t = grad_out_is_btf ? F : 1;
  // grad_x_b (T x K) = sum_f go_b(f, t) W(f, k)
  SimtArgs a;
  a.A = grad_out; a.sam = go_t; a.sako = 0; a.saki = go_f; a.sab = (int64_t)F * T;
  a.B = weight; a.sbn = 1; a.sbko = 0; a.sbki = K; a.sbb = 0;
  a.C = grad_x; a.scm = K; a.scn = 1; a.scb = (int64_t)T * K;
  a.M = T; a.N = K; a.K = F; a.kin = F > 0 ? F : 1;
  int rc = launch_simt(dtype, dtype, a, B, st);
  if (rc) return rc;
  // grad_W (F x K) = sum_{b,t} go(b, f, t) x(b, t, k); reduction index kk = b*T + t
  SimtArgs w;
  w.A = grad_out; w.sam = go_f; w.sako = (int64_t)F * T; w.saki = go_t; w.sab = 0;
  w.B = x; w.sbn = 1; w.sbko = (int64_t)T * K; w.sbki = K; w.sbb = 0;
  w.C = grad_weight; w.scm = K; w.scn = 1; w.scb = 0;
  w.M = F; w.N = K; w.K = B * T; w.kin = T > 0 ? T : 1;
  if (w.K == 0) {
    LTV_HIP_CHECK(hipMemsetAsync(grad_weight, 0, (size_t)F * K * dsize(dtype), st));
    return LTV_OK;
  }
  return launch_simt(dtype, dtype, w, 1, st);
}

extern "C" int ltv_qkv_packed_width(int H, int D, int Da) {
  const int F = H * D + H * Da;
  return (F + 63) / 64 * 64;
}

extern "C" int ltv_qkv_pack_weight(int weight_dtype, const void* weight, void* wpack, int H,
                                   int D, int Da, int C, void* stream) {
  LTV_REQUIRE(weight_dtype == LTV_DTYPE_F32 || weight_dtype == LTV_DTYPE_BF16,
              LTV_ERR_INVALID_ARG, "bad weight dtype %d", weight_dtype);
  LTV_REQUIRE(H > 0 && D > 0 && Da > 0 && C > 0, LTV_ERR_INVALID_ARG, "bad shape");
  LTV_REQUIRE(weight && wpack, LTV_ERR_INVALID_ARG, "null tensor pointer");
  const int Fp = ltv_qkv_packed_width(H, D, Da);
  const int64_t total = (int64_t)Fp * C;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
  hipStream_t st = (hipStream_t)stream;
  if (weight_dtype == LTV_DTYPE_F32)
    hipLaunchKernelGGL(pack_weight_kernel<float>, dim3(blocks), dim3(256), 0, st,
                       reinterpret_cast<const float*>(weight), reinterpret_cast<bf16_t*>(wpack),
                       H, D, Da, C, Fp);
  else
    hipLaunchKernelGGL(pack_weight_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st,
                       reinterpret_cast<const bf16_t*>(weight), reinterpret_cast<bf16_t*>(wpack),
                       H, D, Da, C, Fp);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

extern "C" int ltv_qkv_project_forward(const void* x, const void* wpack, void* combined, int M,
                                       int C, int Fp, void* stream) {
  LTV_REQUIRE(M >= 0 && C > 0 && Fp > 0, LTV_ERR_INVALID_ARG, "bad shape");
  LTV_REQUIRE(C % 8 == 0 && Fp % 8 == 0, LTV_ERR_UNSUPPORTED,
              "C and Fp must be multiples of 8 (C=%d Fp=%d)", C, Fp);
  if (M == 0) return LTV_OK;
  LTV_REQUIRE(x && wpack && combined, LTV_ERR_INVALID_ARG, "null tensor pointer");
  LTV_REQUIRE(aligned16(x) && aligned16(wpack) && aligned16(combined), LTV_ERR_INVALID_ARG,
              "x, wpack and combined must be 16-byte aligned");
  MfmaArgs a;
  a.A = reinterpret_cast<const bf16_t*>(x); a.lda = C;
  a.B = reinterpret_cast<const bf16_t*>(wpack); a.ldb = C;
  a.C = combined; a.ldc = Fp; a.c_split_stride = 0;
  a.M = M; a.N = Fp; a.k_begin = 0; a.k_len = C; a.k_valid = C;
  a.m_valid = M; a.n_valid = Fp;
  a.tiles_m = (M + GBM - 1) / GBM; a.tiles_n = (Fp + GBN - 1) / GBN;
  return launch_mfma<false, false, EPI_BF16>(a, 1, (hipStream_t)stream);
}

namespace {
constexpr int kDwSplitRows = 4096;  // rows of M reduced by one split of the dW GEMM
inline int dw_splits(int M) { return std::max(1, (M + kDwSplitRows - 1) / kDwSplitRows); }
}  // namespace

extern "C" size_t ltv_qkv_project_backward_workspace_size(int M, int C, int H, int D, int Da) {
  const int Fp = ltv_qkv_packed_width(H, D, Da);
  const int Fr = (Fp + GBM - 1) / GBM * GBM;
  return (size_t)dw_splits(M) * Fr * C * sizeof(float);
}

extern "C" int ltv_qkv_project_backward(const void* x, const void* wpack,
                                        const void* grad_combined, void* grad_x,
                                        float* grad_weight, void* workspace,
                                        size_t workspace_bytes, int M, int C, int H, int D,
                                        int Da, void* stream) {
  LTV_REQUIRE(M >= 0 && C > 0 && H > 0 && D > 0 && Da > 0, LTV_ERR_INVALID_ARG, "bad shape");
  LTV_REQUIRE(C % 8 == 0, LTV_ERR_UNSUPPORTED, "C must be a multiple of 8 (C=%d)", C);
  LTV_REQUIRE(x && wpack && grad_combined && grad_x && grad_weight, LTV_ERR_INVALID_ARG,
              "null tensor pointer");
  const int Fp = ltv_qkv_packed_width(H, D, Da);
  const int Fvalid = H * (D + Da);
  hipStream_t st = (hipStream_t)stream;
  if (M == 0) {
    LTV_HIP_CHECK(hipMemsetAsync(grad_weight, 0, (size_t)Fvalid * C * sizeof(float), st));
    return LTV_OK;
  }
  const size_t need = ltv_qkv_project_backward_workspace_size(M, C, H, D, Da);
  LTV_REQUIRE(workspace && workspace_bytes >= need, LTV_ERR_WORKSPACE,
              "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  // dX[M, C] = dC[M, Fp] . Wp[Fp, C]: B(n = c, k = f) at Wp[f * C + c] (N-contiguous)
  MfmaArgs a;
  a.A = reinterpret_cast<const bf16_t*>(grad_combined); a.lda = Fp;
  a.B = reinterpret_cast<const bf16_t*>(wpack); a.ldb = C;
  a.C = grad_x; a.ldc = C; a.c_split_stride = 0;
  a.M = M; a.N = C; a.k_begin = 0; a.k_len = Fp; a.k_valid = Fvalid;
  a.m_valid = M; a.n_valid = C;
  a.tiles_m = (M + GBM - 1) / GBM; a.tiles_n = (C + GBN - 1) / GBN;
  int rc = launch_mfma<false, true, EPI_BF16>(a, 1, st);
  if (rc) return rc;
  // dW partials: P_s[f, c] = sum_{m in split s} dC[m, f] X[m, c]
  const int S = dw_splits(M);
  const int Fr = (Fp + GBM - 1) / GBM * GBM;
  MfmaArgs w;
  w.A = reinterpret_cast<const bf16_t*>(grad_combined); w.lda = Fp;   // A(f, m) at dC[m*Fp + f]
  w.B = reinterpret_cast<const bf16_t*>(x); w.ldb = C;                // B(c, m) at X[m*C + c]
  w.C = workspace; w.ldc = C; w.c_split_stride = (int64_t)Fr * C;
  w.M = Fvalid; w.N = C; w.k_begin = 0; w.k_len = kDwSplitRows; w.k_valid = M;
  w.m_valid = Fr; w.n_valid = C;
  w.tiles_m = Fr / GBM; w.tiles_n = (C + GBN - 1) / GBN;
  rc = launch_mfma<true, true, EPI_F32>(w, S, st);
  if (rc) return rc;
  const int64_t total = (int64_t)Fvalid * C;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL(dw_reduce_kernel, dim3(blocks), dim3(256), 0, st,
                     reinterpret_cast<const float*>(workspace), grad_weight, S,
                     (int64_t)Fr * C, H, D, Da, C);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}
