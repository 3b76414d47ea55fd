// Fused QKV projection for gfx950: bf16 MFMA GEMMs (fp32 accumulate) for the
// filter module's fast path, and the reference-layout fused_linear_transpose
// op (fp32 or bf16 I/O) on the bf16 direct-to-LDS kernels where its layout
// allows, else on the strided fp32-MFMA GEMM of ltv_gemm_f32.hpp.
//
// Reference: cpp_ewma/src/fused_linear_transpose_forward.cu:23-58 (one
// strided-batched GEMM, out[b] = W x[b]^T written (B, F, T)) and
// cpp_ewma/src/fused_linear_transpose_backward.cu:22-132 (B GEMMs for dX and B
// accumulating GEMMs for dW).  Here (M = B T tokens, Wp the parameter with its
// rows regrouped [values, head-major | logits | zero pad], Fp rows):
//   forward   values[B, H, T, D] | logits[M, Lp]  =  X[M, C] . Wp^T
//             one launch; the epilogue writes the scan's head-major layout
//   backward  dX[M, C]   = dC[M, Fp] . Wp                (Wp read transposed from LDS)
//             dW^T[C, Fp] = X^T . dC  over all M          (both operands read transposed),
//             split over M into fp32 partials, reduced in a fixed order into the
//             parameter's interleaved row order.

#include "ltv_device.hpp"
#include "ltv_abi_internal.hpp"
#include "ltv_gemm_dma.hpp"
#include "ltv_gemm_f32.hpp"

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

namespace ltv {

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

// The same packing, 8 columns per thread (C % 8 == 0, 16-byte aligned
// buffers, Fp * C < 2^31): 16-byte loads and stores, 32-bit index arithmetic,
// the same rounding per element.
template <typename TW>
__global__ void __launch_bounds__(256)
pack_weight8_kernel(const TW* __restrict__ w, bf16_t* __restrict__ wp, int H, int D, int Da, int C,
                    int Fp) {
  const int C8 = C / 8;
  const int total = Fp * C8;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const int fpk = i / C8, c = (i - fpk * C8) * 8;
    int src = -1;  // parameter row of packed row fpk (-1: padding)
    if (fpk < H * D) {
      const int h = fpk / D;
      src = h * (D + Da) + (fpk - h * D);
    } else if (fpk < H * (D + Da)) {
      const int q = fpk - H * D, h = q / Da;
      src = h * (D + Da) + D + (q - h * Da);
    }
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = 0.0f;
    if (src >= 0) {
      const TW* p = w + (int64_t)src * C + c;
      if constexpr (sizeof(TW) == 4) {
        const float4 a = reinterpret_cast<const float4*>(p)[0];
        const float4 b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      } else {
        const uint4 q = *reinterpret_cast<const uint4*>(p);
        const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[2 * k] = __uint_as_float(u[k] << 16);
          v[2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
        }
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = (uint32_t)f32_to_bf16_bits(v[2 * k]) | ((uint32_t)f32_to_bf16_bits(v[2 * k + 1]) << 16);
    *reinterpret_cast<uint4*>(wp + (int64_t)i * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// zero columns [c0, c1) of a row-major bf16 (rows, ld) buffer: one thread per
// row, 4-byte stores where the row's strip is 4-byte aligned
__global__ void __launch_bounds__(256)
zero_cols_kernel(bf16_t* __restrict__ p, int rows, int64_t ld, int c0, int c1) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  bf16_t* q = p + (int64_t)r * ld;
  int c = c0;
  if (c < c1 && ((uintptr_t)(q + c) & 2)) q[c++] = 0;
  for (; c + 2 <= c1; c += 2) *reinterpret_cast<uint32_t*>(q + c) = 0u;
  if (c < c1) q[c] = 0;
}

// out[f, k] = sum_s part[s][f, k]  (rows in their own order; fixed order,
// deterministic), written as TO.
template <typename TO>
__global__ void __launch_bounds__(256)
reduce_splits_kernel(const float* __restrict__ part, TO* __restrict__ out, int S,
                     int64_t split_stride, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    float acc = 0.0f;
    for (int s = 0; s < S; ++s) acc += __builtin_nontemporal_load(&part[(int64_t)s * split_stride + i]);
    io_traits<TO>::store(out + i, acc);
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
    for (int s = 0; s < S; ++s)
      acc += __builtin_nontemporal_load(&part[(int64_t)s * split_stride + (int64_t)fpk * C + c]);
    gw[i] = acc;
  }
}

// The same sum, 4 columns per thread (C % 4 == 0, 16-byte aligned buffers,
// F * C < 2^31): 16-byte loads and stores, 32-bit index arithmetic, and the
// partials' loads issued 8 at a time.  The additions run in the same order
// (s = 0 .. S - 1 from 0), so the result is bit-identical.  The partials are
// read once: streaming (nt) loads keep them from evicting what the next
// kernels read (measured at d12: the next step's forward GEMM and scan
// 2-3 us faster).
__device__ __forceinline__ float4 ld_stream4(const float4* p) {
  typedef float f4_t __attribute__((ext_vector_type(4)));
  const f4_t q = __builtin_nontemporal_load(reinterpret_cast<const f4_t*>(p));
  return make_float4(q[0], q[1], q[2], q[3]);
}

__global__ void __launch_bounds__(256)
dw_reduce4_kernel(const float4* __restrict__ part, float4* __restrict__ gw, int S,
                  int64_t split_stride4, int H, int D, int Da, int C4) {
  const int DE = D + Da;
  const int total = H * DE * C4;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const int f = i / C4, c = i - f * C4;
    const int h = f / DE, e = f - h * DE;
    const int fpk = e < D ? h * D + e : H * D + h * Da + (e - D);
    const float4* p = part + (int64_t)fpk * C4 + c;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int s = 0;
    for (; s + 8 <= S; s += 8) {
      float4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = ld_stream4(&p[(int64_t)(s + j) * split_stride4]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc.x += v[j].x;
        acc.y += v[j].y;
        acc.z += v[j].z;
        acc.w += v[j].w;
      }
    }
    for (; s < S; ++s) {
      const float4 v = ld_stream4(&p[(int64_t)s * split_stride4]);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    gw[i] = acc;
  }
}

}  // namespace ltv

// ===========================================================================
// Host side
// ===========================================================================
using namespace ltv;

namespace {

// Staging form of one operand of the fp32-MFMA GEMM (row stride sr, reduction
// strides sko / ski, batch stride sbatch): quads need 4-element-aligned
// starts, and a KQ quad must not straddle two outer reduction indices.
int f32m_stage(const void* p, int64_t sr, int64_t sko, int64_t ski, int64_t sbatch, int batches,
               int kin, int K, int esize) {
  const bool aligned =
      (reinterpret_cast<uintptr_t>(p) % (uintptr_t)(4 * esize)) == 0 &&
      (batches <= 1 || sbatch % 4 == 0);
  const bool outer = kin < K;
  if (aligned && ski == 1 && sr % 4 == 0 && (!outer || (kin % 4 == 0 && sko % 4 == 0)))
    return kF32KQ;
  if (aligned && sr == 1 && ski % 4 == 0 && (!outer || sko % 4 == 0)) return kF32MQ;
  return kF32SC;
}

template <typename TI, typename TO, int LA>
void f32m_launch_b(int lb, const F32mArgs& a, dim3 grid, hipStream_t st) {
  if (lb == kF32KQ)
    hipLaunchKernelGGL((gemm_f32m_kernel<TI, TO, LA, kF32KQ>), grid, dim3(kF32Threads), 0, st, a);
  else if (lb == kF32MQ)
    hipLaunchKernelGGL((gemm_f32m_kernel<TI, TO, LA, kF32MQ>), grid, dim3(kF32Threads), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_f32m_kernel<TI, TO, LA, kF32SC>), grid, dim3(kF32Threads), 0, st, a);
}

template <typename TI, typename TO>
void f32m_launch_ab(int la, int lb, const F32mArgs& a, dim3 grid, hipStream_t st) {
  if (la == kF32KQ)
    f32m_launch_b<TI, TO, kF32KQ>(lb, a, grid, st);
  else if (la == kF32MQ)
    f32m_launch_b<TI, TO, kF32MQ>(lb, a, grid, st);
  else
    f32m_launch_b<TI, TO, kF32SC>(lb, a, grid, st);
}

// C (dtype_out; fp32 for split partials) = A . B^T over `batches` batches and
// `splits` reduction splits of k_split indices each (splits = 1: k_split is
// ignored), on the fp32-MFMA GEMM.
int launch_f32m(int dtype_in, int dtype_out, F32mArgs a, int batches, int splits, int k_split,
                hipStream_t st) {
  if (a.M == 0 || a.N == 0 || batches == 0) return LTV_OK;
  LTV_REQUIRE((dtype_in == LTV_DTYPE_F32 && dtype_out == LTV_DTYPE_F32) ||
                  (dtype_in == LTV_DTYPE_BF16 &&
                   (dtype_out == LTV_DTYPE_BF16 || dtype_out == LTV_DTYPE_F32)),
              LTV_ERR_UNSUPPORTED, "fp32-MFMA GEMM: unsupported dtypes %d -> %d", dtype_in,
              dtype_out);
  a.splits = std::max(1, splits);
  a.k_split = a.splits == 1 ? a.K : k_split;
  LTV_REQUIRE(a.splits == 1 || (a.k_split > 0 && a.k_split % kF32BK == 0 &&
                                (int64_t)a.k_split * a.splits >= a.K),
              LTV_ERR_INVALID_ARG, "bad reduction split (%d x %d for K = %d)", a.splits,
              a.k_split, a.K);
  const int64_t gy = (a.M + kF32B - 1) / kF32B, gz = (int64_t)batches * a.splits;
  LTV_REQUIRE(gy <= 65535 && gz <= 65535, LTV_ERR_UNSUPPORTED,
              "fp32-MFMA GEMM grid too large (%lld row tiles, %lld batches x splits)",
              (long long)gy, (long long)gz);
  const dim3 grid((a.N + kF32B - 1) / kF32B, (unsigned)gy, (unsigned)gz);
  const int es = dtype_in == LTV_DTYPE_BF16 ? 2 : 4;
  const int la = f32m_stage(a.A, a.sam, a.sako, a.saki, a.sab, batches, a.kin, a.K, es);
  const int lb = f32m_stage(a.B, a.sbn, a.sbko, a.sbki, a.sbb, batches, a.kin, a.K, es);
  if (dtype_in == LTV_DTYPE_F32)
    f32m_launch_ab<float, float>(la, lb, a, grid, st);
  else if (dtype_out == LTV_DTYPE_BF16)
    f32m_launch_ab<bf16_t, bf16_t>(la, lb, a, grid, st);
  else
    f32m_launch_ab<bf16_t, float>(la, lb, a, grid, st);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

// Compute units of the current device (cached per device).
int device_cu_count() {
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

// Persistent launch: one workgroup per compute unit (the tiles use most of the
// LDS), or fewer when there are fewer work items.
// Elements an operand spans: rows x k for K-contiguous (ld = row pitch), k x rows for
// row-contiguous (ld = k pitch).
inline int64_t operand_span(const GemmOperand& o, int K, int layout) {
  if (o.blen > 0) return dma_batched_span(o, K, layout);
  return layout == OP_KC ? (int64_t)o.rows * o.ld : (int64_t)K * o.ld;
}

template <int BI, int BJ, int WGI, int WGJ, int PL, int QL, class Epi>
int launch_gemm(GemmArgs a, const Epi& e, int splits, hipStream_t st) {
  LTV_REQUIRE(operand_span(a.P, a.K, PL) < (1ll << 31) && operand_span(a.Q, a.K, QL) < (1ll << 31),
              LTV_ERR_UNSUPPORTED, "GEMM operand spans 2^31 elements or more");
  a.splits = splits;
  const int total = a.tiles_i * a.tiles_j * splits;
  if (total == 0) return LTV_OK;
  int grid = device_cu_count();
  if (total < grid) grid = total;
  hipLaunchKernelGGL((gemm_bf16_kernel<BI, BJ, WGI, WGJ, PL, QL, Epi>), dim3(grid),
                     dim3(WGI * WGJ * 64), 0, st, a, e);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

// Whether the direct-to-LDS kernel takes these operands: spans within its
// 32-bit offsets, KC reduction ends at 8-element chunks, RC rows in 8-row chunks.
inline bool dma_ok(const GemmOperand& op, int64_t K, int layout) {
  if (operand_span(op, K, layout) > kDmaMaxSpan) return false;
  if (layout == OP_KC) return op.k_valid % 8 == 0 && op.ld % 8 == 0;
  return op.rows % 8 == 0 && op.ld % 8 == 0;
}

// Largest output buffer an epilogue of the direct-to-LDS kernel addresses.
inline int64_t dma_epi_bytes(const EpiRowBF16& e, int) { return epi_row_bf16_bytes(e); }
inline int64_t dma_epi_bytes(const EpiRowF32Split& e, int splits) {
  return (int64_t)splits * e.split_stride * 4;
}
inline int64_t dma_epi_bytes(const EpiProjectHM& e, int) {
  return std::max((int64_t)e.m_valid * e.H * e.D * 2, (int64_t)e.m_valid * e.Lp * 2);
}

template <class Epi>
bool dma_usable(const GemmArgs& a, int PL, int QL, const Epi& e, int splits) {
  return dma_ok(a.P, a.K, PL) && dma_ok(a.Q, a.K, QL) && dma_epi_bytes(e, splits) <= kDmaMaxBytes;
}

// Same, with the direct-to-LDS kernel.
template <int BI, int BJ, int WGI, int WGJ, int PL, int QL, class Epi>
int launch_gemm_dma(GemmArgs a, const Epi& e, int splits, hipStream_t st) {
  LTV_REQUIRE(dma_usable(a, PL, QL, e, splits), LTV_ERR_UNSUPPORTED,
              "operands not supported by the direct-to-LDS GEMM");
  a.splits = splits;
  const int total = a.tiles_i * a.tiles_j * splits;
  if (total == 0) return LTV_OK;
  int grid = device_cu_count();
  if (total < grid) grid = total;
  hipLaunchKernelGGL((gemm_dma_kernel<BI, BJ, WGI, WGJ, PL, QL, Epi>), dim3(grid),
                     dim3(WGI * WGJ * 64), 0, st, a, e);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}

// Tile variants of the three projection GEMMs, overridable for tuning with
// LTV_GEMM_CFG="fwd,dx,dw,dw_split_rows[,dma]" (variant indices, rows per dW
// split, 1 = direct-to-LDS kernels).
// Defaults measured on MI355X at d12: 256 x 256 tiles with 8 wavefronts for the
// forward and dX, 128 x 256 tiles with 8192-row splits for dW.
struct GemmTuning {
  int fwd = 1, dx = 1, dw = 0, dw_split = 0, dma = 1;  // dw_split 0: automatic
  GemmTuning() {
    if (const char* e = getenv("LTV_GEMM_CFG")) {
      int a = 0, b = 0, c = 0, d = 4096, f = 0;
      const int n = sscanf(e, "%d,%d,%d,%d,%d", &a, &b, &c, &d, &f);
      if (n >= 4 && d > 0 && d % kGemmBK == 0) {
        fwd = a;
        dx = b;
        dw = c;
        dw_split = d;
        dma = n == 5 ? f : 1;
      }
    }
  }
};

const GemmTuning& gemm_tuning() {
  static const GemmTuning t;
  return t;
}

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

}  // namespace

extern "C" int ltv_linear_transpose_forward(int dtype, const void* x, const void* weight,
                                            void* out, int B, int T, int K, int F,
                                            void* stream) {
  LTV_REQUIRE(dtype == LTV_DTYPE_F32 || dtype == LTV_DTYPE_BF16, LTV_ERR_INVALID_ARG,
              "dtype must be LTV_DTYPE_F32 or LTV_DTYPE_BF16, got %d", dtype);
  LTV_REQUIRE(B >= 0 && T >= 0 && K >= 0 && F >= 0, LTV_ERR_INVALID_ARG, "negative size");
  if ((int64_t)B * T * F == 0) return LTV_OK;
  // an empty reduction (K = 0) reads neither operand and writes zeros
  LTV_REQUIRE(out && (K == 0 || (x && weight)), LTV_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == LTV_DTYPE_BF16 && gemm_tuning().dma && T % 256 == 0 && K % 8 == 0 && K > 0 &&
      aligned16(x) && aligned16(weight) && aligned16(out) && (int64_t)B * T < (1ll << 31)) {
    // bf16 MFMA: Out(i = token m, j = feature f) = sum_k x[m, k] W[f, k] written
    // to out[b, f, t] (m = b T + t): i runs along t, batches F T apart
    const int M = B * T;
    GemmArgs g;
    g.P = GemmOperand{reinterpret_cast<const bf16_t*>(x), K, M, K};       // (m, k) KC
    g.Q = GemmOperand{reinterpret_cast<const bf16_t*>(weight), K, F, K};  // (f, k) KC
    g.K = K;
    g.k_split = round_up(K, kGemmBK);
    EpiRowBF16 e{reinterpret_cast<bf16_t*>(out), T, M, F};
    e.bstride = (int64_t)F * T;
    e.blen = T;
    if (dma_usable(g, OP_KC, OP_KC, e, 1)) {
      g.tiles_i = M / 256;
      g.tiles_j = (F + 255) / 256;
      return launch_gemm_dma<256, 256, 2, 4, OP_KC, OP_KC>(g, e, 1, st);
    }
  }
  // per batch: out_b (F x T) = W (F x K) . x_b^T
  F32mArgs a{};
  a.A = weight; a.sam = K; a.sako = 0; a.saki = 1; a.sab = 0;
  a.B = x; a.sbn = K; a.sbko = 0; a.sbki = 1; a.sbb = (int64_t)T * K;
  a.C = out; a.scm = T; a.scn = 1; a.scb = (int64_t)F * T;
  a.M = F; a.N = T; a.K = K; a.kin = K > 0 ? K : 1;
  return launch_f32m(dtype, dtype, a, B, 1, 0, st);
}

namespace {
// The bf16 direct-to-LDS path of the reference-layout backward: grad_out
// (B, F, T) contiguous, T a multiple of the 256-token tile, K a multiple of 8.
bool lt_backward_mfma(int dtype, int is_btf, int B, int T, int K, int F) {
  return dtype == LTV_DTYPE_BF16 && !is_btf && gemm_tuning().dma && T % 256 == 0 && K % 8 == 0 &&
         K > 0 && F > 0 && (int64_t)B * T < (1ll << 31) && (int64_t)B * F * T < kDmaMaxSpan &&
         (int64_t)B * T * K < kDmaMaxSpan;
}

struct LtSplits {
  int rows, S, Fr;
};
// dW split-K: about one (tile, split) item per CU over the 256 x 256 tiles,
// at least 1024 reduction rows per split
LtSplits lt_splits(int M, int K, int F) {
  LtSplits p;
  p.Fr = round_up(F, 256);
  const int tiles = std::max(1, ((K + 255) / 256) * (p.Fr / 256));
  const int S = std::max(1, device_cu_count() / tiles);
  p.rows = std::max(1024, round_up((M + S - 1) / S, 64));
  p.S = std::max(1, (M + p.rows - 1) / p.rows);
  return p;
}

// grad_weight's split over the B T reduction on the fp32-MFMA GEMM.  With
// `slots` workgroups resident at once (two per CU) and `tiles` 128 x 128
// output tiles, S splits take ceil(tiles S / slots) rounds of M / S
// reduction indices each: S minimises rounds / S (the smallest S within 4%
// of the best, up to 32 splits of at least 256 indices).  At d12 (114 tiles,
// 512 slots) S = 13: 1,482 items in 3 rounds (S = 5 leaves 58 items for a
// second round, S = 4 a quarter of the slots idle).  S = 1 needs no workspace.
LtSplits lt_f32m_splits(int M, int K, int F) {
  LtSplits p;
  p.Fr = F;
  const int tiles = std::max(1, ((K + kF32B - 1) / kF32B) * ((F + kF32B - 1) / kF32B));
  const int slots = 2 * device_cu_count();
  auto cost = [&](int s) { return (double)((tiles * s + slots - 1) / slots) / s; };
  double best = cost(1);
  int smax = 1;
  for (int s = 2; s <= 32 && (M + s - 1) / s >= 256; ++s) {
    best = std::min(best, cost(s));
    smax = s;
  }
  int S = 1;
  while (S < smax && cost(S) > 1.04 * best) ++S;
  p.rows = std::max(kF32BK, round_up((M + S - 1) / S, kF32BK));
  p.S = std::max(1, (M + p.rows - 1) / p.rows);
  return p;
}

// Only tensors with no elements may be null (PyTorch hands those over as 0).
bool lt_backward_pointers_ok(const void* x, const void* weight, const void* grad_out,
                             const void* grad_x, const void* grad_weight, int B, int T, int K,
                             int F) {
  const int64_t nx = (int64_t)B * T * K, nw = (int64_t)F * K, ng = (int64_t)B * F * T;
  return (x || nx == 0) && (grad_x || nx == 0) && (weight || nw == 0) &&
         (grad_weight || nw == 0) && (grad_out || ng == 0);
}

size_t lt_f32m_workspace(int B, int T, int K, int F) {
  const LtSplits p = lt_f32m_splits(B * T, K, F);
  return p.S > 1 ? (size_t)p.S * F * K * sizeof(float) : 0;
}

// Both gradients on the fp32-MFMA GEMM.  grad_weight is split over the B T
// reduction into fp32 partials in `workspace` when it holds
// lt_f32m_workspace() bytes (then summed in a fixed order), else computed in
// one pass per output tile.
int lt_backward_f32m(int dtype, const void* x, const void* weight, const void* grad_out,
                     int grad_out_is_btf, void* grad_x, void* grad_weight, void* workspace,
                     size_t workspace_bytes, int B, int T, int K, int F, hipStream_t st) {
  // grad_out element (b, f, t): (B,F,T) -> b*F*T + f*T + t ; (B,T,F) -> b*T*F + t*F + f
  const int64_t go_f = grad_out_is_btf ? 1 : T;
  const int64_t go_t = grad_out_is_btf ? F : 1;
  // grad_x_b (T x K) = sum_f go_b(f, t) W(f, k)
  F32mArgs a{};
  a.A = grad_out; a.sam = go_t; a.sako = 0; a.saki = go_f; a.sab = (int64_t)F * T;
  a.B = weight; a.sbn = 1; a.sbko = 0; a.sbki = K; a.sbb = 0;
  a.C = grad_x; a.scm = K; a.scn = 1; a.scb = (int64_t)T * K;
  a.M = T; a.N = K; a.K = F; a.kin = F > 0 ? F : 1;
  int rc = launch_f32m(dtype, dtype, a, B, 1, 0, st);
  if (rc) return rc;
  // grad_W (F x K) = sum_{b,t} go(b, f, t) x(b, t, k); reduction index kk = b*T + t
  // (an empty reduction, B T = 0, stores zeros)
  F32mArgs w{};
  w.A = grad_out; w.sam = go_f; w.sako = (int64_t)F * T; w.saki = go_t; w.sab = 0;
  w.B = x; w.sbn = 1; w.sbko = (int64_t)T * K; w.sbki = K; w.sbb = 0;
  w.C = grad_weight; w.scm = K; w.scn = 1; w.scb = 0;
  w.M = F; w.N = K; w.K = B * T; w.kin = T > 0 ? T : 1;
  const LtSplits sp = lt_f32m_splits(w.K, K, F);
  const size_t need = lt_f32m_workspace(B, T, K, F);
  if (need == 0 || workspace == nullptr || workspace_bytes < need)
    return launch_f32m(dtype, dtype, w, 1, 1, 0, st);
  w.C = workspace;
  w.scs = (int64_t)F * K;
  rc = launch_f32m(dtype, LTV_DTYPE_F32, w, 1, sp.S, sp.rows, st);
  if (rc) return rc;
  const int64_t n = (int64_t)F * K;
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 8192);
  if (dtype == LTV_DTYPE_F32)
    hipLaunchKernelGGL(reduce_splits_kernel<float>, dim3(blocks), dim3(256), 0, st,
                       reinterpret_cast<const float*>(workspace),
                       reinterpret_cast<float*>(grad_weight), sp.S, n, n);
  else
    hipLaunchKernelGGL(reduce_splits_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st,
                       reinterpret_cast<const float*>(workspace),
                       reinterpret_cast<bf16_t*>(grad_weight), sp.S, n, n);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}
}  // namespace

extern "C" int ltv_linear_transpose_backward(int dtype, const void* x, const void* weight,
                                             const void* grad_out, int grad_out_is_btf,
                                             void* grad_x, void* grad_weight, int B, int T,
                                             int K, int F, void* stream) {
  LTV_REQUIRE(dtype == LTV_DTYPE_F32 || dtype == LTV_DTYPE_BF16, LTV_ERR_INVALID_ARG,
              "dtype must be LTV_DTYPE_F32 or LTV_DTYPE_BF16, got %d", dtype);
  LTV_REQUIRE(B >= 0 && T >= 0 && K >= 0 && F >= 0, LTV_ERR_INVALID_ARG, "negative size");
  LTV_REQUIRE(lt_backward_pointers_ok(x, weight, grad_out, grad_x, grad_weight, B, T, K, F),
              LTV_ERR_INVALID_ARG, "null tensor pointer");
  return lt_backward_f32m(dtype, x, weight, grad_out, grad_out_is_btf, grad_x, grad_weight,
                          nullptr, 0, B, T, K, F, (hipStream_t)stream);
}

extern "C" size_t ltv_linear_transpose_backward_workspace_size(int dtype, int B, int T, int K,
                                                                int F, int grad_out_is_btf) {
  if (B <= 0 || T <= 0 || K <= 0 || F <= 0) return 0;
  if (!lt_backward_mfma(dtype, grad_out_is_btf, B, T, K, F)) return lt_f32m_workspace(B, T, K, F);
  const LtSplits p = lt_splits(B * T, K, F);
  return (size_t)p.S * p.Fr * K * sizeof(float);
}

extern "C" int ltv_linear_transpose_backward_ws(int dtype, const void* x, const void* weight,
                                                const void* grad_out, int grad_out_is_btf,
                                                void* grad_x, void* grad_weight, void* workspace,
                                                size_t workspace_bytes, int B, int T, int K,
                                                int F, void* stream) {
  LTV_REQUIRE(dtype == LTV_DTYPE_F32 || dtype == LTV_DTYPE_BF16, LTV_ERR_INVALID_ARG,
              "dtype must be LTV_DTYPE_F32 or LTV_DTYPE_BF16, got %d", dtype);
  LTV_REQUIRE(B >= 0 && T >= 0 && K >= 0 && F >= 0, LTV_ERR_INVALID_ARG, "negative size");
  LTV_REQUIRE(lt_backward_pointers_ok(x, weight, grad_out, grad_x, grad_weight, B, T, K, F),
              LTV_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t st = (hipStream_t)stream;
  if (!lt_backward_mfma(dtype, grad_out_is_btf, B, T, K, F) ||
      !(aligned16(x) && aligned16(weight) && aligned16(grad_out) && aligned16(grad_x) &&
        aligned16(grad_weight)))
    return lt_backward_f32m(dtype, x, weight, grad_out, grad_out_is_btf, grad_x, grad_weight,
                            workspace, workspace_bytes, B, T, K, F, st);
  const int M = B * T;
  const LtSplits sp = lt_splits(M, K, F);
  const size_t need = (size_t)sp.S * sp.Fr * K * sizeof(float);
  LTV_REQUIRE(workspace && workspace_bytes >= need, LTV_ERR_WORKSPACE,
              "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  const bf16_t* gp = reinterpret_cast<const bf16_t*>(grad_out);
  // grad_x[m, k] = sum_f g[b, f, t] W[f, k]:  i = k (RC: W[f K + k]), j = m (RC, batched:
  // g at (m / T) F T + f T + m % T)
  {
    GemmArgs a;
    a.P = GemmOperand{reinterpret_cast<const bf16_t*>(weight), K, K, F};
    a.Q = GemmOperand{gp, T, M, F};
    a.Q.bstride = (int64_t)F * T;
    a.Q.blen = T;
    a.K = F;
    a.k_split = round_up(F, kGemmBK);
    EpiRowBF16 e{reinterpret_cast<bf16_t*>(grad_x), K, K, M};
    LTV_REQUIRE(dma_usable(a, OP_RC, OP_RC, e, 1), LTV_ERR_UNSUPPORTED,
                "grad_x operands not supported by the MFMA kernel");
    a.tiles_i = (K + 255) / 256;
    a.tiles_j = M / 256;
    int rc = launch_gemm_dma<256, 256, 2, 4, OP_RC, OP_RC>(a, e, 1, st);
    if (rc) return rc;
  }
  // grad_weight[f, k] = sum_m x[m, k] g[b, f, t]:  i = k (RC: x[m K + k]), j = f (KC with the
  // reduction index m batched: g at (m / T) F T + f T + m % T); fp32 split partials, then a
  // fixed-order sum into grad_weight (bf16)
  {
    GemmArgs a;
    a.P = GemmOperand{reinterpret_cast<const bf16_t*>(x), K, K, M};
    a.Q = GemmOperand{gp, T, F, M};
    a.Q.bstride = (int64_t)F * T;
    a.Q.blen = T;
    a.K = M;
    a.k_split = sp.rows;
    EpiRowF32Split e{reinterpret_cast<float*>(workspace), K, (int64_t)sp.Fr * K, K, sp.Fr};
    LTV_REQUIRE(dma_usable(a, OP_RC, OP_KC, e, sp.S), LTV_ERR_UNSUPPORTED,
                "grad_weight operands not supported by the MFMA kernel");
    a.tiles_i = (K + 255) / 256;
    a.tiles_j = sp.Fr / 256;
    int rc = launch_gemm_dma<256, 256, 2, 4, OP_RC, OP_KC>(a, e, sp.S, st);
    if (rc) return rc;
    const int64_t n = (int64_t)F * K;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(reduce_splits_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st,
                       reinterpret_cast<const float*>(workspace),
                       reinterpret_cast<bf16_t*>(grad_weight), sp.S, (int64_t)sp.Fr * K, n);
    LTV_LAUNCH_CHECK();
  }
  return LTV_OK;
}

extern "C" int ltv_qkv_packed_width(int H, int D, int Da) {
  return round_up(H * D + H * Da, 128);
}

extern "C" int ltv_qkv_logit_width(int H, int Da) { return round_up(H * Da, 8); }

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
  if (C % 8 == 0 && (int64_t)Fp * C < (1ll << 31) && ((uintptr_t)weight & 15) == 0 &&
      ((uintptr_t)wpack & 15) == 0) {
    const int b8 = (int)std::min<int64_t>(((int64_t)Fp * C / 8 + 255) / 256, 8192);
    if (weight_dtype == LTV_DTYPE_F32)
      hipLaunchKernelGGL(pack_weight8_kernel<float>, dim3(b8), dim3(256), 0, st,
                         reinterpret_cast<const float*>(weight), reinterpret_cast<bf16_t*>(wpack),
                         H, D, Da, C, Fp);
    else
      hipLaunchKernelGGL(pack_weight8_kernel<bf16_t>, dim3(b8), dim3(256), 0, st,
                         reinterpret_cast<const bf16_t*>(weight), reinterpret_cast<bf16_t*>(wpack),
                         H, D, Da, C, Fp);
    LTV_LAUNCH_CHECK();
    return LTV_OK;
  }
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

extern "C" int ltv_qkv_project_forward(const void* x, const void* wpack, void* values,
                                       void* logits, int B, int T, int C, int H, int D, int Da,
                                       void* stream) {
  LTV_REQUIRE(B >= 0 && T >= 0 && C > 0 && H > 0 && D > 0 && Da > 0, LTV_ERR_INVALID_ARG,
              "bad shape");
  LTV_REQUIRE(C % 8 == 0 && D % 4 == 0, LTV_ERR_UNSUPPORTED,
              "C must be a multiple of 8 and D of 4 (C=%d D=%d)", C, D);
  const int64_t M64 = (int64_t)B * T;
  LTV_REQUIRE(M64 < (1ll << 31), LTV_ERR_UNSUPPORTED, "too many tokens");
  const int M = (int)M64;
  if (M == 0) return LTV_OK;
  LTV_REQUIRE(x && wpack && values && logits, LTV_ERR_INVALID_ARG, "null tensor pointer");
  LTV_REQUIRE(aligned16(x) && aligned16(wpack) && aligned16(values) && aligned16(logits),
              LTV_ERR_INVALID_ARG, "x, wpack, values and logits must be 16-byte aligned");
  const int Fp = ltv_qkv_packed_width(H, D, Da);
  GemmArgs a;
  a.P = GemmOperand{reinterpret_cast<const bf16_t*>(wpack), C, Fp, C};  // (n, k) KC
  a.Q = GemmOperand{reinterpret_cast<const bf16_t*>(x), C, M, C};       // (m, k) KC
  a.K = C;
  a.k_split = round_up(C, kGemmBK);
  // the logit rows' padding columns [H Da, Lp) come out as zeros (the packed
  // weight's rows past F are zero), so every element of the output is defined
  EpiProjectHM e{reinterpret_cast<bf16_t*>(values), reinterpret_cast<bf16_t*>(logits), H, D, T,
                 ltv_qkv_logit_width(H, Da), H * D + ltv_qkv_logit_width(H, Da), M};
  hipStream_t st = (hipStream_t)stream;
  if (gemm_tuning().dma && dma_usable(a, OP_KC, OP_KC, e, 1)) {
    a.tiles_j = (M + 255) / 256;
    if (gemm_tuning().fwd == 3) {
      a.tiles_i = (Fp + 127) / 128;
      return launch_gemm_dma<128, 256, 2, 4, OP_KC, OP_KC>(a, e, 1, st);
    }
    a.tiles_i = (Fp + 255) / 256;
    return launch_gemm_dma<256, 256, 2, 4, OP_KC, OP_KC>(a, e, 1, st);
  }
  if (gemm_tuning().fwd == 1) {
    a.tiles_i = (Fp + 255) / 256;
    a.tiles_j = (M + 255) / 256;
    return launch_gemm<256, 256, 2, 4, OP_KC, OP_KC>(a, e, 1, st);
  }
  if (gemm_tuning().fwd == 2) {
    a.tiles_i = (Fp + 255) / 256;
    a.tiles_j = (M + 255) / 256;
    return launch_gemm<256, 256, 2, 2, OP_KC, OP_KC>(a, e, 1, st);
  }
  a.tiles_i = Fp / 128;
  a.tiles_j = (M + 255) / 256;
  return launch_gemm<128, 256, 2, 2, OP_KC, OP_KC>(a, e, 1, st);
}

namespace {
inline int dw_splits(int M, int rows) { return std::max(1, (M + rows - 1) / rows); }
inline int dw_rows(int Fp, int variant) { return variant == 1 ? round_up(Fp, 128) : round_up(Fp, 256); }
// Rows of the M reduction per dW split (a multiple of the 64-row k-step).
// Automatic: as many splits as give about one (tile, split) item per CU over
// the 256 x 256 output tiles -- at d12 (M = 32768) 8 splits of 4096 rows, 240
// items; at B = 16 (M = 16384) 8 of 2048 (fixed 4096-row splits left 120 items
// and half the CUs idle).
inline int dw_split_rows(int M, int C, int Fp) {
  const GemmTuning& tu = gemm_tuning();
  if (tu.dw_split > 0) return tu.dw_split;
  const int tiles = std::max(1, ((C + 255) / 256) * (dw_rows(Fp, tu.dw) / 256));
  const int S = std::max(1, device_cu_count() / tiles);
  // at least 1024 rows (16 k-steps) per split: shorter splits cost more in
  // per-item overhead and partial sums than they gain in parallelism
  return std::max(1024, round_up((M + S - 1) / S, 64));
}
// Sum of the S fp32 partials of grad_weight (S slots of Fr x C) into the
// parameter's interleaved row order.
int dw_reduce_launch(void* workspace, float* grad_weight, int S, int Fr, int H, int D, int Da,
                     int C, hipStream_t st) {
  const int Fvalid = H * (D + Da);
  const int64_t total = (int64_t)Fvalid * C;
  if (C % 4 == 0 && total < (1ll << 31) && ((uintptr_t)workspace & 15) == 0 &&
      ((uintptr_t)grad_weight & 15) == 0) {
    const int blocks = (int)std::min<int64_t>((total / 4 + 255) / 256, 8192);
    hipLaunchKernelGGL(dw_reduce4_kernel, dim3(blocks), dim3(256), 0, st,
                       reinterpret_cast<const float4*>(workspace),
                       reinterpret_cast<float4*>(grad_weight), S, (int64_t)Fr * C / 4, H, D, Da,
                       C / 4);
  } else {
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(dw_reduce_kernel, dim3(blocks), dim3(256), 0, st,
                       reinterpret_cast<const float*>(workspace), grad_weight, S,
                       (int64_t)Fr * C, H, D, Da, C);
  }
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}
}  // namespace

extern "C" size_t ltv_qkv_project_backward_workspace_size(int M, int C, int H, int D, int Da) {
  const int Fp = ltv_qkv_packed_width(H, D, Da);
  const GemmTuning& tu = gemm_tuning();
  return (size_t)dw_splits(M, dw_split_rows(M, C, Fp)) * dw_rows(Fp, tu.dw) * C * sizeof(float);
}

namespace {
int project_backward_check(const void* x, const void* wpack, const void* grad_combined, int M,
                           int C, int H, int D, int Da) {
  LTV_REQUIRE(M >= 0 && C > 0 && H > 0 && D > 0 && Da > 0, LTV_ERR_INVALID_ARG, "bad shape");
  LTV_REQUIRE(C % 8 == 0, LTV_ERR_UNSUPPORTED, "C must be a multiple of 8 (C=%d)", C);
  LTV_REQUIRE(x && wpack && grad_combined, LTV_ERR_INVALID_ARG, "null tensor pointer");
  LTV_REQUIRE(aligned16(x) && aligned16(wpack) && aligned16(grad_combined), LTV_ERR_INVALID_ARG,
              "x, wpack and grad_combined must be 16-byte aligned");
  return LTV_OK;
}
}  // namespace

namespace {
// grad_x; pad_zeroed: the caller guarantees grad_combined's columns F ..
// round_up(F, 8) - 1 are zero already (no zeroing launch)
int project_backward_input_impl(const void* x, const void* wpack, void* grad_combined,
                                void* grad_x, int M, int C, int H, int D, int Da, bool pad_zeroed,
                                void* stream) {
  int rc = project_backward_check(x, wpack, grad_combined, M, C, H, D, Da);
  if (rc) return rc;
  LTV_REQUIRE(grad_x && aligned16(grad_x), LTV_ERR_INVALID_ARG, "grad_x null or misaligned");
  if (M == 0) return LTV_OK;
  const int Fp = ltv_qkv_packed_width(H, D, Da);
  const int Fvalid = H * (D + Da);
  // dX[m, c] = sum_f dC[m, f] Wp[f, c]:  i = c (RC: Wp[f * C + c]), j = m (KC: dC[m * Fp + f]);
  // the padding columns of dC (f >= Fvalid) are never read
  GemmArgs a;
  a.P = GemmOperand{reinterpret_cast<const bf16_t*>(wpack), C, C, Fvalid};
  a.Q = GemmOperand{reinterpret_cast<const bf16_t*>(grad_combined), Fp, M, Fvalid};
  a.K = Fp;
  a.k_split = Fp;
  EpiRowBF16 e{reinterpret_cast<bf16_t*>(grad_x), C, C, M};
  a.tiles_j = (M + 255) / 256;
  hipStream_t st = (hipStream_t)stream;
  if (gemm_tuning().dma) {
    // the direct-to-LDS loads fetch dC in 8-column chunks: columns up to the
    // next multiple of 8 past Fvalid are read, so they are set to zero first;
    // the reduction stops there (Fp would add k-steps that only load padding:
    // 38 instead of 37 at d12)
    const int Fv8 = round_up(Fvalid, 8);
    GemmArgs ad = a;
    ad.Q.k_valid = Fv8;
    ad.K = Fv8;
    ad.k_split = Fv8;
    if (dma_usable(ad, OP_RC, OP_KC, e, 1)) {
      if (Fv8 > Fvalid && !pad_zeroed) {
        const int blocks = (M + 255) / 256;
        hipLaunchKernelGGL(zero_cols_kernel, dim3(blocks), dim3(256), 0, st,
                           reinterpret_cast<bf16_t*>(grad_combined), M,
                           (int64_t)Fp, Fvalid, Fv8);
        LTV_LAUNCH_CHECK();
      }
      if (gemm_tuning().dx == 3) {  // 128-row tiles: 2x the work items of the 256-row tiles
        ad.tiles_i = (C + 127) / 128;
        return launch_gemm_dma<128, 256, 2, 4, OP_RC, OP_KC>(ad, e, 1, st);
      }
      ad.tiles_i = (C + 255) / 256;
      return launch_gemm_dma<256, 256, 2, 4, OP_RC, OP_KC>(ad, e, 1, st);
    }
  }
  if (gemm_tuning().dx == 1 && C % 256 == 0) {
    a.tiles_i = C / 256;
    return launch_gemm<256, 256, 2, 4, OP_RC, OP_KC>(a, e, 1, st);
  }
  if (gemm_tuning().dx == 2 && C % 256 == 0) {
    a.tiles_i = C / 256;
    return launch_gemm<256, 256, 2, 2, OP_RC, OP_KC>(a, e, 1, st);
  }
  a.tiles_i = (C + 127) / 128;
  return launch_gemm<128, 256, 2, 2, OP_RC, OP_KC>(a, e, 1, st);
}

}  // namespace

extern "C" int ltv_qkv_project_backward_input(const void* x, const void* wpack,
                                              void* grad_combined, void* grad_x, int M,
                                              int C, int H, int D, int Da, void* stream) {
  return project_backward_input_impl(x, wpack, grad_combined, grad_x, M, C, H, D, Da, false,
                                     stream);
}

extern "C" int ltv_qkv_project_backward_input_zero_padded(const void* x, const void* wpack,
                                                          const void* grad_combined,
                                                          void* grad_x, int M, int C, int H,
                                                          int D, int Da, void* stream) {
  return project_backward_input_impl(x, wpack, const_cast<void*>(grad_combined), grad_x, M, C, H,
                                     D, Da, true, stream);
}

extern "C" int ltv_qkv_project_backward_weight(const void* x, const void* grad_combined,
                                               float* grad_weight, void* workspace,
                                               size_t workspace_bytes, int M, int C, int H,
                                               int D, int Da, void* stream) {
  int rc = project_backward_check(x, x, grad_combined, M, C, H, D, Da);
  if (rc) return rc;
  LTV_REQUIRE(grad_weight, LTV_ERR_INVALID_ARG, "null grad_weight");
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
  const GemmTuning& tu = gemm_tuning();
  // dW^T[c, f] = sum_m X[m, c] dC[m, f]:  i = c (RC: X[m * C + c]), j = f (RC: dC[m * Fp + f]),
  // the reduction over m split into fp32 partials P_s[f][c]
  const int split_rows = dw_split_rows(M, C, Fp);
  const int S = dw_splits(M, split_rows);
  const int Fr = dw_rows(Fp, tu.dw);
  GemmArgs a;
  a.P = GemmOperand{reinterpret_cast<const bf16_t*>(x), C, C, M};
  a.Q = GemmOperand{reinterpret_cast<const bf16_t*>(grad_combined), Fp, Fp, M};
  a.K = M;
  a.k_split = split_rows;
  EpiRowF32Split e{reinterpret_cast<float*>(workspace), C, (int64_t)Fr * C, C, Fr};
  if (tu.dma && dma_usable(a, OP_RC, OP_RC, e, S)) {
    a.tiles_i = (C + 255) / 256;
    a.tiles_j = (Fr + 255) / 256;
    rc = launch_gemm_dma<256, 256, 2, 4, OP_RC, OP_RC>(a, e, S, st);
  } else if (tu.dw == 1) {
    a.tiles_i = (C + 255) / 256;
    a.tiles_j = Fr / 128;
    rc = launch_gemm<256, 128, 2, 2, OP_RC, OP_RC>(a, e, S, st);
  } else if (tu.dw == 2) {
    a.tiles_i = (C + 255) / 256;
    a.tiles_j = Fr / 256;
    rc = launch_gemm<256, 256, 2, 2, OP_RC, OP_RC>(a, e, S, st);
  } else {
    a.tiles_i = (C + 127) / 128;
    a.tiles_j = Fr / 256;
    rc = launch_gemm<128, 256, 2, 2, OP_RC, OP_RC>(a, e, S, st);
  }
  if (rc) return rc;
  return dw_reduce_launch(workspace, grad_weight, S, Fr, H, D, Da, C, st);
}

namespace {
// grad_x and grad_weight in one launch of gemm_dma_bwd_fused_kernel, where
// grad_x's 256 x 256 tiles do not fill their last round of the persistent grid:
// the workgroups that run one grad_x tile fewer take the longer pieces of
// grad_weight's reduction.  Returns LTV_OK when launched (with the
// zeroing and reduction launches around it), 1 when the shapes or tunables
// leave it out (nothing launched), or an error code.
int project_backward_fused(const void* x, const void* wpack, void* grad_combined, void* grad_x,
                           float* grad_weight, void* workspace, int M, int C, int H, int D,
                           int Da, bool pad_zeroed, hipStream_t st) {
  static const bool enabled = [] {
    const char* e = getenv("LTV_GEMM_BWD_FUSED");
    return e == nullptr || atoi(e) != 0;
  }();
  const GemmTuning& tu = gemm_tuning();
  if (!enabled || !tu.dma || tu.dx == 3 || M == 0) return 1;
  const int Fp = ltv_qkv_packed_width(H, D, Da);
  const int Fvalid = H * (D + Da);
  const int Fv8 = round_up(Fvalid, 8);
  // grad_x: as project_backward_input_impl's direct-to-LDS path
  GemmArgs ax;
  ax.P = GemmOperand{reinterpret_cast<const bf16_t*>(wpack), C, C, Fvalid};
  ax.Q = GemmOperand{reinterpret_cast<const bf16_t*>(grad_combined), Fp, M, Fv8};
  ax.K = Fv8;
  ax.k_split = Fv8;
  ax.splits = 1;
  ax.tiles_i = (C + 255) / 256;
  ax.tiles_j = (M + 255) / 256;
  EpiRowBF16 ex{reinterpret_cast<bf16_t*>(grad_x), C, C, M};
  // grad_weight: as ltv_qkv_project_backward_weight's direct-to-LDS path
  const int split_rows = dw_split_rows(M, C, Fp);
  const int S = dw_splits(M, split_rows);
  const int Fr = dw_rows(Fp, tu.dw);
  GemmArgs aw;
  aw.P = GemmOperand{reinterpret_cast<const bf16_t*>(x), C, C, M};
  aw.Q = GemmOperand{reinterpret_cast<const bf16_t*>(grad_combined), Fp, Fp, M};
  aw.K = M;
  aw.k_split = split_rows;
  aw.splits = S;
  aw.tiles_i = (C + 255) / 256;
  aw.tiles_j = (Fr + 255) / 256;
  EpiRowF32Split ew{reinterpret_cast<float*>(workspace), C, (int64_t)Fr * C, C, Fr};
  if (!dma_usable(ax, OP_RC, OP_KC, ex, 1) || !dma_usable(aw, OP_RC, OP_RC, ew, S)) return 1;
  // the plan
  const int G = device_cu_count();
  const int total_x = ax.tiles_i * ax.tiles_j;
  // workgroups [0, total_x % G) run one grad_x tile more than the others
  if (total_x % G == 0) return 1;
  DwPlan p;
  p.n_late = total_x % G;
  const int n_early = G - p.n_late;
  p.nt = aw.tiles_i * aw.tiles_j;
  p.S = S;
  p.e2 = n_early / p.nt;
  p.e1 = p.e2 + 1;
  p.x = n_early - p.nt * p.e2;
  if (p.e2 < 1 || p.S - p.e1 < 1) return 1;
  if (p.x * (p.S - p.e1) + (p.nt - p.x) * (p.S - p.e2) > p.n_late) return 1;
  p.ksteps = (M + kDmaBK - 1) / kDmaBK;
  // an early workgroup starts its piece one grad_x tile (kx k-steps) before a
  // late one; a grad_weight k-step (two row-contiguous operands) takes about
  // 8/7 of a grad_x one (measured at d12: 1.89 against 1.65 us)
  const int kx = (Fv8 + kDmaBK - 1) / kDmaBK;
  static const int delta_pct = [] {
    const char* e = getenv("LTV_GEMM_BWD_DELTA_PCT");
    return e != nullptr && atoi(e) > 0 ? atoi(e) : 87;
  }();
  int delta = (kx * delta_pct + 50) / 100;
  auto lengths = [&](int e, int& a, int& b) {
    for (int d = delta; d >= 0; --d) {
      a = (p.ksteps + (p.S - e) * d) / p.S;
      b = a - d;
      if (b >= 1 && e * a + (p.S - e - 1) * b < p.ksteps) return true;
    }
    return false;
  };
  if (!lengths(p.e1, p.a1, p.b1) || !lengths(p.e2, p.a2, p.b2)) return 1;
  if (Fv8 > Fvalid && !pad_zeroed) {
    hipLaunchKernelGGL(zero_cols_kernel, dim3((M + 255) / 256), dim3(256), 0, st,
                       reinterpret_cast<bf16_t*>(grad_combined), M, (int64_t)Fp, Fvalid, Fv8);
    LTV_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL((gemm_dma_bwd_fused_kernel<EpiRowBF16, EpiRowF32Split>), dim3(G), dim3(512),
                     0, st, ax, ex, aw, ew, p);
  LTV_LAUNCH_CHECK();
  return dw_reduce_launch(workspace, grad_weight, S, Fr, H, D, Da, C, st);
}

int project_backward_impl(const void* x, const void* wpack, void* grad_combined, void* grad_x,
                          float* grad_weight, void* workspace, size_t workspace_bytes, int M,
                          int C, int H, int D, int Da, bool pad_zeroed, void* stream) {
  int rc = project_backward_check(x, wpack, grad_combined, M, C, H, D, Da);
  if (rc) return rc;
  LTV_REQUIRE(grad_x && aligned16(grad_x), LTV_ERR_INVALID_ARG, "grad_x null or misaligned");
  LTV_REQUIRE(grad_weight, LTV_ERR_INVALID_ARG, "null grad_weight");
  if (M > 0) {
    const size_t need = ltv_qkv_project_backward_workspace_size(M, C, H, D, Da);
    LTV_REQUIRE(workspace && workspace_bytes >= need, LTV_ERR_WORKSPACE,
                "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    rc = project_backward_fused(x, wpack, grad_combined, grad_x, grad_weight, workspace, M, C, H,
                                D, Da, pad_zeroed, (hipStream_t)stream);
    if (rc != 1) return rc;
  }
  rc = project_backward_input_impl(x, wpack, grad_combined, grad_x, M, C, H, D, Da, pad_zeroed,
                                   stream);
  if (rc) return rc;
  return ltv_qkv_project_backward_weight(x, grad_combined, grad_weight, workspace,
                                         workspace_bytes, M, C, H, D, Da, stream);
}
}  // namespace

extern "C" int ltv_qkv_project_backward(const void* x, const void* wpack,
                                        void* grad_combined, void* grad_x,
                                        float* grad_weight, void* workspace,
                                        size_t workspace_bytes, int M, int C, int H, int D,
                                        int Da, void* stream) {
  return project_backward_impl(x, wpack, grad_combined, grad_x, grad_weight, workspace,
                               workspace_bytes, M, C, H, D, Da, false, stream);
}

extern "C" int ltv_qkv_project_backward_zero_padded(const void* x, const void* wpack,
                                                    const void* grad_combined, void* grad_x,
                                                    float* grad_weight, void* workspace,
                                                    size_t workspace_bytes, int M, int C, int H,
                                                    int D, int Da, void* stream) {
  return project_backward_impl(x, wpack, const_cast<void*>(grad_combined), grad_x, grad_weight,
                               workspace, workspace_bytes, M, C, H, D, Da, true, stream);
}
