// Microbenchmarks for the roofline peaks that bench.py --workload peaks
// reports beside MI355X's published figures (built into libltv_peaks.so, a
// library of its own: none of this is part of the filter's C ABI).
//
//   ltv_peak_mfma:   a loop of v_mfma_f32_32x32x16_bf16 on every SIMD, eight
//                    independent accumulators per wavefront, two wavefronts
//                    per SIMD -- the instruction and occupancy of the
//                    projection GEMMs.  Operand bits either change from one
//                    MFMA to the next (the power draw of real data, which
//                    lowers the clock) or are all zero.
//   ltv_peak_stream: HBM streams of 16-byte vectors, NR source arrays read and
//                    (optionally) one destination written, either grid-stride
//                    over the arrays or one contiguous slice per workgroup
//                    (the scan's access shape: one workgroup per (b, head,
//                    channel slab) walking its own stretch of each array).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/ltv_peaks.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// bf16 with a random sign and mantissa, exponent of 1.0: finite, no overflow
// of the fp32 accumulators over the loop
__device__ __forceinline__ bf16x8_t random_operand(uint32_t seed) {
  u16x8_t bits;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t h = mix(seed * 8u + (uint32_t)e);
    bits[e] = (unsigned short)(0x3f80u | (h & 0x807fu));
  }
  return __builtin_bit_cast(bf16x8_t, bits);
}

constexpr int kChains = 8;  // independent accumulators per wavefront
constexpr int kOps = 4;     // operand pairs cycled through

// two wavefronts per SIMD (<= 256 registers each), as the GEMMs run
__global__ void __launch_bounds__(256, 2) peak_mfma_kernel(float* __restrict__ out, int iters,
                                                           int zero) {
  const uint32_t tid = blockIdx.x * 256u + threadIdx.x;
  bf16x8_t a[kOps], b[kOps];
#pragma unroll
  for (int o = 0; o < kOps; ++o) {
    a[o] = random_operand(tid * 2u * kOps + 2u * o);
    b[o] = random_operand(tid * 2u * kOps + 2u * o + 1u);
    if (zero) {
      a[o] = bf16x8_t{};
      b[o] = bf16x8_t{};
    }
  }
  f32x16_t acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) acc[c] = f32x16_t{};
  // iters rounds of kChains MFMAs, in groups of kOps rounds so that every
  // operand choice is static
  for (int i = 0; i < iters; i += kOps) {
#pragma unroll
    for (int s = 0; s < kOps; ++s)
#pragma unroll
      for (int c = 0; c < kChains; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c % kOps], b[(c / 2 + s) % kOps],
                                                          acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[c][v];
  out[tid] = s;
}

struct StreamArgs {
  const u32x4_t* src[3];
  u32x4_t* dst;
  int64_t n;      // 16-byte vectors per array
  int64_t slice;  // vectors per workgroup slice (0: grid-stride)
  uint32_t never;  // a value no read-only accumulation takes in practice
};

constexpr int kUnroll = 4;  // vectors per array in flight per thread

template <int NR, bool WR, bool NT>
__global__ void __launch_bounds__(256) peak_stream_kernel(const StreamArgs a) {
  int64_t begin, end, step;
  if (a.slice > 0) {
    begin = (int64_t)blockIdx.x * a.slice;
    end = begin + a.slice < a.n ? begin + a.slice : a.n;
    step = 256;
  } else {
    begin = 0;
    end = a.n;
    step = (int64_t)gridDim.x * 256;
  }
  const int64_t first = begin + (a.slice > 0 ? 0 : (int64_t)blockIdx.x * 256) + threadIdx.x;
  u32x4_t acc = {0u, 0u, 0u, 0u};
  for (int64_t i = first; i < end; i += step * kUnroll) {
    u32x4_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t j = i + u * step;
        if (j < end) v[u] ^= NT ? __builtin_nontemporal_load(&a.src[r][j]) : a.src[r][j];
      }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = i + u * step;
      if (j < end) {
        if (WR) {
          const u32x4_t o = NR > 0 ? v[u] : u32x4_t{(uint32_t)j, (uint32_t)j, 0u, 0u};
          if (NT)
            __builtin_nontemporal_store(o, &a.dst[j]);
          else
            a.dst[j] = o;
        } else {
          acc ^= v[u];
        }
      }
    }
  }
  // read-only streams keep their loads alive through a store that the data
  // practically never triggers
  if (!WR && (acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == a.never) a.dst[0] = acc;
}

template <int NR, bool WR>
hipError_t launch_stream(const StreamArgs& a, int blocks, bool nt, hipStream_t st) {
  if (nt)
    hipLaunchKernelGGL((peak_stream_kernel<NR, WR, true>), dim3(blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((peak_stream_kernel<NR, WR, false>), dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace

extern "C" int ltv_peak_mfma(float* out, int blocks, int iters, int zero_operands,
                             void* stream) {
  if (out == nullptr || blocks <= 0 || iters <= 0) return 1;
  hipLaunchKernelGGL(peak_mfma_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters,
                     zero_operands);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int ltv_peak_stream(const void* const* srcs, int nr, void* dst, int write,
                               int nontemporal, int64_t n16, int64_t slice16, int blocks,
                               uint32_t never, void* stream) {
  if (nr < 0 || nr > 3 || n16 <= 0 || blocks <= 0 || slice16 < 0) return 1;
  if (dst == nullptr || (nr == 0 && !write)) return 1;
  if (slice16 > 0 && (int64_t)blocks * slice16 < n16) return 1;  // every vector has a workgroup
  StreamArgs a{};
  for (int r = 0; r < nr; ++r) {
    if (srcs == nullptr || srcs[r] == nullptr) return 1;
    a.src[r] = static_cast<const u32x4_t*>(srcs[r]);
  }
  a.dst = static_cast<u32x4_t*>(dst);
  a.n = n16;
  a.slice = slice16;
  a.never = never;
  hipStream_t st = (hipStream_t)stream;
  const bool nt = nontemporal != 0;
  hipError_t e = hipErrorInvalidValue;
  if (write) {
    switch (nr) {
      case 0: e = launch_stream<0, true>(a, blocks, nt, st); break;
      case 1: e = launch_stream<1, true>(a, blocks, nt, st); break;
      case 2: e = launch_stream<2, true>(a, blocks, nt, st); break;
      case 3: e = launch_stream<3, true>(a, blocks, nt, st); break;
    }
  } else {
    switch (nr) {
      case 1: e = launch_stream<1, false>(a, blocks, nt, st); break;
      case 2: e = launch_stream<2, false>(a, blocks, nt, st); break;
      case 3: e = launch_stream<3, false>(a, blocks, nt, st); break;
    }
  }
  return e == hipSuccess ? 0 : 3;
}
