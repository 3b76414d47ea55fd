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
//   ltv_peak_overlap: the projection GEMM's k-step without its epilogue, on
//                    every CU: 64 KB of direct-to-LDS loads per step in the
//                    GEMM's row pattern (1,536-byte rows, eight 128-byte
//                    lines per 1 KB instruction) issued one step ahead by 4
//                    of 8 wavefronts, 256 v_mfma_f32_32x32x16_bf16 on
//                    random bits per step, 0 or 3 fragment reads from LDS
//                    per 4 MFMAs, one barrier per step -- each part alone
//                    or together, to see what they cost beside each other.
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

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));

// MODE bit 0: the loads; bit 1: the MFMAs; bits 3-4: fragment reads per 4
// MFMAs (0 or 3); bit 5: the reads go to a sink instead of the operands (no
// MFMA waits on them); bit 6: the reads run two groups ahead instead of one
template <int MODE>
__global__ void __launch_bounds__(512) peak_overlap_kernel(const char* __restrict__ src,
                                                           uint32_t mask, float* __restrict__ out,
                                                           int steps) {
  constexpr bool kLoads = MODE & 1, kMfma = MODE & 2;
  constexpr int kReads = (MODE >> 3) & 3;
  constexpr bool kSink = MODE & 32;
  constexpr int kAhead = MODE & 64 ? 2 : 1;  // groups of 4 MFMAs a read runs ahead
  s16x8_t sink = {};
  __shared__ __attribute__((aligned(16))) char stage[2][32 * 1024];  // the loads' targets
  __shared__ __attribute__((aligned(16))) char frag[16 * 1024];      // read-only fragments
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool loader = w >= 4;
  const uint64_t sa = reinterpret_cast<uint64_t>(src);
  i32x4_t rs;
  rs[0] = (int)(uint32_t)sa;
  rs[1] = (int)(uint32_t)((sa >> 32) & 0xffffu);
  rs[2] = (int)(mask + 1u);
  rs[3] = 0x00020000;
  const uint32_t tid = blockIdx.x * 512u + threadIdx.x;
  bf16x8_t A = random_operand(tid * 2u), B = random_operand(tid * 2u + 1u);
  // the fragment area holds random sign and mantissa bits: XORed into the
  // operands they keep them finite, in [1, 2) in magnitude, and changing
  for (int o = threadIdx.x * 16; o < 16 * 1024; o += 512 * 16)
    *reinterpret_cast<u16x8_t*>(&frag[o]) =
        __builtin_bit_cast(u16x8_t, random_operand(tid * 977u + (uint32_t)o)) & (unsigned short)0x807fu;
  __syncthreads();
  f32x16_t acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;
  uint32_t li = 0;
  // one step's 16 loads of this loader: lane l fetches 16 bytes of row l / 8
  // of an 8-row group (the row's 128-byte line), rows walking down a
  // 1,536-byte-pitch operand; M0 (the LDS target) is an input operand
  auto issue16 = [&](int s) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t lb = (uint32_t)(uintptr_t)&stage[s & 1][((w - 4) * 16 + j) % 32 * 1024];
      const uint32_t row = (blockIdx.x * 8u + (uint32_t)w) * 4096u + li * 8u + (uint32_t)(lane >> 3);
      const uint32_t vo = (row * 1536u + (uint32_t)(lane & 7) * 16u) & mask;
      ++li;
      asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                   :
                   : "v"(vo), "s"(rs), "{m0}"(lb)
                   : "memory");
    }
  };
  if (kLoads && loader) issue16(0);
  for (int s = 0; s < steps; ++s) {
    if (kLoads && loader) issue16(s + 1);
    if (kMfma) {
      // fragments read one group of 4 MFMAs ahead of their use (as the GEMM
      // reads the next k16 sub-step's during the current one's MFMAs), so the
      // reads' latency is covered and only their issue and LDS time count
      s16x8_t f[kAhead + 1][3];
      auto read3 = [&](int m, int buf) {
#pragma unroll
        for (int r = 0; r < kReads; ++r) {
          const int o = ((lane * 16) + (m * 3 + r) * 1024 + w * 64) & (16 * 1024 - 16);
          f[buf][r] = *reinterpret_cast<const s16x8_t*>(&frag[o]);
        }
      };
#pragma unroll
      for (int m = 0; m < kAhead; ++m) read3(m, m);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        if (m + kAhead < 8) read3(m + kAhead, (m + kAhead) % (kAhead + 1));
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, acc[i], 0, 0, 0);
        const int cb = m % (kAhead + 1);
        if (kSink) {
#pragma unroll
          for (int r = 0; r < kReads; ++r) sink ^= f[cb][r];
          continue;
        }
        if (kReads > 0) A = __builtin_bit_cast(bf16x8_t, (s16x8_t)(__builtin_bit_cast(s16x8_t, A) ^ f[cb][0]));
        if (kReads > 1) B = __builtin_bit_cast(bf16x8_t, (s16x8_t)(__builtin_bit_cast(s16x8_t, B) ^ f[cb][1]));
        if (kReads > 2) A = __builtin_bit_cast(bf16x8_t, (s16x8_t)(__builtin_bit_cast(s16x8_t, A) ^ f[cb][2]));
      }
    }
    // this step's loads (issued one step earlier) have landed
    if (kLoads && loader) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    __syncthreads();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) sum += acc[i][v];
  out[tid] = sum + (float)stage[0][lane] + (float)(sink[0] ^ sink[7]);
}

}  // namespace

extern "C" int ltv_peak_overlap(const void* src, uint32_t src_bytes, float* out, int blocks,
                                int steps, int mode, void* stream) {
  if (src == nullptr || out == nullptr || blocks <= 0 || steps <= 0) return 1;
  if (src_bytes < (1u << 20) || (src_bytes & (src_bytes - 1)) != 0) return 1;
  hipStream_t st = (hipStream_t)stream;
  const uint32_t mask = src_bytes - 1;
  const char* p = static_cast<const char*>(src);
  switch (mode) {
    case 5: hipLaunchKernelGGL(peak_overlap_kernel<5>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    case 6: hipLaunchKernelGGL(peak_overlap_kernel<6>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    case 7: hipLaunchKernelGGL(peak_overlap_kernel<7>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    case 30: hipLaunchKernelGGL(peak_overlap_kernel<30>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    case 31: hipLaunchKernelGGL(peak_overlap_kernel<31>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    case 94: hipLaunchKernelGGL(peak_overlap_kernel<94>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    case 95: hipLaunchKernelGGL(peak_overlap_kernel<95>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    case 58: hipLaunchKernelGGL(peak_overlap_kernel<58>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    case 59: hipLaunchKernelGGL(peak_overlap_kernel<59>, dim3(blocks), dim3(512), 0, st, p, mask, out, steps); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

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
