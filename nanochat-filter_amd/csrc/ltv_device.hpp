// Device-side helpers shared by the LTV scan and projection kernels (gfx950).
//
// Element types: the I/O dtype of the filter path is either fp32 or bf16
// (bf16 carried as raw uint16 bits).  State and arithmetic are always fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ltv {

typedef uint16_t bf16_t;

// ---------------------------------------------------------------------------
// bf16 <-> fp32 (round-to-nearest-even, NaN kept quiet)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two fp32 -> packed bf16 pair (lo in bits 0..15), round-to-nearest-even, on
// the gfx950 conversion unit (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

template <typename TIO>
struct io_traits;

template <>
struct io_traits<float> {
  static constexpr int kVec = 4;  // elements per 16-byte vector
  __device__ static __forceinline__ float load(const float* p) { return *p; }
  __device__ static __forceinline__ void store(float* p, float v) { *p = v; }
};

template <>
struct io_traits<bf16_t> {
  static constexpr int kVec = 8;
  __device__ static __forceinline__ float load(const bf16_t* p) {
    return bf16_to_f32(*p);
  }
  __device__ static __forceinline__ void store(bf16_t* p, float v) {
    *p = (bf16_t)f32_to_bf16_bits(v);
  }
};

// 16-byte vector of I/O elements <-> kVec floats.
__device__ __forceinline__ void unpack16(const uint4& q, float (&o)[4], float) {
  o[0] = __uint_as_float(q.x);
  o[1] = __uint_as_float(q.y);
  o[2] = __uint_as_float(q.z);
  o[3] = __uint_as_float(q.w);
}
__device__ __forceinline__ void unpack16(const uint4& q, float (&o)[8], bf16_t) {
  o[0] = __uint_as_float(q.x << 16);
  o[1] = __uint_as_float(q.x & 0xffff0000u);
  o[2] = __uint_as_float(q.y << 16);
  o[3] = __uint_as_float(q.y & 0xffff0000u);
  o[4] = __uint_as_float(q.z << 16);
  o[5] = __uint_as_float(q.z & 0xffff0000u);
  o[6] = __uint_as_float(q.w << 16);
  o[7] = __uint_as_float(q.w & 0xffff0000u);
}
__device__ __forceinline__ uint4 pack16(const float (&v)[4], float) {
  return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]),
                    __float_as_uint(v[2]), __float_as_uint(v[3]));
}
__device__ __forceinline__ uint4 pack16(const float (&v)[8], bf16_t) {
  uint4 q;
  q.x = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
  q.y = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
  q.z = f32_to_bf16_bits(v[4]) | (f32_to_bf16_bits(v[5]) << 16);
  q.w = f32_to_bf16_bits(v[6]) | (f32_to_bf16_bits(v[7]) << 16);
  return q;
}

// ---------------------------------------------------------------------------
// Gate: alpha = 1 / (1 + e^{-x}).  e^{-x} = 2^{-x log2 e} on the hardware
// exp2 unit (v_exp_f32) and the reciprocal on v_rcp_f32 (1 ulp).  For
// x -> +inf the exponent underflows to 0 (alpha = 1); for x -> -inf it
// overflows to +inf and the reciprocal gives 0 (alpha = 0).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sigmoid_f32(float x) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float gate_alpha(float logit_plus_bias, bool use_sigmoid) {
  return use_sigmoid ? sigmoid_f32(logit_plus_bias) : logit_plus_bias;
}

}  // namespace ltv
