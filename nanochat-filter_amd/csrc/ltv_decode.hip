// One decode step (T = 1) of the LTV combined-QKV filter, fused into a single
// kernel: the bf16 projection of the B new tokens and one step of the gated
// recurrence from each head's previous output row (what the KV cache holds).
//
//   comb[m, n] = bf16( sum_c x[m, c] Wp[n, c] )    fp32 accumulation, rounded to
//                                                   bf16 as the projection stores it
//   alpha      = sigmoid(comb[m, logit(h, j)] + bias[h, j])   (or the raw sum)
//   out[m,h,d] = bf16( prev + alpha (u - prev) ),  u = comb[m, value(h, d)],
//                                                   prev = previous row (bf16)
//
// This is the computation the reference runs at decode through its general
// path -- the filter forward with T = 1 (ltv_cuda_fused_concat_head_major_
// register_cast_blelloch_scan_qkv_filter.py:24-73) fed by the KV cache's last
// rows (ltv_combined_qkv_computer_module.py:28-41) -- in one launch instead of
// a projection, a layout change and a scan.  The step form and the bf16
// rounding points are those of the scan and projection kernels, so a decode
// step equals the corresponding step of a full recompute up to fp32
// summation order in the projection.
//
// Work split: one workgroup per (head h, 32-channel block cb).  Its features
// are the 32 value rows of the block and the 32 packed rows starting at the
// block's first gate row (every gate the block's channels use; r >= 1 means at
// most 32).  Sixteen wavefronts: wave w computes, over k slice w / 4 of the
// reduction, the 32 x 32 MFMA block of feature block (w & 1) and token block
// ((w >> 1) & 1) + 2 i, i = 0, 1, ..., with operand fragments loaded straight
// from global memory (the weight slice is read once per workgroup; tokens come
// from L2).  The partial blocks go through LDS, are summed in a fixed order and
// feed the recurrence step, which writes 32 consecutive channels per token.
#include "ltv_abi_internal.hpp"
#include "ltv_device.hpp"
#include "ltv_gemm_mfma.hpp"

namespace ltv {
namespace {

struct DecodeArgs {
  const bf16_t* x;    // (B, C), row stride xs
  int64_t xs;
  const bf16_t* wp;   // packed (Fp, C)
  const bf16_t* prev[3];     // previous rows of q, k, v: (B, H_g, D), strides (b, h), d = 1
  int64_t prev_s[3][2];
  const float* bias;  // (H, Da)
  bf16_t* out;        // (B, H, D) contiguous
  // optional second copy of the new rows of q, k, v: (B, H_g, D), strides
  // (b, h), d = 1 (null: none).  May be the previous rows themselves: every
  // element of prev is read, before it is written, by the thread that writes
  // it (one workgroup per (head, 32 channels), and in it one thread per
  // (token, channel) for the read and the store alike).
  bf16_t* rows[3];
  int64_t rows_s[3][2];
  int B, C, NH, NKVH, D, Da, r, Fp, use_sigmoid;
};

__device__ __forceinline__ float bf16_round_f32(float v) {
  return __uint_as_float(f32_to_bf16_bits(v) << 16);
}

__device__ __forceinline__ bf16x8_t load_frag(const bf16_t* row, bool ok) {
  if (!ok) return bf16x8_t{};
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(row));
}

constexpr int kDecKSlices = 4;  // the reduction split across wavefronts
constexpr int kDecThreads = 2 * 2 * kDecKSlices * 64;
constexpr int kDecBatch = 8;

__global__ void __launch_bounds__(kDecThreads) qkv_decode_kernel(const DecodeArgs a) {
  // [k slice][token block slot][feature block][feature][token]
  __shared__ float lds_p[kDecKSlices][2][2][32][33];

  const int H = a.NH + 2 * a.NKVH;
  const int nblk = (a.D + 31) / 32;
  const int h = blockIdx.x / nblk, cb = blockIdx.x % nblk;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fb = wave & 1;    // 0: value rows, 1: gate rows
  const int tslot = (wave >> 1) & 1;
  const int ks = wave >> 2;   // k slice

  const int c0 = cb * 32;
  const int j0 = c0 / a.r;
  const int nrow0 = fb == 0 ? h * a.D + c0 : H * a.D + h * a.Da + j0;
  // valid feature rows of this wave's block
  const int nrows = fb == 0 ? min(32, a.D - c0) : min(32, a.Da - j0);

  int g, hl;
  if (h < a.NH) {
    g = 0;
    hl = h;
  } else if (h < a.NH + a.NKVH) {
    g = 1;
    hl = h - a.NH;
  } else {
    g = 2;
    hl = h - a.NH - a.NKVH;
  }
  const bf16_t* prevp = g == 0 ? a.prev[0] : g == 1 ? a.prev[1] : a.prev[2];
  const int64_t psb = g == 0 ? a.prev_s[0][0] : g == 1 ? a.prev_s[1][0] : a.prev_s[2][0];
  const int64_t psh = g == 0 ? a.prev_s[0][1] : g == 1 ? a.prev_s[1][1] : a.prev_s[2][1];
  prevp += (int64_t)hl * psh;
  bf16_t* rowsp = a.rows[g];
  const int64_t rsb = a.rows_s[g][0];
  if (rowsp != nullptr) rowsp += (int64_t)hl * a.rows_s[g][1];

  const int nk = a.C / 16;
  const int per = (nk + kDecKSlices - 1) / kDecKSlices;
  const int kb = ks * per, ke = min(nk, kb + per);
  const int ntb = (a.B + 31) / 32;
  const int ri = lane & 31, kh = 8 * (lane >> 5);
  const bool row_ok = ri < nrows;
  const bf16_t* wrow = a.wp + (int64_t)(nrow0 + ri) * a.C + kh;

  const float* bias_h = a.bias + h * a.Da;
  for (int tb0 = 0; tb0 < ntb; tb0 += 2) {
    // the recurrence step's inputs other than the projection, loaded first so
    // their latency overlaps the MFMA phase: thread -> (slot, token, channel)
    constexpr int kItems = 2 * 32 * 32 / kDecThreads;
    float hp_pre[kItems], bias_pre[kItems];
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
      const int it = threadIdx.x + q * kDecThreads;
      const int c = it & 31, mi = (it >> 5) & 31, s = it >> 10;
      const int m = (tb0 + s) * 32 + mi, ch = c0 + c;
      const bool ok = tb0 + s < ntb && m < a.B && ch < a.D;
      hp_pre[q] = ok ? bf16_to_f32(prevp[(int64_t)m * psb + ch]) : 0.0f;
      bias_pre[q] = ok ? bias_h[min(ch, a.D - 1) / a.r] : 0.0f;
    }
    const int tb = tb0 + tslot;
    if (tb < ntb) {
      const int m = tb * 32 + ri;
      const bool tok_ok = m < a.B;
      const bf16_t* xrow = a.x + (int64_t)m * a.xs + kh;
      f32x16_t acc;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
      // batches of kDecBatch k16 steps: all of a batch's fragment loads are
      // issued before its MFMAs
      for (int k0 = kb; k0 < ke; k0 += kDecBatch) {
        bf16x8_t wf[kDecBatch], xf[kDecBatch];
#pragma unroll
        for (int i = 0; i < kDecBatch; ++i) {
          const bool kok = k0 + i < ke;
          wf[i] = load_frag(wrow + 16 * (k0 + i), row_ok && kok);
          xf[i] = load_frag(xrow + 16 * (k0 + i), tok_ok && kok);
        }
#pragma unroll
        for (int i = 0; i < kDecBatch; ++i)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], xf[i], acc, 0, 0, 0);
      }
      // acc[4 q + e] = partial comb(feature 8 q + 4 (lane / 32) + e, token lane % 32)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          lds_p[ks][tslot][fb][8 * q + 4 * (lane >> 5) + e][ri] = acc[4 * q + e];
    }
    __syncthreads();
    // recurrence step: thread -> (token block slot, token, channel), channels
    // fastest; the k slices are summed in a fixed order, then rounded to bf16
    // as the projection stores the values and logits
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
      const int it = threadIdx.x + q * kDecThreads;
      const int c = it & 31, mi = (it >> 5) & 31, s = it >> 10;
      const int tbs = tb0 + s;
      const int m = tbs * 32 + mi, ch = c0 + c;
      if (tbs < ntb && m < a.B && ch < a.D) {
        const int jl = ch / a.r - j0;
        float u = 0.0f, z = 0.0f;
#pragma unroll
        for (int q = 0; q < kDecKSlices; ++q) {
          u += lds_p[q][s][0][c][mi];
          z += lds_p[q][s][1][jl][mi];
        }
        u = bf16_round_f32(u);
        z = bf16_round_f32(z) + bias_pre[q];
        const float alpha = gate_alpha(z, a.use_sigmoid != 0);
        const float hp = hp_pre[q];
        const float hn = fmaf(alpha, u - hp, hp);
        const bf16_t hb = (bf16_t)f32_to_bf16_bits(hn);
        a.out[((int64_t)m * H + h) * a.D + ch] = hb;
        if (rowsp != nullptr) rowsp[(int64_t)m * rsb + ch] = hb;
      }
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace ltv

using namespace ltv;

namespace {
int decode_step_impl(const void* x, int64_t x_row_stride, const void* wpack, const void* prev_q,
                     const void* prev_k, const void* prev_v, const int64_t prev_strides[6],
                     const float* logit_bias, void* out, void* rows_q, void* rows_k,
                     void* rows_v, const int64_t rows_strides[6], int B, int C, int NH, int NKVH,
                     int D, int Da, int use_sigmoid, void* stream) {
  LTV_REQUIRE(B >= 0 && C > 0 && NH >= 0 && NKVH >= 0 && D > 0 && Da > 0, LTV_ERR_INVALID_ARG,
              "bad shape (B=%d C=%d NH=%d NKVH=%d D=%d Da=%d)", B, C, NH, NKVH, D, Da);
  LTV_REQUIRE(D % Da == 0, LTV_ERR_INVALID_ARG, "Da=%d must divide D=%d", Da, D);
  LTV_REQUIRE(C % 16 == 0, LTV_ERR_UNSUPPORTED, "C must be a multiple of 16 (C=%d)", C);
  const int H = NH + 2 * NKVH;
  if (B == 0 || H == 0) return LTV_OK;
  LTV_REQUIRE(x && wpack && logit_bias && out && prev_strides, LTV_ERR_INVALID_ARG,
              "null pointer");
  LTV_REQUIRE((NH == 0 || prev_q) && (NKVH == 0 || (prev_k && prev_v)), LTV_ERR_INVALID_ARG,
              "null previous-row pointer");
  LTV_REQUIRE(aligned16(x) && aligned16(wpack) && x_row_stride % 8 == 0, LTV_ERR_INVALID_ARG,
              "x and wpack must be 16-byte aligned, x rows a multiple of 8 elements apart");
  const int Fp = ltv_qkv_packed_width(H, D, Da);
  LTV_REQUIRE((int64_t)Fp * C < (1ll << 31) && (int64_t)B * x_row_stride < (1ll << 40),
              LTV_ERR_UNSUPPORTED, "decode operands too large");
  DecodeArgs a;
  a.x = reinterpret_cast<const bf16_t*>(x);
  a.xs = x_row_stride;
  a.wp = reinterpret_cast<const bf16_t*>(wpack);
  a.prev[0] = reinterpret_cast<const bf16_t*>(prev_q);
  a.prev[1] = reinterpret_cast<const bf16_t*>(prev_k);
  a.prev[2] = reinterpret_cast<const bf16_t*>(prev_v);
  for (int i = 0; i < 3; ++i) {
    a.prev_s[i][0] = prev_strides[2 * i];
    a.prev_s[i][1] = prev_strides[2 * i + 1];
  }
  a.bias = logit_bias;
  a.out = reinterpret_cast<bf16_t*>(out);
  void* const rows[3] = {rows_q, rows_k, rows_v};
  for (int i = 0; i < 3; ++i) {
    a.rows[i] = nullptr;
    a.rows_s[i][0] = a.rows_s[i][1] = 0;
    if (rows_strides != nullptr && rows[i] != nullptr && (i == 0 ? NH : NKVH) > 0) {
      a.rows[i] = reinterpret_cast<bf16_t*>(rows[i]);
      a.rows_s[i][0] = rows_strides[2 * i];
      a.rows_s[i][1] = rows_strides[2 * i + 1];
    }
  }
  a.B = B;
  a.C = C;
  a.NH = NH;
  a.NKVH = NKVH;
  a.D = D;
  a.Da = Da;
  a.r = D / Da;
  a.Fp = Fp;
  a.use_sigmoid = use_sigmoid;
  const int grid = H * ((D + 31) / 32);
  hipLaunchKernelGGL(qkv_decode_kernel, dim3(grid), dim3(kDecThreads), 0, (hipStream_t)stream, a);
  LTV_LAUNCH_CHECK();
  return LTV_OK;
}
}  // namespace

extern "C" int ltv_qkv_decode_step(const void* x, int64_t x_row_stride, const void* wpack,
                                   const void* prev_q, const void* prev_k, const void* prev_v,
                                   const int64_t prev_strides[6], const float* logit_bias,
                                   void* out, int B, int C, int NH, int NKVH, int D, int Da,
                                   int use_sigmoid, void* stream) {
  return decode_step_impl(x, x_row_stride, wpack, prev_q, prev_k, prev_v, prev_strides,
                          logit_bias, out, nullptr, nullptr, nullptr, nullptr, B, C, NH, NKVH, D,
                          Da, use_sigmoid, stream);
}

extern "C" int ltv_qkv_decode_step_rows(const void* x, int64_t x_row_stride, const void* wpack,
                                        void* prev_q, void* prev_k, void* prev_v,
                                        const int64_t prev_strides[6], const float* logit_bias,
                                        void* out, void* rows_q, void* rows_k, void* rows_v,
                                        const int64_t rows_strides[6], int B, int C, int NH,
                                        int NKVH, int D, int Da, int use_sigmoid, void* stream) {
  LTV_REQUIRE(rows_strides != nullptr, LTV_ERR_INVALID_ARG, "null rows stride array");
  LTV_REQUIRE((NH == 0 || rows_q) && (NKVH == 0 || (rows_k && rows_v)), LTV_ERR_INVALID_ARG,
              "null rows pointer");
  return decode_step_impl(x, x_row_stride, wpack, prev_q, prev_k, prev_v, prev_strides,
                          logit_bias, out, rows_q, rows_k, rows_v, rows_strides, B, C, NH, NKVH,
                          D, Da, use_sigmoid, stream);
}
