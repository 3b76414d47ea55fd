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
// Work split: one workgroup per (head h, 16-channel block cb, 32-token block
// tb).  Its 32 MFMA rows are the block's 16 value rows and, from row 16, the
// gate rows its channels use (channels c0 .. c0 + 15 use gates c0 / r ..
// (c0 + 15) / r: at most 16), so one 32 x 32 block covers values and gates.
// Six wavefronts, each a sixth of the reduction (8 k16 steps at C = 768: 256
// contiguous bytes of every row), load all their operand fragments straight
// from global memory in one batch, then run their MFMAs; the partial blocks
// are summed through LDS in a fixed order and feed the recurrence step, one
// thread per (token, channel).  The step is latency-bound (7,000 MFMAs and
// 4 MB of weight at d12, B = 64).  Measured on MI355X (d12, B = 64, kernel
// durations): the earlier (head, 32 channels) split with 72 workgroups 13.2
// us; this split with 16 wavefronts of 3 k16 steps 9.8 us, with 12 of 4 8.6
// us, with 6 of 8 7.9 us -- a fragment load touches one 32-byte piece of 32
// rows, and the longer a wavefront's stretch of each row, the more of those
// pieces the L1 merges into one L2 request.  The same kernel with no operand
// loads or MFMAs takes 5.1 us (an empty launch 1.4 us): the floor of a launch
// that loads, reduces and stores.
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
  // it (one workgroup per (head, 16 channels, 32 tokens), and in it one thread
  // per (token, channel) for the read and the store alike).
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

constexpr int kDecCh = 16;       // channels per workgroup
constexpr int kDecKSlices = 6;   // wavefronts: slices of the reduction
constexpr int kDecThreads = kDecKSlices * 64;
constexpr int kDecBatch = 8;     // k16 steps whose loads are in flight together

__global__ void __launch_bounds__(kDecThreads) qkv_decode_kernel(const DecodeArgs a) {
  // [k slice][row: 16 values, then 16 gates][token]
  __shared__ float lds_p[kDecKSlices][32][33];

  const int H = a.NH + 2 * a.NKVH;
  const int nblk = (a.D + kDecCh - 1) / kDecCh;
  const int ntb = (a.B + 31) / 32;
  // workgroup w runs on XCD w % 8: the workgroups are dealt to the XCDs in
  // contiguous ranges of (head, channel block, token block), so the token
  // blocks that read the same weight rows share one L2
  const int nb = (int)gridDim.x, xcd = (int)blockIdx.x % 8, q = nb / 8, rr = nb % 8;
  const int u = xcd * q + (xcd < rr ? xcd : rr) + (int)blockIdx.x / 8;
  const int tb = u % ntb;
  const int hc = u / ntb;
  const int h = hc / nblk, cb = hc % nblk;
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // k slice

  const int c0 = cb * kDecCh;
  const int j0 = c0 / a.r;
  const int ngate = (min(c0 + kDecCh, a.D) - 1) / a.r - j0 + 1;  // <= 16

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

  // the recurrence step's inputs other than the projection, loaded first so
  // their latency overlaps the MFMA phase: item it -> (token it / 16, channel
  // it % 16), kDecItems items per thread
  constexpr int kDecItems = (32 * kDecCh + kDecThreads - 1) / kDecThreads;
  float hp[kDecItems], bias[kDecItems];
#pragma unroll
  for (int q = 0; q < kDecItems; ++q) {
    const int it = threadIdx.x + q * kDecThreads;
    const int it_m = it / kDecCh, m_out = tb * 32 + it_m, ch_out = c0 + it % kDecCh;
    const bool out_ok = it_m < 32 && m_out < a.B && ch_out < a.D;
    hp[q] = out_ok ? bf16_to_f32(prevp[(int64_t)m_out * psb + ch_out]) : 0.0f;
    bias[q] = out_ok ? a.bias[h * a.Da + ch_out / a.r] : 0.0f;
  }

  // MFMA phase: row ri of the block, k offset kh within each k16 step
  const int ri = lane & 31, kh = 8 * (lane >> 5);
  const bool vrow = ri < kDecCh;
  const bool row_ok = vrow ? c0 + ri < a.D : ri - kDecCh < ngate;
  const int64_t nrow = vrow ? (int64_t)h * a.D + c0 + ri
                            : (int64_t)H * a.D + (int64_t)h * a.Da + j0 + (ri - kDecCh);
  const bf16_t* wrow = a.wp + (row_ok ? nrow : 0) * a.C + kh;
  const int m = tb * 32 + ri;
  const bool tok_ok = m < a.B;
  const bf16_t* xrow = a.x + (int64_t)(tok_ok ? m : 0) * a.xs + kh;
  const int nk = a.C / 16;
  const int per = (nk + kDecKSlices - 1) / kDecKSlices;
  const int kb = ks * per, ke = min(nk, kb + per);
  f32x16_t acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
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
  // acc[4 q + e] = partial comb(row 8 q + 4 (lane / 32) + e, token lane % 32)
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) lds_p[ks][8 * q + 4 * (lane >> 5) + e][ri] = acc[4 * q + e];
  __syncthreads();

  // recurrence step: the k slices summed in a fixed order, then rounded to
  // bf16 as the projection stores the values and logits
#pragma unroll
  for (int q = 0; q < kDecItems; ++q) {
    const int it = threadIdx.x + q * kDecThreads;
    const int it_c = it % kDecCh, it_m = it / kDecCh;
    const int m_out = tb * 32 + it_m, ch_out = c0 + it_c;
    if (it_m < 32 && m_out < a.B && ch_out < a.D) {
      const int jl = ch_out / a.r - j0;
      float u = 0.0f, z = 0.0f;
#pragma unroll
      for (int s = 0; s < kDecKSlices; ++s) {
        u += lds_p[s][it_c][it_m];
        z += lds_p[s][kDecCh + jl][it_m];
      }
      u = bf16_round_f32(u);
      z = bf16_round_f32(z) + bias[q];
      const float alpha = gate_alpha(z, a.use_sigmoid != 0);
      const float hn = fmaf(alpha, u - hp[q], hp[q]);
      const bf16_t hb = (bf16_t)f32_to_bf16_bits(hn);
      a.out[((int64_t)m_out * H + h) * a.D + ch_out] = hb;
      if (rowsp != nullptr) rowsp[(int64_t)m_out * rsb + ch_out] = hb;
    }
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
  const int64_t grid64 = (int64_t)H * ((D + kDecCh - 1) / kDecCh) * ((B + 31) / 32);
  LTV_REQUIRE(grid64 < (1ll << 31), LTV_ERR_UNSUPPORTED, "decode grid too large");
  const int grid = (int)grid64;
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
