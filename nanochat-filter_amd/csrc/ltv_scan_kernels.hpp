// LTV head-major gated EWMA scan, forward and backward, for gfx950.
//
// Recurrence (per channel d of head h, gate group j = d / r):
//   alpha_t = sigmoid(logit_t[j] + bias[h, j])          (or the raw sum)
//   h_t     = (1 - alpha_t) * h_{t-1} + alpha_t * u_t,   h_{-1} = inits
// as in nanochat/ops/ltv_reference_ops.py:83-124 and the CUDA kernels
// cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_{forward,backward}.cu.
// Each step is evaluated as h + alpha * (u - h) (one subtract, one FMA).
//
// Work decomposition (a workgroup owns all of T for one (b, head, channel slab)):
//   * a lane owns V = 16 / sizeof(io) consecutive channels (one 16-byte vector)
//     and a run of L consecutive time steps; the L vectors stay packed in
//     registers in the I/O format and are widened to fp32 when used;
//   * a 64-lane wavefront is CL channel lanes x TG = 64 / CL time groups, lane =
//     cl * TG + tg, so the TG time groups of one channel vector are adjacent lanes
//     of one 16-lane DPP row (when TG <= 16);
//   * NW wavefronts split time further; one tile covers TW = NW * TG * L steps and
//     the workgroup walks T tile by tile, carrying the fp32 state in registers.
// A tile is a three-level affine scan of (A, X) pairs, (A1,X1) then (A2,X2) =
// (A1 A2, A2 X1 + X2):
//   1. per lane: sequential fold of its L steps;
//   2. per wavefront: inclusive scan over the TG time-group lanes (DPP row shifts);
//   3. per workgroup: wavefront totals through LDS (one barrier per tile),
//      composed in wavefront order onto the running carry.
// The lane then re-runs its L steps from its exact carry-in and stores, so every
// element is read from HBM once and written once.
//
// The backward walks the tiles in reverse.  Per tile each lane reads the state
// entering its first step from the saved outputs (the inits at t = 0) -- the
// I/O-dtype state the reference backward reads back, ltv_reference_ops.py:7-34
// -- and recomputes the states of its other steps from it, rounded to the I/O
// dtype like the saved outputs; then it runs the reverse scan
//   g_t = gy_t + (1 - alpha_{t+1}) g_{t+1},   g_T = 0
// and emits du = alpha g, dalpha = (u - h_{t-1}) g reduced over each gate group,
// dlogit = alpha (1 - alpha) dalpha, dinit = (1 - alpha_0) g_0 and a per-(b, h)
// dbias partial.  All reductions run in a fixed order (LDS, no atomics), so the
// results are bitwise reproducible.

#pragma once

#include <type_traits>

#include "ltv_device.hpp"
#include "ltv_abi_internal.hpp"

namespace ltv {

// ---------------------------------------------------------------------------
// Argument blocks (passed by value as kernel arguments)
// ---------------------------------------------------------------------------
struct View4 {
  const void* p;
  int64_t s[4];  // element strides (b, h, t, c)
};

struct OutHeads {
  void* p[3];       // q, k, v
  int64_t s[3][4];  // element strides (b, h_local, t, d)
};

// One of the q / k / v members of an OutHeads, picked with selects: indexing
// the argument block with the run-time head group makes the compiler re-read
// the strides from memory (and wait for them) before every use.
struct HeadView {
  void* p;
  int64_t s[4];
};

__device__ __forceinline__ HeadView head_view(const OutHeads& o, int which) {
  HeadView r;
  r.p = which == 0 ? o.p[0] : which == 1 ? o.p[1] : o.p[2];
#pragma unroll
  for (int k = 0; k < 4; ++k) r.s[k] = which == 0 ? o.s[0][k] : which == 1 ? o.s[1][k] : o.s[2][k];
  return r;
}

struct ScanShape {
  int B, T, NH, NKVH, Da, r, D, H;
  int nslab;  // channel slabs per head (forward only)
  int use_sigmoid;
};

// Chunk windows of the look-back scan (nanochat/ops/ltv_reference_ops.py:65-75,
// 99-101): chunk 0 covers [0, min(P, T)), chunk c >= 1 covers
// [P + (c - 1) Q, min(P + c Q, T)); each chunk [st, hi) restarts the recurrence
// from the inits at lo = max(0, st - (K - 1)) and owns the outputs of [st, hi).
// P >= T gives the single window [0, T) of the full recurrence.
struct Window {
  int lo, st, hi;
};

__host__ __device__ inline Window look_back_window(int c, int T, int P, int Q, int K) {
  Window w;
  if (c == 0) {
    w.st = 0;
    w.hi = P < T ? P : T;
  } else {
    w.st = P + (c - 1) * Q;  // < T for every chunk that exists
    w.hi = (int64_t)w.st + Q < T ? w.st + Q : T;
  }
  w.lo = w.st - (K - 1) > 0 ? w.st - (K - 1) : 0;
  return w;
}

// Number of chunk windows (1 when P >= T).
__host__ __device__ inline int look_back_nwin(int T, int P, int Q) {
  return T > P ? 1 + (int)(((int64_t)T - P + Q - 1) / Q) : 1;
}

// Host-set control of the chained kernels' bounded carry waits.
struct ChainCtl {
  // Mapped host word (or null): a chained launch that fails stores its error
  // code there as well as in the workspace header, so the host learns of it
  // without a device synchronisation.
  uint32_t* host_err;
  int spin_max;    // polls before a carry wait gives up
  int no_publish;  // test hook: publishers publish nothing, every wait runs out
};

struct FwdArgs {
  ScanShape sh;
  View4 u;     // values   (B, H, T, D)
  View4 lg;    // logits   (B, H, T, Da)
  View4 init;  // inits    (B, H, D) -- s[2] unused
  // 1: the inits are fp32 in memory (with bf16 I/O), rounded to bf16 when read
  int init_f32;
  const float* bias;  // (H, Da) contiguous fp32
  OutHeads out;
  int P, Q, K, nwin;  // chunk windows; one workgroup per (b, h, window, slab)
  // Warm-up mode (wst != null): each window runs only its warm-up [lo, st) and
  // stores the states to wst (B, H, nwin, kw, D) in the I/O dtype, row t - lo.
  void* wst;
  int kw;
  int lanes;  // short-window kernels: lanes per window (a power of two >= D / V)
};

struct BwdArgs {
  ScanShape sh;
  View4 u;
  View4 lg;
  View4 init;
  const float* bias;
  OutHeads h;     // saved forward outputs
  OutHeads gy;    // upstream gradients
  View4 du;       // gradient of the value slots (B, H, T, D)
  View4 dlg;      // gradient of the logit slots (B, H, T, Da)
  View4 dinit;    // (B, H, D)
  // 1: inits and dinit are fp32 in memory (with bf16 I/O); the inits are
  // rounded to bf16 when read, the dinit values to bf16 before they are
  // widened and stored (the gradient of a bf16 tensor cast from fp32)
  int init_f32;
  // non-null: dinit goes here instead, (B H, D) fp32 contiguous, rounded to
  // the I/O dtype, for the reduction that sums it over the batch
  float* dinit_ws;
  float* dbias_partial;  // (B, H, nchunk, Da) fp32 workspace
  // Time chunks: the tile kernel runs one workgroup per (b, h, chunk) of
  // chunk_steps steps (a multiple of its tile), entering each chunk with the
  // gradient carry g at the chunk's end from `carry` (B H, nchunk, D); with
  // nchunk == 1 the carry is 0 and `carry` is unused.
  int nchunk, chunk_steps;
  // The chunk maps are formed over finer sub-chunks of fine_steps steps (a
  // divisor of chunk_steps), nfine per sequence, for parallelism.
  int nfine, fine_steps;
  float* agg;          // (2, B H, nfine, D): each sub-chunk's map g_start = A g_end + G
  float* carry;        // (B H, nchunk, D)
  // Look-back windows (the LB kernels): chunk c of the nchunk = nwin windows
  // runs its own reverse chain over [lo, hi) from g_hi = 0 with upstream
  // gradients on [st, hi) only.  The states entering its warm-up steps come
  // from wst (B, H, nwin, kw, D), I/O dtype, row t - lo; its contributions on
  // warm-up steps go to wdu (B, H, nwin, kw, D) and wdl (B, H, nwin, kw, Da)
  // in fp32 (added to the owning chunk's gradient by scan_lb_fold_kernel), and
  // its inits gradient to wdi (B, H, nwin, D).
  int P, Q, K, kw;
  const void* wst;
  float* wdu;
  float* wdl;
  float* wdi;
  int lanes;  // short-window kernel: lanes per window (a power of two >= D / V)
  int wpl;    // short-window backward: consecutive windows per lane (1: one each)
  // Chained mode of the tile kernel (one tile per chunk, chunks of a sequence
  // handed their gradient carry through tagged words): the ticket counter, the
  // error word and the words, (B H, nchunk - 1, CL V) -- the same zeroed
  // workspace layout as the chained forward's.
  uint32_t* ch_ticket;
  uint32_t* ch_err;
  unsigned long long* ch_words;
  ChainCtl ch_ctl;
};

// How a lane finds the gate of each of its V channels.
enum GateMode {
  GATE_LANE = 0,     // r % V == 0: one gate for the whole lane
  GATE_CHAN = 1,     // per-channel gate j = c / r, scalar logit loads
  GATE_CHANVEC = 2,  // r == 1 with channel-contiguous logits: one 16-byte logit load
};

__device__ __forceinline__ void head_select(int h, int NH, int NKVH, int& which, int& hl) {
  if (h < NH) {
    which = 0;
    hl = h;
  } else if (h < NH + NKVH) {
    which = 1;
    hl = h - NH;
  } else {
    which = 2;
    hl = h - NH - NKVH;
  }
}

// ---------------------------------------------------------------------------
// Packed 16-byte vectors of I/O elements
// ---------------------------------------------------------------------------
template <typename TIO>
struct Pack;

template <>
struct Pack<bf16_t> {
  static constexpr int V = 8;
  __device__ static __forceinline__ float get(const uint4& q, int v) {
    const uint32_t w = v < 2 ? q.x : v < 4 ? q.y : v < 6 ? q.z : q.w;
    return __uint_as_float((v & 1) ? (w & 0xffff0000u) : (w << 16));
  }
  __device__ static __forceinline__ uint32_t raw(const bf16_t* p) { return *p; }
  __device__ static __forceinline__ void put_raw(uint32_t (&w)[4], int v, uint32_t bits) {
    w[v >> 1] |= bits << (16 * (v & 1));
  }
  __device__ static __forceinline__ uint4 pack(const float (&x)[8]) {
    return make_uint4(cvt_pk_bf16(x[0], x[1]), cvt_pk_bf16(x[2], x[3]),
                      cvt_pk_bf16(x[4], x[5]), cvt_pk_bf16(x[6], x[7]));
  }
  __device__ static __forceinline__ void store1(bf16_t* p, float x) {
    *p = (bf16_t)(cvt_pk_bf16(x, 0.0f) & 0xffffu);
  }
  __device__ static __forceinline__ float load1(const bf16_t* p) {
    return __uint_as_float((uint32_t)*p << 16);
  }
};

template <>
struct Pack<float> {
  static constexpr int V = 4;
  __device__ static __forceinline__ float get(const uint4& q, int v) {
    return __uint_as_float(v == 0 ? q.x : v == 1 ? q.y : v == 2 ? q.z : q.w);
  }
  __device__ static __forceinline__ uint32_t raw(const float* p) { return __float_as_uint(*p); }
  __device__ static __forceinline__ void put_raw(uint32_t (&w)[4], int v, uint32_t bits) {
    w[v] = bits;
  }
  __device__ static __forceinline__ uint4 pack(const float (&x)[4]) {
    return make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                      __float_as_uint(x[3]));
  }
  __device__ static __forceinline__ void store1(float* p, float x) { *p = x; }
  __device__ static __forceinline__ float load1(const float* p) { return *p; }
};

// V channels at base, base + sc, ... (channels >= nvalid read as zero).
template <typename TIO, bool VEC>
__device__ __forceinline__ uint4 ld_vec(const TIO* base, int64_t sc, int nvalid) {
  if (VEC) return *reinterpret_cast<const uint4*>(base);
  constexpr int V = Pack<TIO>::V;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int v = 0; v < V; ++v)
    if (v < nvalid) Pack<TIO>::put_raw(w, v, Pack<TIO>::raw(base + v * sc));
  return make_uint4(w[0], w[1], w[2], w[3]);
}

template <typename TIO, bool VEC>
__device__ __forceinline__ void st_vec(TIO* base, int64_t sc, int nvalid,
                                       const float (&x)[Pack<TIO>::V]) {
  if (VEC) {
    *reinterpret_cast<uint4*>(base) = Pack<TIO>::pack(x);
  } else {
#pragma unroll
    for (int v = 0; v < Pack<TIO>::V; ++v)
      if (v < nvalid) Pack<TIO>::store1(base + v * sc, x[v]);
  }
}

// V fp32 values to p[0], ..., p[nvalid - 1] (16-byte stores when VEC: p is
// then 16-byte aligned and all V values are valid).
template <bool VEC, int V>
__device__ __forceinline__ void st_f32(float* p, int nvalid, const float (&x)[V]) {
  if (VEC) {
#pragma unroll
    for (int q = 0; q < V / 4; ++q)
      reinterpret_cast<float4*>(p)[q] = make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]);
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (v < nvalid) p[v] = x[v];
  }
}

// ---------------------------------------------------------------------------
// Buffer accesses of the tile kernels.  A buffer resource holds a wave-uniform
// base address (a view's (b, h) slice at the current tile's first step); each
// lane adds a 32-bit byte offset.  A lane that must not touch memory passes
// kOob: the range check turns its load into 0 and drops its store, so masked
// accesses need no branch.  Without branches the compiler counts the vector
// memory operations in flight exactly and waits only for those a use needs; a
// load or store under a data-dependent branch makes it drain the queue
// (vmcnt(0)) at the next wait, which puts the prefetch of the next tile
// behind the stores of the current one.  The host keeps every in-tile offset
// below 2^31 (scan_offsets_fit in the launcher).
// ---------------------------------------------------------------------------
using Rsrc = __amdgpu_buffer_rsrc_t;
constexpr uint32_t kOob = 0x80000000u;
typedef int i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ Rsrc make_rsrc(const void* base) {
  // num_records 2^31 - 1 bytes, raw (stride 0) addressing, 32-bit data format
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                           0x00020000);
}
// Store cache policy (the instruction's aux bits): kStNormal, or kStStream
// (gfx950 `nt`: non-temporal).  Measured on MI355X: streaming stores take the
// per-channel-gate forward (r = 1, configs[1]) from 106 to 91 us; they slow the
// d12 forward (62 -> 69 us) and the d12 backward (124 -> 128 us with streaming
// value gradients, 168 us with streaming 2-byte logit gradients: partial-line
// streaming writes), so everything else stores normally.
constexpr int kStNormal = 0;
constexpr int kStStream = 2;
// Load cache policy, the same bits: kLdStream (`nt`) marks data read once.
// Measured on MI355X at d12: the backward's value, output-gradient and state
// loads as streaming take it from 125 to 117 us, and the grad_x GEMM that
// follows it from 135 to 122 us (the grad_combined it reads stays cached);
// the forwards lose with them (configs[1] 95 -> 104 us, the look-back
// window kernels 67 -> 72 and 176 -> 179 us), so only the tile backward
// streams its loads.
constexpr int kLdNormal = 0;
constexpr int kLdStream = 2;
template <int AUX = kLdNormal>
__device__ __forceinline__ uint4 bld128(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
}
template <int AUX = kStNormal>
__device__ __forceinline__ void bst128(Rsrc r, uint32_t off, uint4 x) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, x), r, off, 0, AUX);
}
template <int AUX = kStNormal>
__device__ __forceinline__ void bst_b32(Rsrc r, uint32_t off, float x) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, off, 0, AUX);
}

// Hides x's value from the optimiser: offsets derived from it are formed where
// they are used instead of being hoisted out of the tile loop, where one live
// register per (step, channel) offset would cost more than the adds.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// log2 of a power of two
__host__ __device__ constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

// f(integral_constant<int, I>) for I = I0 .. N - 1
template <int I, int N, class F>
__device__ __forceinline__ void static_loop(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_loop<I + 1, N>(f);
  }
}

// One element as raw bits (bf16: the 16 bits; fp32: the word) and its store.
template <typename TIO, int AUX = kLdNormal>
__device__ __forceinline__ uint32_t bld1(Rsrc r, uint32_t off) {
  if constexpr (sizeof(TIO) == 2)
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, AUX);
  else
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
}
template <typename TIO, int AUX = kStNormal>
__device__ __forceinline__ void bst1(Rsrc r, uint32_t off, float x) {
  if constexpr (sizeof(TIO) == 2)
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)(cvt_pk_bf16(x, 0.0f) & 0xffffu), r,
                                          off, 0, AUX);
  else
    bst_b32<AUX>(r, off, x);
}

// V channels at byte offset off, scb bytes apart; channels >= nvalid and
// lanes with ok == false read 0.
template <typename TIO, bool VEC, int AUX = kLdNormal>
__device__ __forceinline__ uint4 bld_vec(Rsrc r, uint32_t off, uint32_t scb, int nvalid, bool ok) {
  if (VEC) return bld128<AUX>(r, ok ? off : kOob);
  constexpr int V = Pack<TIO>::V;
  off = opaque(off);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int v = 0; v < V; ++v)
    Pack<TIO>::put_raw(w, v, bld1<TIO, AUX>(r, ok && v < nvalid ? off + v * scb : kOob));
  return make_uint4(w[0], w[1], w[2], w[3]);
}

template <typename TIO, bool VEC, int AUX = kStNormal>
__device__ __forceinline__ void bst_vec(Rsrc r, uint32_t off, uint32_t scb, int nvalid, bool ok,
                                        const float (&x)[Pack<TIO>::V]) {
  if (VEC) {
    bst128<AUX>(r, ok ? off : kOob, Pack<TIO>::pack(x));
  } else {
    off = opaque(off);
#pragma unroll
    for (int v = 0; v < Pack<TIO>::V; ++v)
      bst1<TIO, AUX>(r, ok && v < nvalid ? off + v * scb : kOob, x[v]);
  }
}

// x rounded to the I/O dtype (the value a store and a reload would give).
template <typename TIO>
__device__ __forceinline__ float round_io(float x) {
  if constexpr (sizeof(TIO) == 2)
    return __uint_as_float(cvt_pk_bf16(x, 0.0f) << 16);
  else
    return x;
}

// The inits of V channels as a packed I/O vector.  With f32 (bf16 I/O only)
// they are fp32 in memory -- the parameter before the cast that feeds the
// reference's bf16 kernel -- and are rounded to bf16 here as that cast
// rounds them.  Pointer form (channel stride sc elements) and buffer form
// (byte offset off, channel stride scb bytes; lanes with ok == false read 0).
template <typename TIO, bool VEC>
__device__ __forceinline__ uint4 ld_init(const void* base, int64_t sc, int nvalid, bool f32) {
  if constexpr (sizeof(TIO) == 2 && VEC) {
    // no branch on the dtype (its join would wait for every load in flight):
    // the second 16 bytes are read from the fp32 row's second half, or again
    // from the first (never past the inits), and the result is selected
    const uint4* p4 = reinterpret_cast<const uint4*>(base);
    const uint4 a = p4[0];
    const uint4 b = *(f32 ? p4 + 1 : p4);
    const float x[8] = {__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z),
                        __uint_as_float(a.w), __uint_as_float(b.x), __uint_as_float(b.y),
                        __uint_as_float(b.z), __uint_as_float(b.w)};
    const uint4 cv = Pack<bf16_t>::pack(x);
    return make_uint4(f32 ? cv.x : a.x, f32 ? cv.y : a.y, f32 ? cv.z : a.z, f32 ? cv.w : a.w);
  } else if constexpr (sizeof(TIO) == 2) {
    if (f32) {
      const float* fp = reinterpret_cast<const float*>(base);
      float x[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) x[v] = v < nvalid ? fp[v * sc] : 0.0f;
      return Pack<bf16_t>::pack(x);
    }
  }
  return ld_vec<TIO, VEC>(reinterpret_cast<const TIO*>(base), sc, nvalid);
}
template <typename TIO, bool VEC>
__device__ __forceinline__ uint4 bld_init(Rsrc r, uint32_t off, uint32_t scb, int nvalid, bool ok,
                                          bool f32) {
  if constexpr (sizeof(TIO) == 2) {
    if (f32) {
      float x[8];
      if (VEC) {
        const uint4 lo = bld128(r, ok ? off : kOob), hi = bld128(r, ok ? off + 16u : kOob);
        x[0] = __uint_as_float(lo.x); x[1] = __uint_as_float(lo.y);
        x[2] = __uint_as_float(lo.z); x[3] = __uint_as_float(lo.w);
        x[4] = __uint_as_float(hi.x); x[5] = __uint_as_float(hi.y);
        x[6] = __uint_as_float(hi.z); x[7] = __uint_as_float(hi.w);
      } else {
        off = opaque(off);
#pragma unroll
        for (int v = 0; v < 8; ++v)
          x[v] = __uint_as_float(bld1<float>(r, ok && v < nvalid ? off + v * scb : kOob));
      }
      return Pack<bf16_t>::pack(x);
    }
  }
  return bld_vec<TIO, VEC>(r, off, scb, nvalid, ok);
}

// V fp32 values at off, off + 4, ... (16-byte stores when VEC: off is then
// 16-byte aligned and all V values are valid).
template <bool VEC, int V>
__device__ __forceinline__ void bst_f32(Rsrc r, uint32_t off, int nvalid, bool ok,
                                        const float (&x)[V]) {
  if (VEC) {
#pragma unroll
    for (int q = 0; q < V / 4; ++q)
      bst128(r, ok ? off + 16 * q : kOob,
             make_uint4(__float_as_uint(x[4 * q]), __float_as_uint(x[4 * q + 1]),
                        __float_as_uint(x[4 * q + 2]), __float_as_uint(x[4 * q + 3])));
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) bst_b32(r, ok && v < nvalid ? off + 4 * v : kOob, x[v]);
  }
}

// Makes the compiler treat the packed vectors as rewritten, so it widens them
// again where they are next used instead of keeping L x V fp32 copies alive
// across the scan levels (widening is one shift or mask per element).
template <int N>
__device__ __forceinline__ void reload_barrier(uint4 (&q)[N]) {
#pragma unroll
  for (int s = 0; s < N; ++s)
    asm volatile("" : "+v"(q[s].x), "+v"(q[s].y), "+v"(q[s].z), "+v"(q[s].w));
}

// ---------------------------------------------------------------------------
// Shifts inside segments of TG adjacent lanes.  For TG <= 16 the segment lies in
// one 16-lane row and a DPP row shift is exact for every lane the caller keeps
// (tg >= off, resp. tg + off < TG); wider segments go through ds_bpermute.
// ---------------------------------------------------------------------------
// Lanes without a source in the row read 0 (bound_ctrl): no old value to
// materialise, and the move can fold into the instruction that consumes it.
template <int TG, int OFF>
__device__ __forceinline__ float shift_up(float x) {
  if constexpr (TG <= 16) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x110 + OFF, 0xf, 0xf, true));
  } else {
    return __shfl_up(x, OFF, TG);
  }
}

template <int TG, int OFF>
__device__ __forceinline__ float shift_down(float x) {
  if constexpr (TG <= 16) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x100 + OFF, 0xf, 0xf, true));
  } else {
    return __shfl_down(x, OFF, TG);
  }
}

// Inclusive then exclusive prefix (time order) of (A, X) pairs over the TG lanes.
template <int TG, int NA, int V, int GI_LANE>
struct SegScan {
  template <int OFF>
  __device__ static __forceinline__ void up_level(int tg, float (&A)[NA], float (&X)[V]) {
    if constexpr (OFF < TG) {
      float Ap[NA], Xp[V];
#pragma unroll
      for (int i = 0; i < NA; ++i) Ap[i] = shift_up<TG, OFF>(A[i]);
#pragma unroll
      for (int v = 0; v < V; ++v) Xp[v] = shift_up<TG, OFF>(X[v]);
      if (tg >= OFF) {
#pragma unroll
        for (int v = 0; v < V; ++v) X[v] = fmaf(A[GI_LANE ? 0 : v], Xp[v], X[v]);
#pragma unroll
        for (int i = 0; i < NA; ++i) A[i] *= Ap[i];
      }
      up_level<OFF * 2>(tg, A, X);
    }
  }
  template <int OFF>
  __device__ static __forceinline__ void down_level(int tg, float (&A)[NA], float (&X)[V]) {
    if constexpr (OFF < TG) {
      float An[NA], Xn[V];
#pragma unroll
      for (int i = 0; i < NA; ++i) An[i] = shift_down<TG, OFF>(A[i]);
#pragma unroll
      for (int v = 0; v < V; ++v) Xn[v] = shift_down<TG, OFF>(X[v]);
      if (tg + OFF < TG) {
#pragma unroll
        for (int v = 0; v < V; ++v) X[v] = fmaf(A[GI_LANE ? 0 : v], Xn[v], X[v]);
#pragma unroll
        for (int i = 0; i < NA; ++i) A[i] *= An[i];
      }
      down_level<OFF * 2>(tg, A, X);
    }
  }
};

// ---------------------------------------------------------------------------
// Per-lane gate setup
// ---------------------------------------------------------------------------
template <int GM, int V>
struct GateIdx {
  static constexpr int NA = GM == GATE_LANE ? 1 : V;
  int64_t off[NA];  // element offset of each gate's logit along the channel axis
  float bias[NA];
  __device__ __forceinline__ void init(const float* bias_h, int c0, int nvalid, int D, int r,
                                       int64_t sc) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int c = min(c0 + (GM == GATE_LANE ? 0 : i), D - 1);
      const int j = nvalid > 0 ? c / r : 0;
      off[i] = (int64_t)j * sc;
      bias[i] = bias_h[j];
    }
  }
};

// Raw logits of NS steps as loaded from memory: GATE_LANE keeps one value per
// step (raw bits), the per-channel modes one packed 16-byte vector per step
// (the V channels' logits, gathered for GATE_CHAN).  Step s lies at byte
// offset off0 + s lstb of the buffer (off0 includes the lane's channel offset
// for GATE_CHANVEC); steps at or beyond T and inactive lanes read 0.
template <typename TIO, int GM, int NS>
struct LogitRaw {
  static constexpr int V = Pack<TIO>::V;
  // raw element bits as loaded (16-bit for bf16: widened only where used, so
  // no zero-extension waits for the load right after it is issued)
  using Raw = std::conditional_t<sizeof(TIO) == 2, uint16_t, uint32_t>;
  Raw one[GM == GATE_LANE ? NS : 1];
  uint4 vec[GM == GATE_LANE ? 1 : NS];

  // (steps below Tlo read 0 too).  OPQ: an opaque step index per s, where the
  // compiler would otherwise relate the bounds of consecutive steps and branch
  // over the later loads (the look-back kernels' per-lane windows)
  template <bool OPQ = false>
  __device__ __forceinline__ void load(Rsrc rs, uint32_t off0, uint32_t lstb,
                                           const GateIdx<GM, V>& gi, int t0, int T, bool active,
                                           int nvalid, int Tlo = -2147483647 - 1) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int ts = !OPQ || s == 0 ? t0 + s : (int)opaque((uint32_t)(t0 + s));
      const bool ok = active && ts < T && ts >= Tlo;
      const uint32_t o = GM == GATE_CHAN ? opaque(off0 + s * lstb) : off0 + s * lstb;
      if (GM == GATE_LANE) {
        one[s] = (Raw)bld1<TIO>(rs, ok ? o + (uint32_t)(gi.off[0] * sizeof(TIO)) : kOob);
      } else if (GM == GATE_CHANVEC) {
        vec[s] = bld128(rs, ok ? o : kOob);
      } else {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int v = 0; v < V; ++v)
          Pack<TIO>::put_raw(
              w, v, bld1<TIO>(rs, ok && v < nvalid ? o + (uint32_t)(gi.off[v] * sizeof(TIO)) : kOob));
        vec[s] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }

  // alpha per step and gate; padded steps get alpha = 0 (the identity step)
  template <int NA>
  __device__ __forceinline__ void gates(const GateIdx<GM, V>& gi, int t0, int T, bool active,
                                        bool use_sig, float (&al)[NS][NA]) const {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const bool ok = active && (t0 + s) < T;
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const float raw = GM == GATE_LANE
                              ? __uint_as_float(sizeof(TIO) == 2 ? (uint32_t)one[s] << 16
                                                                 : (uint32_t)one[s])
                              : Pack<TIO>::get(vec[s], i);
        // computed for every lane, then selected: guarding the exp / rcp with
        // a branch makes the compiler wait there for every outstanding
        // memory operation, the previous tile's stores included
        float a = gate_alpha(raw + gi.bias[i], use_sig);
        asm volatile("" : "+v"(a));
        al[s][i] = ok ? a : 0.0f;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <typename TIO, int CL, int L, int NW, bool VEC, int GM>
__global__ void __launch_bounds__(NW * 64)
scan_fwd_kernel(const FwdArgs args) {
  constexpr int V = Pack<TIO>::V;
  constexpr int TG = 64 / CL;
  constexpr int NA = GM == GATE_LANE ? 1 : V;
  constexpr int TW = NW * TG * L;
  constexpr bool GL = GM == GATE_LANE;
  const ScanShape& S = args.sh;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int cl = lane / TG;
  const int tg = lane % TG;

  int bid = blockIdx.x;
  const int slab = bid % S.nslab;
  bid /= S.nslab;
  const int win = bid % args.nwin;
  bid /= args.nwin;
  const int h = bid % S.H;
  const int b = bid / S.H;
  const Window wd = look_back_window(win, S.T, args.P, args.Q, args.K);
  // steps [t_lo, t_hi) are scanned from the inits; [t_st, t_hi) are stored
  int t_lo = wd.lo, t_st = wd.st, t_hi = wd.hi;

  const int c0 = (slab * CL + cl) * V;
  const int nvalid = min(V, S.D - c0);
  const bool active = nvalid > 0;

  constexpr int E = sizeof(TIO);
  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView ov = head_view(args.out, which);
  // (b, h) slices (wave-uniform byte addresses)
  char* obh = reinterpret_cast<char*>(ov.p) + ((int64_t)b * ov.s[0] + (int64_t)hl * ov.s[1]) * E;
  int64_t ost = ov.s[2], osc = ov.s[3];
  if (args.wst != nullptr) {  // warm-up mode: the states of [lo, st), rows t - lo
    t_hi = t_st;
    t_st = t_lo;
    obh = reinterpret_cast<char*>(args.wst) +
          ((((int64_t)b * S.H + h) * args.nwin + win) * args.kw - t_lo) * S.D * E;
    ost = S.D;
    osc = 1;
  }
  const char* ubh = reinterpret_cast<const char*>(args.u.p) +
                    ((int64_t)b * args.u.s[0] + (int64_t)h * args.u.s[1]) * E;
  const char* lbh = reinterpret_cast<const char*>(args.lg.p) +
                    ((int64_t)b * args.lg.s[0] + (int64_t)h * args.lg.s[1]) * E;

  GateIdx<GM, V> gi;
  gi.init(args.bias + h * S.Da, c0, nvalid, S.D, S.r, args.lg.s[3]);

  float carry[V];
  {
    const int64_t ie = (int64_t)b * args.init.s[0] + (int64_t)h * args.init.s[1] +
                       (int64_t)c0 * args.init.s[3];
    const void* ip = reinterpret_cast<const char*>(args.init.p) +
                     ie * (args.init_f32 ? (int64_t)sizeof(float) : (int64_t)sizeof(TIO));
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    if (active) q = ld_init<TIO, VEC>(ip, args.init.s[3], nvalid, args.init_f32 != 0);
#pragma unroll
    for (int v = 0; v < V; ++v) carry[v] = Pack<TIO>::get(q, v);
  }

  __shared__ float lds_a[2][NW][CL][NA];
  __shared__ float4 lds_x[2][NW][CL][V / 4];

  const int ntiles = (t_hi - t_lo + TW - 1) / TW;
  const bool use_sig = S.use_sigmoid != 0;

  // Step t of the tile starting at Tt lies (t - Tt) time strides after the
  // tile's buffer base, so each lane's byte offsets are fixed for the run.
  const int tl0 = (w * TG + tg) * L;
  const uint32_t ustb = (uint32_t)(args.u.s[2] * E), uscb = (uint32_t)(args.u.s[3] * E);
  const uint32_t lstb = (uint32_t)(args.lg.s[2] * E), ostb = (uint32_t)(ost * E);
  const uint32_t oscb = (uint32_t)(osc * E);
  const uint32_t uoff = (uint32_t)tl0 * ustb + (uint32_t)c0 * uscb;
  const uint32_t loff = (uint32_t)tl0 * lstb +
                        (GM == GATE_CHANVEC ? (uint32_t)c0 * (uint32_t)E : 0u);  // r == 1: j == c
  const uint32_t ooff = (uint32_t)tl0 * ostb + (uint32_t)c0 * oscb;

  // the next tile's packed values and raw logits are loaded while the current
  // tile is scanned, so every wavefront keeps loads in flight; alternate tiles
  // use two buffers (with one, the compiler copies the new loads into the
  // body's registers at the end of each tile, waiting there for every
  // outstanding memory operation, the tile's stores included)
  uint4 nu[2][L];
  LogitRaw<TIO, GM, L> nl[2];
  auto load_tile = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int Tt = t_lo + it * TW;
    const int t0 = Tt + tl0;
    const Rsrc ur = make_rsrc(ubh + (int64_t)Tt * args.u.s[2] * E);
#pragma unroll
    for (int s = 0; s < L; ++s)
      nu[buf][s] = bld_vec<TIO, VEC>(ur, uoff + s * ustb, uscb, nvalid, active && (t0 + s) < t_hi);
    nl[buf].load(make_rsrc(lbh + (int64_t)Tt * args.lg.s[2] * E), loff, lstb, gi, t0, t_hi,
                 active, nvalid);
  };

  auto process_tile = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int Tt = t_lo + it * TW;
    const int t0 = Tt + tl0;
    uint4 uq[L];
#pragma unroll
    for (int s = 0; s < L; ++s) uq[s] = nu[buf][s];
    float al[L][NA];
    nl[buf].gates(gi, t0, t_hi, active, use_sig, al);
    // past the end: every lane masked, no memory access
    load_tile(it + 1, std::integral_constant<int, 1 - buf>{});

    // level 1: lane-local fold (padded steps have alpha = 0: the identity)
    float A[NA], X[V];
#pragma unroll
    for (int i = 0; i < NA; ++i) A[i] = 1.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) X[v] = 0.0f;
#pragma unroll
    for (int s = 0; s < L; ++s) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float a = al[s][GL ? 0 : v];
        X[v] = fmaf(a, Pack<TIO>::get(uq[s], v) - X[v], X[v]);
      }
#pragma unroll
      for (int i = 0; i < NA; ++i) A[i] = fmaf(-A[i], al[s][i], A[i]);
    }

    // level 2: inclusive scan over the time-group lanes, then the exclusive prefix
    SegScan<TG, NA, V, GL>::template up_level<1>(tg, A, X);
    float Ae[NA], Xe[V];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const float t = shift_up<TG, 1>(A[i]);
      Ae[i] = tg == 0 ? 1.0f : t;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float t = shift_up<TG, 1>(X[v]);
      Xe[v] = tg == 0 ? 0.0f : t;
    }

    // level 3: wavefront totals through LDS, composed onto the running carry
    const int par = it & 1;
    if (tg == TG - 1) {
#pragma unroll
      for (int i = 0; i < NA; ++i) lds_a[par][w][cl][i] = A[i];
#pragma unroll
      for (int q = 0; q < V / 4; ++q)
        lds_x[par][w][cl][q] = make_float4(X[4 * q], X[4 * q + 1], X[4 * q + 2], X[4 * q + 3]);
    }
    __syncthreads();
    float hw[V];
#pragma unroll
    for (int v = 0; v < V; ++v) hw[v] = carry[v];
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      if (ww == w) {
#pragma unroll
        for (int v = 0; v < V; ++v) hw[v] = carry[v];
      }
      float Aw[NA];
#pragma unroll
      for (int i = 0; i < NA; ++i) Aw[i] = lds_a[par][ww][cl][i];
#pragma unroll
      for (int q = 0; q < V / 4; ++q) {
        const float4 x4 = lds_x[par][ww][cl][q];
        carry[4 * q + 0] = fmaf(Aw[GL ? 0 : 4 * q + 0], carry[4 * q + 0], x4.x);
        carry[4 * q + 1] = fmaf(Aw[GL ? 0 : 4 * q + 1], carry[4 * q + 1], x4.y);
        carry[4 * q + 2] = fmaf(Aw[GL ? 0 : 4 * q + 2], carry[4 * q + 2], x4.z);
        carry[4 * q + 3] = fmaf(Aw[GL ? 0 : 4 * q + 3], carry[4 * q + 3], x4.w);
      }
    }

    // re-run the lane's steps from its exact carry-in and store
    reload_barrier(uq);
    const Rsrc orr = make_rsrc(obh + (int64_t)Tt * ost * E);
    float hv[V];
#pragma unroll
    for (int v = 0; v < V; ++v) hv[v] = fmaf(Ae[GL ? 0 : v], hw[v], Xe[v]);
#pragma unroll
    for (int s = 0; s < L; ++s) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float a = al[s][GL ? 0 : v];
        hv[v] = fmaf(a, Pack<TIO>::get(uq[s], v) - hv[v], hv[v]);
      }
      bst_vec<TIO, VEC, GM == GATE_CHANVEC ? kStStream : kStNormal>(
          orr, ooff + s * ostb, oscb, nvalid, active && (t0 + s) >= t_st && (t0 + s) < t_hi, hv);
    }
  };

  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  load_tile(0, B0{});
  for (int it = 0; it < ntiles; it += 2) {
    process_tile(it, B0{});
    if (it + 1 < ntiles) process_tile(it + 1, B1{});
  }
}

// ---------------------------------------------------------------------------
// Forward with chained chunk states (one pass over HBM, parallel over T)
// ---------------------------------------------------------------------------
// Each workgroup scans one chunk of TW = NW * TG * L steps of one (b, head,
// channel slab) sequence, holding all of the chunk's values and logits in
// registers, so the grid grows with T instead of one workgroup walking all of
// T (the tile kernel above).  The state entering chunk c is the state leaving
// chunk c - 1: that chunk's workgroup publishes it as soon as it has its own
// entering state, so only this short hand-off is sequential.
//   * Publication: one 64-bit word per channel, fp32 state in the low half and
//     a nonzero tag in the high half, stored and polled with device-scope
//     atomics (coherent across the XCDs' L2s).  A word is either absent or
//     whole, so no fence has to order it against other memory.
//   * Order: a workgroup takes a ticket from a counter when it starts, and
//     tickets map chunk-major onto (sequence, chunk).  The chunk a workgroup
//     waits for holds an earlier ticket, so it is already running and itself
//     waits only on earlier tickets: every wait ends.  A wait is still bounded
//     (ChainCtl::spin_max polls, by default kChainSpinMax, about a second; a
//     chunk's wait is normally a few microseconds); past the bound the kernel
//     reports error 1 (chain_report), goes on with a zero state and exits
//     normally.
//   * Zero invariant: the reader of a word clears it, the last chunk of a
//     sequence publishes nothing, and the workgroup that draws the last ticket
//     resets the counter, so the workspace is all zeros again when the kernel
//     ends and a launch needs no clearing pass (nor a memset in a captured
//     graph).  A reader that gives up swaps an "abandoned" marker into the
//     empty word (compare-and-swap); the publisher's own compare-and-swap
//     then fails on it, and the publisher clears the word instead: a late
//     carry is never left behind for a later launch to read.
// The chunk composes its wavefront totals onto the entering state in the
// tile kernel's order, so with the same launch shape (CL, L, NW) both kernels
// give bitwise equal outputs.
struct ChainArgs {
  uint32_t* ticket;           // chunk ticket counter (0 between launches)
  uint32_t* err;              // 1: a wait ran past its bound; 2: counter not 0 at launch
  unsigned long long* words;  // (nseq, nchunk - 1, CL * V) tagged states (0 between launches)
  int nseq;                   // B * H * nslab
  int nchunk;                 // chunks per sequence
  ChainCtl ctl;
};
constexpr int kChainSpinMax = 1 << 20;
constexpr unsigned long long kChainTag = 1ull << 32;        // a published carry
constexpr unsigned long long kChainAbandoned = 2ull << 32;  // its reader gave up

// Record error `code` in the workspace header and the host's mailbox.
__device__ __forceinline__ void chain_report(uint32_t* err, const ChainCtl& ctl, uint32_t code) {
  __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (ctl.host_err != nullptr)
    __hip_atomic_store(ctl.host_err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The carry published in *pw, waited for at most ctl.spin_max polls; the word
// is left zero.  Past the bound: an abandoned marker replaces the empty word
// (unless the carry landed meanwhile), error 1 is reported and 0 returned.
__device__ __forceinline__ float chain_take(unsigned long long* pw, uint32_t* err,
                                            const ChainCtl& ctl) {
  unsigned long long wv = 0;
  for (int spin = 0;; ++spin) {
    wv = __hip_atomic_load(pw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((wv >> 32) == (kChainTag >> 32)) break;
    if (spin >= ctl.spin_max) {
      unsigned long long expect = 0;
      if (__hip_atomic_compare_exchange_strong(pw, &expect, kChainAbandoned, __ATOMIC_RELAXED,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        chain_report(err, ctl, 1u);
        return 0.0f;
      }
      if ((expect >> 32) != (kChainTag >> 32)) {
        // a marker left by an earlier failed launch: the workspace was not
        // zeroed after that error
        chain_report(err, ctl, 2u);
        __hip_atomic_store(pw, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return 0.0f;
      }
      wv = expect;  // the carry landed between the last poll and the swap
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __hip_atomic_store(pw, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __uint_as_float((uint32_t)wv);
}

// Publish carry p into the empty word *pw.  Returns the word's previous
// value: non-zero (the abandoned marker) means the reader gave up, and the
// caller must then clear the word with chain_clear_abandoned -- late, so the
// atomic's round trip is not waited for on the chain's path.
__device__ __forceinline__ unsigned long long chain_publish(unsigned long long* pw, float p,
                                                            const ChainCtl& ctl) {
  if (ctl.no_publish) return 0ull;
  unsigned long long expect = 0;
  __hip_atomic_compare_exchange_strong(pw, &expect, kChainTag | __float_as_uint(p),
                                       __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return expect;
}

__device__ __forceinline__ void chain_clear_abandoned(unsigned long long* pw,
                                                      unsigned long long prev) {
  // The empty asm keeps the whole returned value live up to here: otherwise
  // the compiler tests it right after the compare-and-swap and waits for the
  // atomic's round trip before the workgroup barrier that follows it.
  asm volatile("" : "+v"(prev));
  if (prev != 0ull) __hip_atomic_store(pw, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename TIO, int CL, int L, int NW, bool VEC, int GM>
__global__ void __launch_bounds__(NW * 64)
scan_fwd_chain_kernel(const FwdArgs args, const ChainArgs ch) {
  constexpr int V = Pack<TIO>::V;
  constexpr int TG = 64 / CL;
  constexpr int NA = GM == GATE_LANE ? 1 : V;
  constexpr int TW = NW * TG * L;
  constexpr int NCH = CL * V;  // channels per slab: one per lane of wavefront 0
  static_assert(NCH <= 64, "a slab's channels must fit one wavefront");
  constexpr bool GL = GM == GATE_LANE;
  const ScanShape& S = args.sh;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int cl = lane / TG;
  const int tg = lane % TG;

  __shared__ int lds_ticket;
  __shared__ float lds_a[NW][CL][NA];
  __shared__ float4 lds_x[NW][CL][V / 4];
  __shared__ float lds_c[NCH];  // the state entering the chunk

  if (threadIdx.x == 0) {
    const uint32_t t =
        __hip_atomic_fetch_add(ch.ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // every other workgroup has drawn its ticket: leave the counter at 0
    if (t == gridDim.x - 1)
      __hip_atomic_store(ch.ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_ticket = (int)t;
  }
  __syncthreads();
  const int ticket = lds_ticket;
  // a counter that was not zero at the launch (a workspace not zeroed before
  // its first use) hands out tickets past the grid: such a workgroup only
  // reports it (the waits of the others end at their bound)
  if (ticket >= (int)gridDim.x) {
    if (threadIdx.x == 0) chain_report(ch.err, ch.ctl, 2u);
    return;
  }
  const int seq = ticket % ch.nseq;
  const int chunk = ticket / ch.nseq;
  const int slab = seq % S.nslab;
  const int h = (seq / S.nslab) % S.H;
  const int b = seq / S.nslab / S.H;
  const int T = S.T;
  const int Tt = chunk * TW;  // the chunk's first step

  const int c0 = (slab * CL + cl) * V;
  const int nvalid = min(V, S.D - c0);
  const bool active = nvalid > 0;

  constexpr int E = sizeof(TIO);
  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView ov = head_view(args.out, which);
  const char* obh = reinterpret_cast<const char*>(ov.p) +
                    ((int64_t)b * ov.s[0] + (int64_t)hl * ov.s[1]) * E;
  const char* ubh = reinterpret_cast<const char*>(args.u.p) +
                    ((int64_t)b * args.u.s[0] + (int64_t)h * args.u.s[1]) * E;
  const char* lbh = reinterpret_cast<const char*>(args.lg.p) +
                    ((int64_t)b * args.lg.s[0] + (int64_t)h * args.lg.s[1]) * E;

  GateIdx<GM, V> gi;
  gi.init(args.bias + h * S.Da, c0, nvalid, S.D, S.r, args.lg.s[3]);
  const bool use_sig = S.use_sigmoid != 0;

  const int tl0 = (w * TG + tg) * L;
  const int t0 = Tt + tl0;
  const uint32_t ustb = (uint32_t)(args.u.s[2] * E), uscb = (uint32_t)(args.u.s[3] * E);
  const uint32_t lstb = (uint32_t)(args.lg.s[2] * E), ostb = (uint32_t)(ov.s[2] * E);
  const uint32_t oscb = (uint32_t)(ov.s[3] * E);
  const uint32_t uoff = (uint32_t)tl0 * ustb + (uint32_t)c0 * uscb;
  const uint32_t loff = (uint32_t)tl0 * lstb +
                        (GM == GATE_CHANVEC ? (uint32_t)c0 * (uint32_t)E : 0u);  // r == 1: j == c
  const uint32_t ooff = (uint32_t)tl0 * ostb + (uint32_t)c0 * oscb;

  // the whole chunk is loaded at once: L vectors and logits per lane in flight
  uint4 uq[L];
  LogitRaw<TIO, GM, L> lr;
  {
    const Rsrc ur = make_rsrc(ubh + (int64_t)Tt * args.u.s[2] * E);
#pragma unroll
    for (int s = 0; s < L; ++s)
      uq[s] = bld_vec<TIO, VEC>(ur, uoff + s * ustb, uscb, nvalid, active && (t0 + s) < T);
    lr.load(make_rsrc(lbh + (int64_t)Tt * args.lg.s[2] * E), loff, lstb, gi, t0, T, active,
            nvalid);
  }
  // chunk 0 enters from the inits (lanes of wavefront 0's first time group
  // hand them to the chain step through lds_c)
  if (chunk == 0 && w == 0 && tg == 0) {
    const int64_t ie = (int64_t)b * args.init.s[0] + (int64_t)h * args.init.s[1] +
                       (int64_t)c0 * args.init.s[3];
    const void* ip = reinterpret_cast<const char*>(args.init.p) +
                     ie * (args.init_f32 ? (int64_t)sizeof(float) : (int64_t)sizeof(TIO));
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    if (active) q = ld_init<TIO, VEC>(ip, args.init.s[3], nvalid, args.init_f32 != 0);
#pragma unroll
    for (int v = 0; v < V; ++v) lds_c[cl * V + v] = Pack<TIO>::get(q, v);
  }

  float al[L][NA];
  lr.gates(gi, t0, T, active, use_sig, al);

  // level 1: lane-local fold (padded steps have alpha = 0: the identity)
  float A[NA], X[V];
#pragma unroll
  for (int i = 0; i < NA; ++i) A[i] = 1.0f;
#pragma unroll
  for (int v = 0; v < V; ++v) X[v] = 0.0f;
#pragma unroll
  for (int s = 0; s < L; ++s) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float a = al[s][GL ? 0 : v];
      X[v] = fmaf(a, Pack<TIO>::get(uq[s], v) - X[v], X[v]);
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) A[i] = fmaf(-A[i], al[s][i], A[i]);
  }

  // level 2: inclusive scan over the time-group lanes, then the exclusive prefix
  SegScan<TG, NA, V, GL>::template up_level<1>(tg, A, X);
  float Ae[NA], Xe[V];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const float t = shift_up<TG, 1>(A[i]);
    Ae[i] = tg == 0 ? 1.0f : t;
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const float t = shift_up<TG, 1>(X[v]);
    Xe[v] = tg == 0 ? 0.0f : t;
  }

  // level 3: wavefront totals through LDS
  if (tg == TG - 1) {
#pragma unroll
    for (int i = 0; i < NA; ++i) lds_a[w][cl][i] = A[i];
#pragma unroll
    for (int q = 0; q < V / 4; ++q)
      lds_x[w][cl][q] = make_float4(X[4 * q], X[4 * q + 1], X[4 * q + 2], X[4 * q + 3]);
  }
  __syncthreads();

  // the chain step: wavefront 0, lane j = slab channel j, takes the entering
  // state, publishes the leaving one and hands the entering one to the others
  // the published word's previous value (wavefront 0, chunks before the
  // last); its address is recomputed at the end, so only the value stays live
  unsigned long long pub_prev = 0ull;
  if (w == 0 && lane < NCH) {
    const int j = lane;
    float cin;
    if (chunk == 0) {
      cin = lds_c[j];
    } else {
      cin = chain_take(ch.words + ((int64_t)seq * (ch.nchunk - 1) + chunk - 1) * NCH + j, ch.err,
                       ch.ctl);
    }
    if (chunk + 1 < ch.nchunk) {
      const float* xa = reinterpret_cast<const float*>(&lds_x[0][0][0]);
      float p = cin;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww)
        p = fmaf(lds_a[ww][j / V][GL ? 0 : j % V], p, xa[ww * NCH + j]);
      pub_prev =
          chain_publish(ch.words + ((int64_t)seq * (ch.nchunk - 1) + chunk) * NCH + j, p, ch.ctl);
    }
    lds_c[j] = cin;
  }
  __syncthreads();

  // the state entering this wavefront: the chunk's entering state composed
  // with the totals of the wavefronts before it
  float hw[V];
#pragma unroll
  for (int v = 0; v < V; ++v) hw[v] = lds_c[cl * V + v];
#pragma unroll
  for (int ww = 0; ww < NW - 1; ++ww) {
    if (ww < w) {
      float Aw[NA];
#pragma unroll
      for (int i = 0; i < NA; ++i) Aw[i] = lds_a[ww][cl][i];
#pragma unroll
      for (int q = 0; q < V / 4; ++q) {
        const float4 x4 = lds_x[ww][cl][q];
        hw[4 * q + 0] = fmaf(Aw[GL ? 0 : 4 * q + 0], hw[4 * q + 0], x4.x);
        hw[4 * q + 1] = fmaf(Aw[GL ? 0 : 4 * q + 1], hw[4 * q + 1], x4.y);
        hw[4 * q + 2] = fmaf(Aw[GL ? 0 : 4 * q + 2], hw[4 * q + 2], x4.z);
        hw[4 * q + 3] = fmaf(Aw[GL ? 0 : 4 * q + 3], hw[4 * q + 3], x4.w);
      }
    }
  }

  // re-run the lane's steps from its exact carry-in and store
  reload_barrier(uq);
  const Rsrc orr = make_rsrc(obh + (int64_t)Tt * ov.s[2] * E);
  float hv[V];
#pragma unroll
  for (int v = 0; v < V; ++v) hv[v] = fmaf(Ae[GL ? 0 : v], hw[v], Xe[v]);
#pragma unroll
  for (int s = 0; s < L; ++s) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float a = al[s][GL ? 0 : v];
      hv[v] = fmaf(a, Pack<TIO>::get(uq[s], v) - hv[v], hv[v]);
    }
    bst_vec<TIO, VEC, GM == GATE_CHANVEC ? kStStream : kStNormal>(
        orr, ooff + s * ostb, oscb, nvalid, active && (t0 + s) < T, hv);
  }
  if (w == 0 && lane < NCH && chunk + 1 < ch.nchunk)
    chain_clear_abandoned(ch.words + ((int64_t)seq * (ch.nchunk - 1) + chunk) * NCH + lane,
                          pub_prev);
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
// GATE_LANE: r % V == 0; the gate group spans r / V adjacent channel lanes and
//   dalpha is summed across them with lane shuffles; at most kMaxLaneGroups
//   groups.
// GATE_CHAN / GATE_CHANVEC: V % r == 0; each lane holds V / r whole groups.
constexpr int kMaxLaneGroups = 16;

// CHAIN: one tile per chunk (chunk_steps == TW), chunks taken last to first in
// ticket order, each entering with the gradient carry that the workgroup of
// the chunk after it publishes (the chained forward's hand-off, run in
// reverse).  The carry is composed from the same wavefront totals in the same
// order as the tile loop's, so every output but the dbias partials (one per
// chunk instead of one per sequence) is bitwise that of the unchunked kernel
// with the same launch shape.  Deadlock-free for the chained forward's
// reason: a workgroup waits only for a smaller ticket, drawn by a workgroup
// that is already running.
template <typename TIO, int CL, int L, int NW, bool VEC, int GM, bool LB, bool CHAIN = false>
__global__ void __launch_bounds__(NW * 64)
scan_bwd_kernel(const BwdArgs args) {
  constexpr int V = Pack<TIO>::V;
  constexpr int TG = 64 / CL;
  constexpr int NA = GM == GATE_LANE ? 1 : V;
  constexpr int TW = NW * TG * L;
  constexpr int NT = NW * 64;
  constexpr int NCH = CL * V;  // chained mode: one carry word per channel slot
  constexpr bool GL = GM == GATE_LANE;
  static_assert(!(CHAIN && LB), "the chained backward runs the full recurrence");
  static_assert(!CHAIN || NCH <= NT, "the chain step takes one thread per channel slot");
  const ScanShape& S = args.sh;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int cl = lane / TG;
  const int tg = lane % TG;

  // one workgroup per (b, head, time chunk): every gate group of the head inside
  int bh = blockIdx.x / args.nchunk, chunk = blockIdx.x % args.nchunk;
  __shared__ int lds_ticket;
  __shared__ float lds_cin[CHAIN ? NCH : 1];  // the carry entering the chunk
  if constexpr (CHAIN) {
    if (threadIdx.x == 0) {
      const uint32_t t =
          __hip_atomic_fetch_add(args.ch_ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // every other workgroup has drawn its ticket: leave the counter at 0
      if (t == gridDim.x - 1)
        __hip_atomic_store(args.ch_ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      lds_ticket = (int)t;
    }
    __syncthreads();
    const int ticket = lds_ticket;
    // a counter that was not zero at the launch hands out tickets past the
    // grid: such a workgroup only reports it (the others' waits end at their
    // bound)
    if (ticket >= (int)gridDim.x) {
      if (threadIdx.x == 0) chain_report(args.ch_err, args.ch_ctl, 2u);
      return;
    }
    const int nseq = S.B * S.H;
    bh = ticket % nseq;
    chunk = args.nchunk - 1 - ticket / nseq;
  }
  const int h = bh % S.H;
  const int b = bh / S.H;

  const int c0 = cl * V;
  const int nvalid = min(V, S.D - c0);
  const bool active = nvalid > 0;

  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView hvw = head_view(args.h, which), gvw = head_view(args.gy, which);
  const int64_t hs[4] = {hvw.s[0], hvw.s[1], hvw.s[2], hvw.s[3]};
  const int64_t gs[4] = {gvw.s[0], gvw.s[1], gvw.s[2], gvw.s[3]};
  constexpr int E = sizeof(TIO);
  // (b, h) slices (wave-uniform byte addresses)
  const char* hbh = reinterpret_cast<const char*>(hvw.p) + ((int64_t)b * hs[0] + (int64_t)hl * hs[1]) * E;
  const char* gbh = reinterpret_cast<const char*>(gvw.p) + ((int64_t)b * gs[0] + (int64_t)hl * gs[1]) * E;
  const char* ubh = reinterpret_cast<const char*>(args.u.p) +
                    ((int64_t)b * args.u.s[0] + (int64_t)h * args.u.s[1]) * E;
  const char* lbh = reinterpret_cast<const char*>(args.lg.p) +
                    ((int64_t)b * args.lg.s[0] + (int64_t)h * args.lg.s[1]) * E;
  const char* dubh = reinterpret_cast<const char*>(args.du.p) +
                     ((int64_t)b * args.du.s[0] + (int64_t)h * args.du.s[1]) * E;
  const char* dlbh = reinterpret_cast<const char*>(args.dlg.p) +
                     ((int64_t)b * args.dlg.s[0] + (int64_t)h * args.dlg.s[1]) * E;
  const bool init_f32 = args.init_f32 != 0;
  const int64_t EI = init_f32 ? (int64_t)sizeof(float) : (int64_t)E;  // bytes per init element
  const Rsrc irs = make_rsrc(reinterpret_cast<const char*>(args.init.p) +
                             ((int64_t)b * args.init.s[0] + (int64_t)h * args.init.s[1]) * EI);

  GateIdx<GM, V> gi;
  gi.init(args.bias + h * S.Da, c0, nvalid, S.D, S.r, args.lg.s[3]);

  const bool use_sig = S.use_sigmoid != 0;
  const int gl_lanes = GL ? S.r / V : 1;           // lanes per gate group (GATE_LANE)

  // wavefront totals, double-buffered by tile parity: with one barrier per
  // tile (GATE_CHAN*) a wavefront may write the next tile's totals while
  // another still reads this tile's
  __shared__ float lds_ba[2][NW][CL][NA];
  __shared__ float4 lds_bx[2][NW][CL][V / 4];
  __shared__ float lds_red[NT][GL ? 1 : V];

  float gcarry[V];  // g at the first step after the current tile
#pragma unroll
  for (int v = 0; v < V; ++v) gcarry[v] = 0.0f;
  if (!LB && !CHAIN && args.nchunk > 1) {
    const float* cp = args.carry + ((int64_t)bh * args.nchunk + chunk) * S.D + c0;
#pragma unroll
    for (int v = 0; v < V; ++v) gcarry[v] = v < nvalid ? cp[v] : 0.0f;
  }
  // dbias accumulators: GATE_CHAN* keeps one per channel slot; GATE_LANE one
  // in the last lane of each gate group (the lane that emits its dlogits)
  float dacc[GL ? 1 : V];
#pragma unroll
  for (int k = 0; k < (GL ? 1 : V); ++k) dacc[k] = 0.0f;

  // tiles it_lo..it_hi of TW steps from t_base; steps < t_hi exist, upstream
  // gradients and owned outputs start at t_st
  int t_base, t_st, t_hi, it_lo, it_hi;
  if (LB) {
    const Window wd = look_back_window(chunk, S.T, args.P, args.Q, args.K);
    t_base = wd.lo;
    t_st = wd.st;
    t_hi = wd.hi;
    it_lo = 0;
    it_hi = (t_hi - t_base + TW - 1) / TW - 1;  // -1: empty window
  } else {
    t_base = 0;
    t_st = 0;
    t_hi = S.T;
    const int ntiles = (S.T + TW - 1) / TW;
    const int tiles_pc = args.chunk_steps / TW;
    it_lo = chunk * tiles_pc;
    it_hi = min(ntiles, it_lo + tiles_pc) - 1;
  }
  // this window's rows of the look-back workspaces (row t - t_base)
  const int64_t wrow0 = LB ? ((int64_t)bh * args.nchunk + chunk) * args.kw : 0;
  const char* wsbh = LB ? reinterpret_cast<const char*>(args.wst) + wrow0 * S.D * E : nullptr;
  const char* wdubh = LB ? reinterpret_cast<const char*>(args.wdu + wrow0 * S.D) : nullptr;
  const char* wdlbh = LB ? reinterpret_cast<const char*>(args.wdl + wrow0 * S.Da) : nullptr;

  // Step t of the tile starting at Tt lies (t - Tt) time strides after the
  // tile's buffer base (the saved state h_{t-1} after the base at Tt - 1), so
  // each lane's byte offsets are fixed for the run.
  const int tl0 = (w * TG + tg) * L;
  const uint32_t ustb = (uint32_t)(args.u.s[2] * E), uscb = (uint32_t)(args.u.s[3] * E);
  const uint32_t gstb = (uint32_t)(gs[2] * E), gscb = (uint32_t)(gs[3] * E);
  const uint32_t hstb = (uint32_t)(hs[2] * E), hscb = (uint32_t)(hs[3] * E);
  const uint32_t lstb = (uint32_t)(args.lg.s[2] * E);
  const uint32_t dustb = (uint32_t)(args.du.s[2] * E), duscb = (uint32_t)(args.du.s[3] * E);
  const uint32_t dlstb = (uint32_t)(args.dlg.s[2] * E), dlscb = (uint32_t)(args.dlg.s[3] * E);
  const uint32_t iscb = (uint32_t)(args.init.s[3] * EI);
  const uint32_t wstb = (uint32_t)(S.D * E), wdustb = (uint32_t)(S.D * 4), wdlstb = (uint32_t)(S.Da * 4);
  const uint32_t uoff = (uint32_t)tl0 * ustb + (uint32_t)c0 * uscb;
  const uint32_t goff = (uint32_t)tl0 * gstb + (uint32_t)c0 * gscb;
  const uint32_t hoff = (uint32_t)tl0 * hstb + (uint32_t)c0 * hscb;
  const uint32_t woff = (uint32_t)tl0 * wstb + (uint32_t)c0 * E;
  const uint32_t ioff = (uint32_t)c0 * iscb;
  const uint32_t loff = (uint32_t)tl0 * lstb +
                        (GM == GATE_CHANVEC ? (uint32_t)c0 * (uint32_t)E : 0u);  // r == 1: j == c
  const uint32_t duoff = (uint32_t)tl0 * dustb + (uint32_t)c0 * duscb;
  const uint32_t wduoff = (uint32_t)tl0 * wdustb + (uint32_t)c0 * 4;

  // The packed u, gy and raw logits of an earlier tile, and the state entering
  // each lane's first step, are loaded while the current tile is processed, so
  // each wavefront keeps its loads in flight across the tile's barriers and
  // stores: PD tiles ahead (two when a lane's steps are few enough for the
  // registers, else one).  Where the registers allow (NB = 2), alternate
  // tiles use two buffers: with one buffer the compiler copies the new loads
  // into the body's registers at the end of each tile, waiting there for
  // every outstanding memory operation, the tile's own stores included.  The state h_{t0-1} entering a lane is the saved
  // forward output of the step before (the inits at t = t_base; the warm-up
  // states before t_st in a look-back window); the lane recomputes its other
  // L - 1 states h_t = h_{t-1} + alpha_t (u_t - h_{t-1}) itself, rounded to
  // the I/O dtype as the forward stores them.  A tile before it_lo is all
  // masked: no memory access.
  // (The chained mode runs one tile: no prefetch, one buffer.)
  constexpr int PD = CHAIN || L > 2 ? 1 : 2;
  constexpr int NB = !CHAIN && (PD == 2 || (GL && L <= 4)) ? 2 : 1;
  // the state entering the lane comes from one of three masked loads, kept
  // apart until the tile uses it (merging them at once would wait for the
  // loads just issued)
  uint4 nu[NB][L], ng[NB][L], nh0[NB], nw0[LB ? NB : 1];
  // The inits of this lane's channels are read once, here, raw (16-byte
  // vectors; fp32 inits with bf16 I/O are two), and converted by selects in
  // the tile whose lane starts at t_base: a branch on the dtype inside the
  // tile loop would make the compiler wait for the prefetched loads at its
  // join.  Only that lane (tl0 == 0 of tile 0) needs them.
  uint4 init_a = make_uint4(0u, 0u, 0u, 0u), init_b = make_uint4(0u, 0u, 0u, 0u);
  {
    const bool need = active && tl0 == 0 && it_lo == 0;
    if constexpr (VEC) {
      init_a = bld128(irs, need ? ioff : kOob);
      if constexpr (sizeof(TIO) == 2) init_b = bld128(irs, need && init_f32 ? ioff + 16u : kOob);
    } else {
      init_a = bld_init<TIO, false>(irs, ioff, iscb, nvalid, need, init_f32);
    }
  }
  auto init_vec = [&]() -> uint4 {
    if constexpr (VEC && sizeof(TIO) == 2) {
      const float x[8] = {__uint_as_float(init_a.x), __uint_as_float(init_a.y),
                          __uint_as_float(init_a.z), __uint_as_float(init_a.w),
                          __uint_as_float(init_b.x), __uint_as_float(init_b.y),
                          __uint_as_float(init_b.z), __uint_as_float(init_b.w)};
      const uint4 cv = Pack<bf16_t>::pack(x);
      return make_uint4(init_f32 ? cv.x : init_a.x, init_f32 ? cv.y : init_a.y,
                        init_f32 ? cv.z : init_a.z, init_f32 ? cv.w : init_a.w);
    }
    return init_a;
  };
  LogitRaw<TIO, GM, L + 1> nl[NB];
  auto load_tile = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int Tt = t_base + it * TW;
    const int t0 = Tt + tl0;
    const bool tile_ok = active && it >= it_lo;
    const Rsrc ur = make_rsrc(ubh + (int64_t)Tt * args.u.s[2] * E);
    const Rsrc gr = make_rsrc(gbh + (int64_t)Tt * gs[2] * E);
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const int t = t0 + s;
      const bool ok = tile_ok && t < t_hi;
      nu[buf][s] = bld_vec<TIO, VEC, kLdStream>(ur, uoff + s * ustb, uscb, nvalid, ok);
      ng[buf][s] = bld_vec<TIO, VEC, kLdStream>(gr, goff + s * gstb, gscb, nvalid,
                                                ok && (!LB || t >= t_st));
    }
    // exactly one of the sources is unmasked; the others read 0
    const bool ok0 = tile_ok && t0 < t_hi;
    const bool from_init = ok0 && t0 == t_base;
    const bool from_wst = LB && ok0 && !from_init && t0 - 1 < t_st;
    const bool from_h = ok0 && !from_init && !from_wst;
    nh0[buf] = bld_vec<TIO, VEC, kLdStream>(make_rsrc(hbh + (int64_t)(Tt - 1) * hs[2] * E), hoff,
                                            hscb, nvalid, from_h);
    if constexpr (LB)
      nw0[buf] = bld_vec<TIO, VEC>(make_rsrc(wsbh + (int64_t)(Tt - 1 - t_base) * S.D * E), woff,
                                   E, nvalid, from_wst);
    nl[buf].load(make_rsrc(lbh + (int64_t)Tt * args.lg.s[2] * E), loff, lstb, gi, t0, t_hi,
                 tile_ok, nvalid);
  };

  // GATE_LANE: this lane's gate group j = cl / gl_lanes spans channel lanes
  // [seg0, seg0 + gl_lanes); its last lane emits the group's dlogits
  const int gj = GL ? cl / gl_lanes : 0;
  const int seg0 = gj * gl_lanes;
  const bool glead = GL && active && cl == seg0 + gl_lanes - 1;
  float dinit_v[V];  // (1 - alpha) g at each tile's first lane step; the last tile's is kept
#pragma unroll
  for (int v = 0; v < V; ++v) dinit_v[v] = 0.0f;

  // the chained mode's published word's previous value (the word is cleared at
  // the end if its reader gave up; its address is recomputed there)
  unsigned long long pub_prev = 0ull;
  auto process_tile = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int T0 = t_base + it * TW;
    const int t0 = T0 + tl0;

    uint4 uq[L], gq[L], hq[L];
#pragma unroll
    for (int s = 0; s < L; ++s) {
      uq[s] = nu[buf][s];
      gq[s] = ng[buf][s];
    }
    {
      uint4 q = nh0[buf];
      // the lane that starts at t_base enters from the inits (its h load was
      // masked); every other lane ORs zeros
      const bool at_init = active && t0 == t_base && t0 < t_hi;
      const uint4 iv = init_vec();  // loop-invariant: formed once, before the tile loop
      const uint4 qi = at_init ? iv : make_uint4(0u, 0u, 0u, 0u);
      q = make_uint4(q.x | qi.x, q.y | qi.y, q.z | qi.z, q.w | qi.w);
      if constexpr (LB) {
        const uint4 qw = nw0[buf];
        q = make_uint4(q.x | qw.x, q.y | qw.y, q.z | qw.z, q.w | qw.w);
      }
      hq[0] = q;
    }
    float al[L + 1][NA];
    nl[buf].gates(gi, t0, t_hi, active, use_sig, al);
    if constexpr (!CHAIN)
      load_tile(it - PD, std::integral_constant<int, PD == 1 && NB == 2 ? 1 - buf : buf>{});
    // h_{t-1} of the lane's later steps (padded steps have alpha = 0)
#pragma unroll
    for (int s = 1; s < L; ++s) {
      float hv[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float hp_ = Pack<TIO>::get(hq[s - 1], v);
        hv[v] = fmaf(al[s - 1][GL ? 0 : v], Pack<TIO>::get(uq[s - 1], v) - hp_, hp_);
      }
      hq[s] = Pack<TIO>::pack(hv);
    }

    // ---- reverse scan: g_t = gy_t + (1 - alpha_{t+1}) g_{t+1}
    // dk[s][i]: decay carrying g_{t+1} into g_t, zero for the last step of the
    // sequence.  Steps at or past t_hi (padding) need no guard: their gy reads
    // 0, and the step before the first of them has decay 0, so they leave the
    // lane's map as if skipped.
    float dk[L][NA];
#pragma unroll
    for (int s = 0; s < L; ++s)
#pragma unroll
      for (int i = 0; i < NA; ++i) dk[s][i] = t0 + s + 1 < t_hi ? 1.0f - al[s + 1][i] : 0.0f;
    float gin[V];
    {
      float A[NA], G[V];
#pragma unroll
      for (int i = 0; i < NA; ++i) A[i] = dk[L - 1][i];
#pragma unroll
      for (int v = 0; v < V; ++v) G[v] = Pack<TIO>::get(gq[L - 1], v);
#pragma unroll
      for (int s = L - 2; s >= 0; --s) {
#pragma unroll
        for (int v = 0; v < V; ++v) G[v] = fmaf(dk[s][GL ? 0 : v], G[v], Pack<TIO>::get(gq[s], v));
#pragma unroll
        for (int i = 0; i < NA; ++i) A[i] *= dk[s][i];
      }
      SegScan<TG, NA, V, GL>::template down_level<1>(tg, A, G);
      float Ae[NA], Ge[V];
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const float t = shift_down<TG, 1>(A[i]);
        Ae[i] = tg == TG - 1 ? 1.0f : t;
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float t = shift_down<TG, 1>(G[v]);
        Ge[v] = tg == TG - 1 ? 0.0f : t;
      }
      const int par = it & 1;
      if (tg == 0) {
#pragma unroll
        for (int i = 0; i < NA; ++i) lds_ba[par][w][cl][i] = A[i];
#pragma unroll
        for (int q = 0; q < V / 4; ++q)
          lds_bx[par][w][cl][q] = make_float4(G[4 * q], G[4 * q + 1], G[4 * q + 2], G[4 * q + 3]);
      }
      __syncthreads();  // (2)
      if constexpr (CHAIN) {
        // the chain step: thread j (channel slot j) takes the carry entering
        // the chunk from the chunk after it, publishes the carry leaving it
        // for the chunk before, and hands the entering one to every lane
        if (threadIdx.x < NCH) {
          const int j = threadIdx.x, jl = j / V, jv = j % V;
          float cin = 0.0f;
          if (j < S.D) {
            const int64_t row = (int64_t)bh * (args.nchunk - 1);
            if (chunk + 1 < args.nchunk)
              cin = chain_take(args.ch_words + (row + chunk) * NCH + j, args.ch_err,
                               args.ch_ctl);
            if (chunk > 0) {
              // the tile loop's composition, last wavefront first
              const float* xb = reinterpret_cast<const float*>(&lds_bx[par][0][0][0]);
              float p = cin;
#pragma unroll
              for (int ww = NW - 1; ww >= 0; --ww)
                p = fmaf(lds_ba[par][ww][jl][GL ? 0 : jv], p, xb[(ww * CL + jl) * V + jv]);
              pub_prev = chain_publish(args.ch_words + (row + chunk - 1) * NCH + j, p,
                                       args.ch_ctl);
            }
          }
          lds_cin[j] = cin;
        }
        __syncthreads();
#pragma unroll
        for (int v = 0; v < V; ++v) gcarry[v] = lds_cin[c0 + v];
      }
      float gw[V];
#pragma unroll
      for (int v = 0; v < V; ++v) gw[v] = gcarry[v];
#pragma unroll
      for (int ww = NW - 1; ww >= 0; --ww) {
        if (ww == w) {
#pragma unroll
          for (int v = 0; v < V; ++v) gw[v] = gcarry[v];
        }
        float Aw[NA];
#pragma unroll
        for (int i = 0; i < NA; ++i) Aw[i] = lds_ba[par][ww][cl][i];
#pragma unroll
        for (int q = 0; q < V / 4; ++q) {
          const float4 x4 = lds_bx[par][ww][cl][q];
          gcarry[4 * q + 0] = fmaf(Aw[GL ? 0 : 4 * q + 0], gcarry[4 * q + 0], x4.x);
          gcarry[4 * q + 1] = fmaf(Aw[GL ? 0 : 4 * q + 1], gcarry[4 * q + 1], x4.y);
          gcarry[4 * q + 2] = fmaf(Aw[GL ? 0 : 4 * q + 2], gcarry[4 * q + 2], x4.z);
          gcarry[4 * q + 3] = fmaf(Aw[GL ? 0 : 4 * q + 3], gcarry[4 * q + 3], x4.w);
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) gin[v] = fmaf(Ae[GL ? 0 : v], gw[v], Ge[v]);
    }

    // ---- re-run backwards: du, dinit and the gate-group dalpha sums; steps
    // before t_st (look-back warm-up) go to the fp32 workspaces
    // (No reload_barrier on uq / gq here: re-widening them for the re-run
    // cost 12% of the tile loop's instructions at d12, and keeping their
    // fp32 forms fits the registers -- 229 VGPRs at (16, 4, 2), 186 for the
    // chained (16, 4, 4).)
    const Rsrc dur = make_rsrc(dubh + (int64_t)T0 * args.du.s[2] * E);
    const Rsrc dlr = make_rsrc(dlbh + (int64_t)T0 * args.dlg.s[2] * E);
    const Rsrc wdur = make_rsrc(LB ? wdubh + (int64_t)(T0 - t_base) * S.D * 4 : dubh);
    const Rsrc wdlr = make_rsrc(LB ? wdlbh + (int64_t)(T0 - t_base) * S.Da * 4 : dlbh);
    float pl[L];  // GATE_LANE: this lane's dalpha partial per step
#pragma unroll
    for (int s = L - 1; s >= 0; --s) {
      const int t = t0 + s;
      const bool ok = active && t < t_hi;
      const bool wu = LB && t < t_st;
      float gv[V], duv[V], dav[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int ia = GL ? 0 : v;
        gv[v] = fmaf(dk[s][ia], gin[v], Pack<TIO>::get(gq[s], v));
        gin[v] = gv[v];
        duv[v] = al[s][ia] * gv[v];
        dav[v] = (Pack<TIO>::get(uq[s], v) - Pack<TIO>::get(hq[s], v)) * gv[v];
      }
      bst_vec<TIO, VEC>(dur, duoff + s * dustb, duscb, nvalid, ok && !wu, duv);
      if (LB) bst_f32<VEC, V>(wdur, wduoff + s * wdustb, nvalid, ok && wu, duv);
      if (GL) {
        float p = 0.0f;
#pragma unroll
        // (16-byte vectors: every channel of an active lane is valid, and an
        // inactive lane's partial is dropped by `ok` below -- no per-channel
        // select)
        for (int v = 0; v < V; ++v) p += (VEC || v < nvalid) ? dav[v] : 0.0f;
        pl[s] = ok ? p : 0.0f;
      } else {
        // whole groups of r channels (r | V, a power of two) inside the lane:
        // butterfly sums leave every channel holding its group's total; the
        // group's first channel stores the dlogit
#pragma unroll
        for (int m = 1; m < V; m <<= 1) {
          if (m < S.r) {
            float tsum[V];
#pragma unroll
            for (int v = 0; v < V; ++v) tsum[v] = dav[v] + dav[v ^ m];
#pragma unroll
            for (int v = 0; v < V; ++v) dav[v] = tsum[v];
          }
        }
        float dl[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float a = al[s][v];
          dl[v] = use_sig ? dav[v] * (a * (1.0f - a)) : dav[v];
        }
        const uint32_t srow = GM == GATE_CHAN ? opaque(tl0 + s) : (uint32_t)(tl0 + s);
        if (GM == GATE_CHANVEC) {
          // r == 1: the V dlogits of this lane are contiguous
          bst_vec<TIO, true>(dlr, srow * dlstb + (uint32_t)c0 * E, E, V, ok && !wu, dl);
          if (LB) bst_f32<true, V>(wdlr, srow * wdlstb + (uint32_t)c0 * 4, V, ok && wu, dl);
#pragma unroll
          for (int v = 0; v < V; ++v) dacc[v] += ok ? dl[v] : 0.0f;
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const bool lead = ok && (v & (S.r - 1)) == 0 && v < nvalid;
            const uint32_t j = (uint32_t)((c0 + v) / S.r);
            dacc[v] += lead ? dl[v] : 0.0f;
            bst1<TIO>(dlr, lead && !wu ? srow * dlstb + j * dlscb : kOob, dl[v]);
            if (LB) bst_b32(wdlr, lead && wu ? srow * wdlstb + j * 4 : kOob, dl[v]);
          }
        }
      }
    }
    // kept from the last tile processed (it_lo), whose lane tl0 == 0 holds t_base
#pragma unroll
    for (int v = 0; v < V; ++v) dinit_v[v] = (1.0f - al[0][GL ? 0 : v]) * gin[v];

    if (GL) {
      // ---- dlogit[t, j] = slope_t * sum of the group's lane partials: a
      // segmented inclusive scan over the group's channel lanes (TG lanes
      // apart), in a fixed order, leaves the total in the group's last lane,
      // whose own gate gives the slope
      // (compile-time levels with masked adds: a loop or a branch around the
      // shuffles makes the compiler drain every outstanding memory operation
      // at the top of the tile loop).  Every level is a cross-lane shuffle:
      // a group of a non-power-of-two number of lanes (r / V = 3, 5, 6, ...)
      // straddles 16-lane rows, and a lane on the path to its lead can then
      // need a source in the row before, which a DPP row shift cannot reach
      // (it reads 0 there).
      static_loop<0, ilog2(CL)>([&](auto lc) __attribute__((always_inline)) {
        constexpr int d = 1 << decltype(lc)::value;
        const bool take = d < gl_lanes && cl - d >= seg0;
#pragma unroll
        for (int s = 0; s < L; ++s) {
          const float q = __shfl_up(pl[s], d * TG, 64);
          pl[s] += take ? q : 0.0f;
        }
      });
#pragma unroll
      for (int s = 0; s < L; ++s) {
        const int t = t0 + s;
        const bool ok = glead && t < t_hi;
        const bool wu = LB && t < t_st;
        const float a = al[s][0];
        const float d = pl[s] * (use_sig ? a * (1.0f - a) : 1.0f);
        dacc[0] += ok ? d : 0.0f;
        const uint32_t srow = (uint32_t)(tl0 + s);
        bst1<TIO>(dlr, ok && !wu ? srow * dlstb + (uint32_t)gj * dlscb : kOob, d);
        if (LB) bst_b32(wdlr, ok && wu ? srow * wdlstb + (uint32_t)gj * 4 : kOob, d);
      }
    }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  load_tile(it_hi, B0{});
  if constexpr (NB == 2) {
    if constexpr (PD == 2) load_tile(it_hi - 1, B1{});
    for (int it = it_hi; it >= it_lo; it -= 2) {
      process_tile(it, B0{});
      if (it - 1 >= it_lo) process_tile(it - 1, B1{});
    }
  } else {
    for (int it = it_hi; it >= it_lo; --it) process_tile(it, B0{});
  }

  // ---- dinit: the state gradient at t_base, from lane tl0 == 0 of tile it_lo
  if (active && it_hi >= it_lo && it_lo == 0 && tl0 == 0) {
    if (LB) {
      st_f32<VEC, V>(args.wdi + ((int64_t)bh * args.nchunk + chunk) * S.D + c0, nvalid, dinit_v);
    } else if (args.dinit_ws != nullptr || init_f32) {
      // the gradient of the I/O-dtype inits, widened to fp32: into the batch
      // sum's workspace, or straight to fp32 grad_inits
      float rv[V];
#pragma unroll
      for (int v = 0; v < V; ++v) rv[v] = round_io<TIO>(dinit_v[v]);
      if (args.dinit_ws != nullptr) {
        st_f32<VEC, V>(args.dinit_ws + (int64_t)bh * S.D + c0, nvalid, rv);
      } else {
        float* p = reinterpret_cast<float*>(const_cast<void*>(args.dinit.p)) +
                   (int64_t)b * args.dinit.s[0] + (int64_t)h * args.dinit.s[1] +
                   (int64_t)c0 * args.dinit.s[3];
#pragma unroll
        for (int v = 0; v < V; ++v)
          if (v < nvalid) p[v * args.dinit.s[3]] = rv[v];
      }
    } else {
      st_vec<TIO, VEC>(reinterpret_cast<TIO*>(const_cast<void*>(args.dinit.p)) +
                           (int64_t)b * args.dinit.s[0] + (int64_t)h * args.dinit.s[1] +
                           (int64_t)c0 * args.dinit.s[3],
                       args.dinit.s[3], nvalid, dinit_v);
    }
  }

  // ---- dbias partial for (b, h): fixed-order sum of the accumulators
#pragma unroll
  for (int k = 0; k < (GL ? 1 : V); ++k) lds_red[threadIdx.x][k] = dacc[k];
  __syncthreads();
  for (int j = threadIdx.x; j < S.Da; j += NT) {
    float acc = 0.0f;
    if (GL) {
      // group j's dlogits were emitted by its last channel lane, in every
      // time lane (w, tg) of the workgroup
      const int lcl = (j + 1) * gl_lanes - 1;
      for (int ww = 0; ww < NW; ++ww)
        for (int q = 0; q < TG; ++q) acc += lds_red[ww * 64 + lcl * TG + q][0];
    } else {
      // group j is led by channel c = j r: lane cl = c / V, slot c % V, in every
      // time lane (w, tg) of the workgroup
      const int c = j * S.r;
      const int lcl = c / V, k = c % V;
      for (int ww = 0; ww < NW; ++ww)
        for (int q = 0; q < TG; ++q) acc += lds_red[ww * 64 + lcl * TG + q][k];
    }
    args.dbias_partial[((int64_t)bh * args.nchunk + chunk) * S.Da + j] = acc;
  }
  if constexpr (CHAIN) {
    if (threadIdx.x < NCH && (int)threadIdx.x < S.D && chunk > 0)
      chain_clear_abandoned(
          args.ch_words + ((int64_t)bh * (args.nchunk - 1) + chunk - 1) * NCH + threadIdx.x,
          pub_prev);
  }
}

// ---------------------------------------------------------------------------
// Time-chunked backward.  Within a chunk [ts, te) the reverse recurrence maps
// the gradient entering from the chunk's end affinely onto its first step:
//   g_ts = A g_te + G,   A = prod_{t=ts}^{te-1} (1 - alpha_{t+1}),
// with alpha_T taken as 1 (g_T = 0).  scan_bwd_agg_kernel computes (A, G) per
// (b, h, sub-chunk, channel) from gy and the logits alone, one thread per
// channel vector and sub-chunk walking its steps in reverse (V channels per
// lane: one 16-byte gy load per step); scan_bwd_carry_kernel composes the maps
// of the later sub-chunks, last to first, into each chunk's carry g_te; the
// tile kernel then runs all chunks independently.
// ---------------------------------------------------------------------------
template <typename TIO, bool VEC>
__global__ void __launch_bounds__(256) scan_bwd_agg_kernel(const BwdArgs args) {
  constexpr int V = Pack<TIO>::V;
  const ScanShape& S = args.sh;
  const int ncl = (S.D + V - 1) / V;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * args.nfine * ncl) return;
  const int cl = (int)(idx % ncl);
  const int64_t rest = idx / ncl;
  const int chunk = (int)(rest % args.nfine);
  const int bh = (int)(rest / args.nfine);
  const int h = bh % S.H, b = bh / S.H;
  const int c0 = cl * V;
  const int nvalid = min(V, S.D - c0);

  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView gvw = head_view(args.gy, which);
  const int64_t gs[4] = {gvw.s[0], gvw.s[1], gvw.s[2], gvw.s[3]};
  const TIO* gp = reinterpret_cast<const TIO*>(gvw.p) + (int64_t)b * gs[0] +
                  (int64_t)hl * gs[1] + (int64_t)c0 * gs[3];
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1];
  const int64_t lst = args.lg.s[2];
  const bool use_sig = S.use_sigmoid != 0;
  int64_t loff[V];
  float bias[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int j = min(c0 + v, S.D - 1) / S.r;
    loff[v] = (int64_t)j * args.lg.s[3];
    bias[v] = args.bias[h * S.Da + j];
  }
  const bool one_gate = S.r % V == 0;  // every channel of the lane in one gate group
  auto decay = [&](int t, float (&an)[V]) {  // 1 - alpha_t, 0 past the sequence end
    if (t >= S.T) {
#pragma unroll
      for (int v = 0; v < V; ++v) an[v] = 0.0f;
    } else if (one_gate) {
      const float a = gate_alpha(Pack<TIO>::load1(lp + (int64_t)t * lst + loff[0]) + bias[0],
                                 use_sig);
#pragma unroll
      for (int v = 0; v < V; ++v) an[v] = 1.0f - a;
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v)
        an[v] = 1.0f - gate_alpha(Pack<TIO>::load1(lp + (int64_t)t * lst + loff[v]) + bias[v],
                                  use_sig);
    }
  };

  const int ts = chunk * args.fine_steps;
  const int te = min(S.T, ts + args.fine_steps);
  float A[V], G[V], an[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    A[v] = 1.0f;
    G[v] = 0.0f;
  }
  decay(te, an);
  // blocks of KB steps, newest first: all of a block's loads are issued before
  // its (sequential) arithmetic, so the walk is not one load latency per step
  constexpr int KB = 16;
  for (int tb = te; tb > ts; tb -= KB) {
    uint4 q[KB];
    float lraw[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const int t = tb - 1 - k;
      const bool ok = t >= ts;
      q[k] = ok ? ld_vec<TIO, VEC>(gp + (int64_t)t * gs[2], gs[3], nvalid)
                : make_uint4(0u, 0u, 0u, 0u);
      lraw[k] = ok && one_gate ? Pack<TIO>::load1(lp + (int64_t)t * lst + loff[0]) : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const int t = tb - 1 - k;
      if (t >= ts) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          G[v] = fmaf(an[v], G[v], Pack<TIO>::get(q[k], v));
          A[v] *= an[v];
        }
        if (one_gate) {
          const float a = gate_alpha(lraw[k] + bias[0], use_sig);
#pragma unroll
          for (int v = 0; v < V; ++v) an[v] = 1.0f - a;
        } else {
          decay(t, an);
        }
      }
    }
  }
  const int64_t o = ((int64_t)bh * args.nfine + chunk) * S.D + c0;
  const int64_t plane = (int64_t)S.B * S.H * args.nfine * S.D;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if (v < nvalid) {
      args.agg[o + v] = A[v];
      args.agg[plane + o + v] = G[v];
    }
  }
}

// ---------------------------------------------------------------------------
// Look-back backward: the contributions of later windows' warm-ups.
//
// A step t lies in the warm-up [lo_c, st_c) of the windows c = c0(t), c0(t)+1,
// ... while lo_c <= t, where c0(t) is the first window starting after t.  Its
// gradient is the owning window's (already in du / dlg, written by the LB tile
// kernel) plus those windows' fp32 contributions, added in window order and
// rounded once.  One thread per (b h, window, warm-up row, channel of the
// D + Da value and logit slots); the thread whose window is c0(t) does the sum,
// so each step is written by exactly one thread.
// ---------------------------------------------------------------------------
template <typename TIO>
__global__ void __launch_bounds__(256) scan_lb_fold_kernel(const BwdArgs args) {
  const ScanShape& S = args.sh;
  const int nw = args.nchunk;
  const int nch = S.D + S.Da;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * nw * args.kw * nch) return;
  const int ch = (int)(idx % nch);
  int64_t rest = idx / nch;
  const int row = (int)(rest % args.kw);
  rest /= args.kw;
  const int win = (int)(rest % nw);
  const int64_t bh = rest / nw;
  if (win == 0) return;  // the first window has no warm-up
  const Window wd = look_back_window(win, S.T, args.P, args.Q, args.K);
  const int t = wd.lo + row;
  if (t >= wd.st) return;
  const int cfirst = t < args.P ? 1 : (t - args.P) / args.Q + 2;  // first window with st > t
  if (win != cfirst) return;
  const int h = (int)(bh % S.H), b = (int)(bh / S.H);
  TIO* gp;
  if (ch < S.D) {
    gp = reinterpret_cast<TIO*>(const_cast<void*>(args.du.p)) + (int64_t)b * args.du.s[0] +
         (int64_t)h * args.du.s[1] + (int64_t)t * args.du.s[2] + (int64_t)ch * args.du.s[3];
  } else {
    gp = reinterpret_cast<TIO*>(const_cast<void*>(args.dlg.p)) + (int64_t)b * args.dlg.s[0] +
         (int64_t)h * args.dlg.s[1] + (int64_t)t * args.dlg.s[2] +
         (int64_t)(ch - S.D) * args.dlg.s[3];
  }
  float acc = Pack<TIO>::load1(gp);
  for (int c = win; c < nw; ++c) {
    const Window wc = look_back_window(c, S.T, args.P, args.Q, args.K);
    if (wc.lo > t) break;
    const int64_t r = (bh * nw + c) * args.kw + (t - wc.lo);
    acc += ch < S.D ? args.wdu[r * S.D + ch] : args.wdl[r * S.Da + (ch - S.D)];
  }
  Pack<TIO>::store1(gp, acc);
}

// grad_inits[b, h, d] = sum over the non-empty windows of their fp32
// contributions, in window order.  With grad_inits summed over the batch
// (args.dinit_ws set), the per-sequence gradient goes there instead, rounded to
// the I/O dtype as a per-sequence gradient tensor would be, for the batch sum
// of the dbias reduction launch.
template <typename TIO>
__global__ void __launch_bounds__(256) scan_lb_dinit_kernel(const BwdArgs args) {
  const ScanShape& S = args.sh;
  const int nw = args.nchunk;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * S.D) return;
  const int d = (int)(idx % S.D);
  const int64_t bh = idx / S.D;
  const int h = (int)(bh % S.H), b = (int)(bh / S.H);
  // only the first window can be empty (P = 0); the shares are read in batches
  // so the walk over the windows is not one load latency per window
  const Window w0 = look_back_window(0, S.T, args.P, args.Q, args.K);
  const float* wp = args.wdi + bh * nw * S.D + d;
  float acc = 0.0f;
  constexpr int KB = 16;
  for (int c0 = w0.hi > w0.lo ? 0 : 1; c0 < nw; c0 += KB) {
    float x[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) x[k] = c0 + k < nw ? wp[(int64_t)(c0 + k) * S.D] : 0.0f;
#pragma unroll
    for (int k = 0; k < KB; ++k) acc += x[k];
  }
  if (args.dinit_ws != nullptr) {
    args.dinit_ws[bh * S.D + d] = round_io<TIO>(acc);
    return;
  }
  const int64_t o = (int64_t)b * args.dinit.s[0] + (int64_t)h * args.dinit.s[1] +
                    (int64_t)d * args.dinit.s[3];
  if (args.init_f32) {
    // fp32 inits read as bf16: the gradient of the bf16 tensor, widened
    reinterpret_cast<float*>(const_cast<void*>(args.dinit.p))[o] =
        __uint_as_float(cvt_pk_bf16(acc, 0.0f) << 16);
  } else {
    Pack<TIO>::store1(reinterpret_cast<TIO*>(const_cast<void*>(args.dinit.p)) + o, acc);
  }
}

// ---------------------------------------------------------------------------
// Generic backward for gate groups that neither fill whole lanes nor fit inside
// one (r neither a multiple nor a divisor of V, or too many groups per head).
// One thread per (b, h, channel) walks T backwards; the per-channel dalpha terms
// go to an fp32 workspace and a second kernel reduces each group in channel
// order.
// ---------------------------------------------------------------------------
template <typename TIO>
__global__ void scan_bwd_channel_kernel(const BwdArgs args, float* __restrict__ dalpha_ws) {
  const ScanShape& S = args.sh;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * S.D) return;
  const int c = (int)(idx % S.D);
  const int h = (int)((idx / S.D) % S.H);
  const int b = (int)(idx / ((int64_t)S.D * S.H));
  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView hvw = head_view(args.h, which), gvw = head_view(args.gy, which);
  const TIO* hp = reinterpret_cast<const TIO*>(hvw.p) + (int64_t)b * hvw.s[0] +
                  (int64_t)hl * hvw.s[1] + (int64_t)c * hvw.s[3];
  const TIO* gp = reinterpret_cast<const TIO*>(gvw.p) + (int64_t)b * gvw.s[0] +
                  (int64_t)hl * gvw.s[1] + (int64_t)c * gvw.s[3];
  const TIO* up = reinterpret_cast<const TIO*>(args.u.p) + (int64_t)b * args.u.s[0] +
                  (int64_t)h * args.u.s[1] + (int64_t)c * args.u.s[3];
  TIO* dup = reinterpret_cast<TIO*>(const_cast<void*>(args.du.p)) + (int64_t)b * args.du.s[0] +
             (int64_t)h * args.du.s[1] + (int64_t)c * args.du.s[3];
  const int j = c / S.r;
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1] + (int64_t)j * args.lg.s[3];
  const float bias = args.bias[h * S.Da + j];
  const bool use_sig = S.use_sigmoid != 0;
  float g = 0.0f, a_next = 0.0f;
  for (int t = S.T - 1; t >= 0; --t) {
    const float alpha = gate_alpha(Pack<TIO>::load1(lp + (int64_t)t * args.lg.s[2]) + bias, use_sig);
    g = fmaf(a_next, g, Pack<TIO>::load1(gp + (int64_t)t * gvw.s[2]));
    Pack<TIO>::store1(dup + (int64_t)t * args.du.s[2], alpha * g);
    float hprev;
    if (t == 0) {
      const TIO* ip = reinterpret_cast<const TIO*>(args.init.p) + (int64_t)b * args.init.s[0] +
                      (int64_t)h * args.init.s[1] + (int64_t)c * args.init.s[3];
      hprev = Pack<TIO>::load1(ip);
      TIO* dip = reinterpret_cast<TIO*>(const_cast<void*>(args.dinit.p)) +
                 (int64_t)b * args.dinit.s[0] + (int64_t)h * args.dinit.s[1] +
                 (int64_t)c * args.dinit.s[3];
      Pack<TIO>::store1(dip, (1.0f - alpha) * g);
    } else {
      hprev = Pack<TIO>::load1(hp + (int64_t)(t - 1) * hvw.s[2]);
    }
    const float da = (Pack<TIO>::load1(up + (int64_t)t * args.u.s[2]) - hprev) * g;
    dalpha_ws[(((int64_t)b * S.H + h) * S.T + t) * S.D + c] = da;
    a_next = 1.0f - alpha;
  }
}

// One thread per (b, h, gate group j) over all t, so the dbias partial needs
// no extra pass.  du_ws (look-back windows): the group's value gradients,
// summed over windows in fp32, rounded to the I/O dtype here.
template <typename TIO>
__global__ void scan_bwd_group_reduce_kernel(const BwdArgs args,
                                             const float* __restrict__ dalpha_ws,
                                             const float* __restrict__ du_ws) {
  const ScanShape& S = args.sh;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * S.Da) return;
  const int j = (int)(idx % S.Da);
  const int h = (int)((idx / S.Da) % S.H);
  const int b = (int)(idx / ((int64_t)S.Da * S.H));
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1] + (int64_t)j * args.lg.s[3];
  TIO* dlp = reinterpret_cast<TIO*>(const_cast<void*>(args.dlg.p)) + (int64_t)b * args.dlg.s[0] +
             (int64_t)h * args.dlg.s[1] + (int64_t)j * args.dlg.s[3];
  const float bias = args.bias[h * S.Da + j];
  const bool use_sig = S.use_sigmoid != 0;
  TIO* dup = reinterpret_cast<TIO*>(const_cast<void*>(args.du.p)) + (int64_t)b * args.du.s[0] +
             (int64_t)h * args.du.s[1] + (int64_t)j * S.r * args.du.s[3];
  float acc_b = 0.0f;
  for (int t = 0; t < S.T; ++t) {
    const int64_t ro = (((int64_t)b * S.H + h) * S.T + t) * S.D + (int64_t)j * S.r;
    const float* row = dalpha_ws + ro;
    float p = 0.0f;
    for (int q = 0; q < S.r; ++q) p += row[q];
    if (du_ws != nullptr)
      for (int q = 0; q < S.r; ++q)
        Pack<TIO>::store1(dup + (int64_t)t * args.du.s[2] + (int64_t)q * args.du.s[3],
                          du_ws[ro + q]);
    const float alpha = gate_alpha(Pack<TIO>::load1(lp + (int64_t)t * args.lg.s[2]) + bias, use_sig);
    const float d = use_sig ? p * (alpha * (1.0f - alpha)) : p;
    Pack<TIO>::store1(dlp + (int64_t)t * args.dlg.s[2], d);
    acc_b += d;
  }
  args.dbias_partial[idx] = acc_b;
}

// Look-back windows with such gate groups: the same walk per (b, h, channel),
// window by window from the last.  Each window runs its reverse chain over
// [lo, hi), with upstream gradients on its own steps [st, hi) only; the state
// before step t is the saved output (t - 1 >= st), the warm-up state in wst
// (lo <= t - 1 < st: row t - 1 - lo of the window's rows) or the inits
// (t = lo).  A step lies in its own window and in the warm-ups of later ones:
// its du and dalpha terms are summed in fp32 workspaces (B, H, T, D), where
// the first window to reach it writes -- the latest that covers it, as the
// windows run latest first, so the step lies below the next window's lo --
// and the others add; the group reduction then rounds du once.  The inits
// gradient sums every window's term at its first step.
template <typename TIO>
__global__ void scan_lb_channel_kernel(const BwdArgs args, float* __restrict__ dalpha_ws,
                                       float* __restrict__ du_ws) {
  const ScanShape& S = args.sh;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)S.B * S.H * S.D) return;
  const int c = (int)(idx % S.D);
  const int h = (int)((idx / S.D) % S.H);
  const int b = (int)(idx / ((int64_t)S.D * S.H));
  int which, hl;
  head_select(h, S.NH, S.NKVH, which, hl);
  const HeadView hvw = head_view(args.h, which), gvw = head_view(args.gy, which);
  const TIO* hp = reinterpret_cast<const TIO*>(hvw.p) + (int64_t)b * hvw.s[0] +
                  (int64_t)hl * hvw.s[1] + (int64_t)c * hvw.s[3];
  const TIO* gp = reinterpret_cast<const TIO*>(gvw.p) + (int64_t)b * gvw.s[0] +
                  (int64_t)hl * gvw.s[1] + (int64_t)c * gvw.s[3];
  const TIO* up = reinterpret_cast<const TIO*>(args.u.p) + (int64_t)b * args.u.s[0] +
                  (int64_t)h * args.u.s[1] + (int64_t)c * args.u.s[3];
  const int j = c / S.r;
  const TIO* lp = reinterpret_cast<const TIO*>(args.lg.p) + (int64_t)b * args.lg.s[0] +
                  (int64_t)h * args.lg.s[1] + (int64_t)j * args.lg.s[3];
  const float bias = args.bias[h * S.Da + j];
  const bool use_sig = S.use_sigmoid != 0;
  const float init = Pack<TIO>::load1(reinterpret_cast<const TIO*>(args.init.p) +
                                      (int64_t)b * args.init.s[0] + (int64_t)h * args.init.s[1] +
                                      (int64_t)c * args.init.s[3]);
  const int nwin = args.nchunk;
  const TIO* wsp = reinterpret_cast<const TIO*>(args.wst) +
                   ((int64_t)b * S.H + h) * nwin * args.kw * S.D + c;
  const int64_t base = ((int64_t)b * S.H + h) * S.T * S.D + c;
  float dinit = 0.0f;
  int lo_next = S.T;  // lo of the window after the current one (T: none)
  for (int w = nwin - 1; w >= 0; --w) {
    const Window wd = look_back_window(w, S.T, args.P, args.Q, args.K);
    float g = 0.0f, a_next = 0.0f;
    for (int t = wd.hi - 1; t >= wd.lo; --t) {
      const float alpha =
          gate_alpha(Pack<TIO>::load1(lp + (int64_t)t * args.lg.s[2]) + bias, use_sig);
      const float gy = t >= wd.st ? Pack<TIO>::load1(gp + (int64_t)t * gvw.s[2]) : 0.0f;
      g = fmaf(a_next, g, gy);
      float hprev;
      if (t == wd.lo)
        hprev = init;
      else if (t - 1 >= wd.st)
        hprev = Pack<TIO>::load1(hp + (int64_t)(t - 1) * hvw.s[2]);
      else
        hprev = Pack<TIO>::load1(wsp + ((int64_t)w * args.kw + (t - 1 - wd.lo)) * S.D);
      const float du = alpha * g;
      const float da = (Pack<TIO>::load1(up + (int64_t)t * args.u.s[2]) - hprev) * g;
      const int64_t o = base + (int64_t)t * S.D;
      if (t < lo_next) {
        du_ws[o] = du;
        dalpha_ws[o] = da;
      } else {
        du_ws[o] += du;
        dalpha_ws[o] += da;
      }
      a_next = 1.0f - alpha;
    }
    dinit += a_next * g;  // the window's first step reads the inits
    lo_next = wd.lo;
  }
  Pack<TIO>::store1(reinterpret_cast<TIO*>(const_cast<void*>(args.dinit.p)) +
                        (int64_t)b * args.dinit.s[0] + (int64_t)h * args.dinit.s[1] +
                        (int64_t)c * args.dinit.s[3],
                    dinit);
}

// ---------------------------------------------------------------------------
// Launch configuration and host launchers (ltv_scan_fwd*.hip / ltv_scan_bwd.hip)
// ---------------------------------------------------------------------------
struct ScanCfg {
  int CL, L, NW;
};

// Forward: grid = B * H * nslab workgroups of NW * 64 threads.
int scan_launch_fwd(bool bf16, const FwdArgs& a, ScanCfg cfg, int grid, bool vec, int gm,
                    hipStream_t st);
// Forward with chained chunk states: grid = nseq * nchunk workgroups (vector
// accesses only; gate modes GATE_LANE and GATE_CHANVEC).
int scan_launch_fwd_chain(bool bf16, const FwdArgs& a, const ChainArgs& ch, ScanCfg cfg, int gm,
                          hipStream_t st);
// Backward main kernel: grid = B * H * nchunk; CL channel lanes cover the whole
// head; lb selects the look-back window kernels.
int scan_launch_bwd(bool bf16, const BwdArgs& a, ScanCfg cfg, int grid, bool vec, int gm,
                    bool lb, hipStream_t st);
// Chained backward: grid = B * H * nchunk workgroups, one tile per chunk
// (vector accesses only; gate modes GATE_LANE and GATE_CHANVEC).
int scan_launch_bwd_chain(bool bf16, const BwdArgs& a, ScanCfg cfg, int grid, int gm,
                          hipStream_t st);
// Look-back backward: warm-up contributions into du / dlg, then grad_inits.
int scan_launch_lb_fold(bool bf16, const BwdArgs& a, hipStream_t st);
int scan_launch_lb_dinit(bool bf16, const BwdArgs& a, hipStream_t st);
// Short-window look-back kernels (ltv_scan_lb.hip): one lane per (b, h,
// window, channel vector).  The backward also needs kw_max >= K - 1 (8 or 16).
// buf: every view spans less than 2^31 bytes, so the buffer-addressed kernels apply
int scan_launch_lb_short_fwd(bool bf16, const FwdArgs& a, bool vec, int gm, bool buf,
                             hipStream_t st);
int scan_launch_lb_short_bwd(bool bf16, const BwdArgs& a, bool vec, int gm, int kw_max, bool buf,
                             hipStream_t st);
// Backward for gate groups outside the main kernel's reduction patterns.
int scan_launch_bwd_channel(bool bf16, const BwdArgs& a, float* dalpha_ws, hipStream_t st);
// The same for look-back windows (a.nchunk windows, warm-up states in a.wst):
// value and dalpha terms summed over windows in fp32 workspaces of
// (B, H, T, D) each.
int scan_launch_lb_channel(bool bf16, const BwdArgs& a, float* dalpha_ws, float* du_ws,
                           hipStream_t st);
// The batch sum of the inits gradient, done by the dbias reduction's launch:
// out[h, d] (strides sh, sd elements; fp32, or bf16 with out_bf16) = the sum
// over b, in batch order, of ws[(b H + h) D + d].
struct DinitSum {
  const float* ws = nullptr;  // null: no sum
  void* out = nullptr;
  int64_t sh = 0, sd = 0;
  int D = 0, out_bf16 = 0;
};
// Zeroes `pad` slots of the logit-gradient view past the last head's last
// gate in every (b, t) row: slot q = q0 + p at b sb + t st + q sq elements
// (esize bytes each), done by the dbias reduction's launch.  For a consumer
// that reads whole 16-byte chunks past the last logit column.
struct PadZero {
  char* base = nullptr;  // null: nothing to zero
  int64_t sb = 0, st = 0, sq = 0;
  int B = 0, T = 0, q0 = 0, pad = 0, esize = 2;
};
// dbias[h, j] = sum_b partial[b, h, j] (and the inits gradient's batch sum,
// and the padding slots' zeros)
int scan_launch_dbias_reduce(const float* partial, float* dbias, int B, int H, int NC, int Da,
                             hipStream_t st, const DinitSum& ds = DinitSum(),
                             const PadZero& pz = PadZero());

}  // namespace ltv
