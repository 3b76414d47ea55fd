// bf16 MFMA GEMM with direct global -> LDS loads (gfx950 buffer_load ... lds).
//
//   Out(i, j) = sum_k P(i, k) * Q(j, k)         (same contract as ltv_gemm_mfma.hpp)
//
// The operand tiles never pass through VGPRs: each wavefront issues
// buffer_load_dwordx4 with the LDS bit, which writes its 64 lanes' 16-byte chunks
// to 1 KB of LDS at the M0 base.  A k-step is kDmaBK = 64 reduction indices, so
// every row of a KC operand is fetched as one full 128-byte line: the L2 serves
// about one request per channel per clock whatever its size, and 64-byte
// requests halve its throughput.  Two stages (2 x 64 KB for a 256 x 256 tile)
// double-buffer the k-steps: the loads of step s + 1 are issued at the start of
// step s, by half of the wavefronts, and waited for at its end, one barrier per
// step; the last k16 sub-step of each step runs after that barrier.
//
// LDS layouts (no padding; 16-byte chunks XOR-swizzled so both fragment reads
// are bank-conflict free):
//   KC tile [R rows][64 k] (128 B rows): chunk c of row r sits at slot
//       c ^ ((r >> 1) & 7); any 16 consecutive rows then cover 16 distinct
//       16-byte bank windows for the ds_read_b128 fragment reads.
//   RC tile [64 k][R rows] (2R-byte rows): row-chunk c of k-row k sits at slot
//       c ^ (4 (k & 3)); the 4 k-rows one 16-lane group of ds_read_b64_tr_b16
//       reads then land in 4 disjoint 64-byte windows.
// The swizzle is applied on the load side by choosing which global chunk each
// lane fetches (a lane's LDS destination is fixed by its lane index); the
// lanes that fill one row still fetch one whole 128-byte line.
//
// Chunks past an operand's rows or reduction range are not fetched: the lane
// gets an offset the buffer range check rejects, which writes zeros to LDS.
// The wait for a stage is an explicit s_waitcnt vmcnt on this wavefront's own
// loads followed by s_barrier, so every wavefront's loads into the stage have
// landed before any wavefront reads it.
#pragma once

#include "ltv_gemm_mfma.hpp"

namespace ltv {

// Reduction indices per k-step and LDS stages (kDmaStages - 1 k-steps in
// flight).  Measured on MI355X at d12: 64 x 2 stages beats 32 x 4 stages
// (forward GEMM 134 vs 148 us, dX 140 vs 166 us) -- twice the barriers and
// half-line L2 requests cost more than the deeper pipeline gains.
constexpr int kDmaBK = 64;
constexpr int kDmaStages = 2;
constexpr int kDmaRowBytes = kDmaBK * 2;          // a KC tile row
constexpr int kDmaRowSlots = kDmaRowBytes / 16;   // 16-byte chunks per KC row
constexpr int kDmaRowPhase = 256 / kDmaRowBytes;  // KC rows per 256-byte bank window
static_assert(kDmaBK % 16 == 0 && kDmaRowPhase >= 1 && kDmaStages >= 2, "bad DMA step");

// LDS slot of 16-byte chunk c in row r of a KC tile: any 16 consecutive rows
// then cover 16 distinct 16-byte bank windows for one chunk index.
__host__ __device__ constexpr int dma_kc_slot(int r, int c) {
  return c ^ ((r / kDmaRowPhase) & (kDmaRowSlots - 1));
}

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer resource (stride 0) over [p, p + bytes): gfx9 word 3 = 0x00020000.
__device__ __forceinline__ i32x4_t make_buffer_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  i32x4_t r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)(uint32_t)((a >> 32) & 0xffffu);
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}

// One wavefront-wide 16-byte-per-lane load into LDS at lds_base (wave-uniform
// byte address): lane l's chunk goes to lds_base + 16 l.
// lds_base is bound to M0 as an input operand ("{m0}"), so the compiler
// writes M0 itself and knows it is read here; nothing clobbers the register
// it reserves.  The load stays inline asm rather than the
// buffer-load-to-LDS builtin: with the builtin the compiler cannot tell that
// a k-step's loads fill the other LDS stage, and waits for all of them
// (vmcnt(0)) before the first fragment read of the row-contiguous kernels'
// every k-step.  The nop covers the M0 write -> LDS-DMA hazard.
__device__ __forceinline__ void dma16(uint32_t lds_base, i32x4_t rsrc, uint32_t voffset,
                                      uint32_t soffset) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds_base)
               : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// s_waitcnt vmcnt(n) for a wave-uniform runtime n in [LO, HI] (binary dispatch
// to the immediate forms).
template <int LO, int HI>
__device__ __forceinline__ void wait_vmcnt_range(int n) {
  if constexpr (LO == HI) {
    wait_vmcnt<LO>();
  } else {
    constexpr int MID = (LO + HI) / 2;
    if (n <= MID)
      wait_vmcnt_range<LO, MID>(n);
    else
      wait_vmcnt_range<MID + 1, HI>(n);
  }
}

// Wait until at most n of this wavefront's vector memory instructions are
// outstanding (n above the 6-bit counter's range waits for 63).
__device__ __forceinline__ void wait_vmcnt_rt(int n) { wait_vmcnt_range<0, 63>(n < 63 ? n : 63); }

// Cache policy of the epilogue stores: streaming (nt) at device scope (sc1).
// The output is not read again by the kernel, and every CU ends its tiles at
// about the same time: measured on MI355X this burst drains faster than with
// the default policy (a GEMM of the forward's shape: 139 vs 146 us), and the
// scan that reads the forward's outputs next runs faster after streaming
// stores (62 against 69 us after default ones).  The split partials of dW,
// which dw_reduce reads back at once, are stored without nt (sc1 only): dW
// 131 -> 127-128 us.
#ifndef LTV_EPI_STORE_POLICY
#define LTV_EPI_STORE_POLICY " nt sc1"
#endif
#ifndef LTV_EPI_PARTIAL_POLICY
#define LTV_EPI_PARTIAL_POLICY " sc1"
#endif

typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// One buffer store instruction each (exactly one vmcnt event, whatever the
// lanes' offsets; lanes with an offset past num_records write nothing).
__device__ __forceinline__ void buf_store_b64(u32x2_t v, uint32_t voff, i32x4_t rsrc) {
  asm volatile("buffer_store_dwordx2 %0, %1, %2, 0 offen" LTV_EPI_STORE_POLICY : : "v"(v),
               "v"(voff), "s"(rsrc) : "memory");
}
// A store of more than 8 bytes reads its data registers a cycle late: the nop
// keeps the next VALU write to them from landing first (the compiler inserts
// such wait states for its own instructions, not around inline asm).
__device__ __forceinline__ void buf_store_b128(u32x4_t v, uint32_t voff, i32x4_t rsrc) {
  asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen" LTV_EPI_STORE_POLICY "\n\ts_nop 1"
               : : "v"(v), "v"(voff), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void buf_store_b128_partial(u32x4_t v, uint32_t voff, i32x4_t rsrc) {
  asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen" LTV_EPI_PARTIAL_POLICY "\n\ts_nop 1"
               : : "v"(v), "v"(voff), "s"(rsrc) : "memory");
}

__device__ __forceinline__ void lds_fence() { asm volatile("" : : : "memory"); }

template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// Byte offset that the buffer range check rejects: such a lane's load writes
// zeros to LDS.  Operands are limited to kDmaMaxSpan elements, so num_records
// <= kDmaOob, and kDmaOob plus any in-range byte offset (< 2^31 - 2^21) plus
// 16 stays below 2^32: a row past the operand keeps a rejected offset when the
// k-step's offset is added to it.
constexpr uint32_t kDmaOob = 0x80000000u;
constexpr int64_t kDmaMaxSpan = (1ll << 30) - (1ll << 20);

// Per-operand DMA plan: which global 8-element chunk each lane fetches for each
// of its wavefront's instructions in a stage (fixed per work item), plus the
// resource.  The whole offset is per lane (the scalar offset is 0), and a chunk
// is fetched only if its rows and reductions indices are all valid:
//   KC: row < rows and k0 + c8 < kend   (kend a multiple of 8 or the chunk
//       straddling it reads buffer contents past kend, which must then be 0)
//   RC: rows a multiple of 8, row0 + c8 < rows and k < kend
// Elements an operand in the batched layout spans (the batched index's
// extent -- rows for RC, the reduction K for KC -- rounded up to whole batches).
__host__ __device__ inline int64_t dma_batched_span(const GemmOperand& op, int K, int layout) {
  const int n = layout == OP_KC ? K : op.rows;
  return (int64_t)((n + op.blen - 1) / op.blen) * op.bstride;
}

template <int R, int L, int NW>
struct DmaOperand {
  static constexpr int kInstr = R * kDmaBK * 2 / 1024;  // 1 KB instructions per stage
  static constexpr int kPerWave = kInstr / NW;
  static_assert(kInstr % NW == 0 && kPerWave >= 1, "tile too small for the wavefronts");
  static_assert(L == OP_KC || R >= 128, "RC tiles need >= 16 chunks per k-row");
  i32x4_t rsrc;
  uint32_t base[kPerWave];  // byte offset at k0 = 0, or kDmaOob
  int kk[kPerWave];         // this lane's reduction offset within a k-step
  uint32_t kstride;         // elements per unit of k
  int kend;
  int64_t kbstride;  // KC batched reduction index (kblen > 0): k0 -> batch k0 / kblen
  int kblen;

  __device__ __forceinline__ void setup(const GemmOperand& op, int K, int row0, int ke, int wave,
                                        int lane) {
    const int64_t span = op.blen > 0 ? dma_batched_span(op, K, L)
                                     : L == OP_KC ? (int64_t)op.rows * op.ld : (int64_t)K * op.ld;
    rsrc = make_buffer_rsrc(op.p, (uint32_t)(span * 2));
    kbstride = L == OP_KC ? op.bstride : 0;
    kblen = L == OP_KC ? op.blen : 0;
    // RC batched rows: the tile's rows lie in batch row0 / blen
    const int64_t rbase =
        L == OP_RC && op.blen > 0 ? (int64_t)(row0 / op.blen) * op.bstride + row0 % op.blen : row0;
#pragma unroll
    for (int w = 0; w < 4; ++w) rsrc[w] = __builtin_amdgcn_readfirstlane(rsrc[w]);
    kstride = L == OP_KC ? 1u : (uint32_t)op.ld;
    kend = min(ke, op.k_valid);
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const int o = (wave * kPerWave + i) * 1024 + lane * 16;  // byte offset in the tile
      if (L == OP_KC) {
        const int row = o / kDmaRowBytes, slot = (o >> 4) % kDmaRowSlots;
        const int c = dma_kc_slot(row, slot);  // the swizzle is an involution
        kk[i] = c * 8;
        base[i] = row0 + row < op.rows ? (uint32_t)((row0 + row) * (int64_t)op.ld + c * 8) * 2u
                                       : kDmaOob;
      } else {
        const int k = o / (R * 2), slot = (o % (R * 2)) >> 4;
        const int c = slot ^ (4 * (k & 3));
        kk[i] = k;
        base[i] = row0 + c * 8 < op.rows ? (uint32_t)(k * (int64_t)op.ld + rbase + c * 8) * 2u
                                         : kDmaOob;
      }
    }
  }

  // loads of the k-step starting at k0 into the stage at lds_stage (byte address)
  __device__ __forceinline__ void issue(uint32_t lds_stage, int k0, int wave) const {
    const uint32_t koff = kblen > 0 ? (uint32_t)((int64_t)(k0 / kblen) * kbstride + k0 % kblen)
                                    : (uint32_t)k0 * kstride;
    const uint32_t koff2 = koff * 2u;
    if (k0 + kDmaBK <= kend) {
      // every reduction index of the step is valid: one add per load (a row
      // past the operand keeps an offset >= kDmaOob)
#pragma unroll
      for (int i = 0; i < kPerWave; ++i)
        dma16(__builtin_amdgcn_readfirstlane(lds_stage + (uint32_t)((wave * kPerWave + i) * 1024)),
              rsrc, base[i] + koff2, 0u);
    } else {
#pragma unroll
      for (int i = 0; i < kPerWave; ++i) {
        const bool ok = base[i] != kDmaOob && k0 + kk[i] < kend;
        dma16(__builtin_amdgcn_readfirstlane(lds_stage + (uint32_t)((wave * kPerWave + i) * 1024)),
              rsrc, ok ? base[i] + koff2 : kDmaOob, 0u);
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Epilogues of the direct-to-LDS kernel.  Same outputs as the epilogues in
// ltv_gemm_mfma.hpp, but written with buffer stores whose masked lanes carry an
// out-of-range offset, so every call issues a wave-uniform, known number of
// store instructions: store_block returns that number, which the kernel adds
// to its vmcnt bookkeeping.  Output buffers must be at most kDmaMaxBytes.
// ---------------------------------------------------------------------------
constexpr int64_t kDmaMaxBytes = 1ll << 31;

__device__ __forceinline__ i32x4_t uniform_rsrc(const void* p, int64_t bytes) {
  i32x4_t r = make_buffer_rsrc(p, (uint32_t)bytes);
#pragma unroll
  for (int w = 0; w < 4; ++w) r[w] = __builtin_amdgcn_readfirstlane(r[w]);
  return r;
}

__device__ __forceinline__ u32x2_t pack4_bf16_v(const f32x16_t& v, int q) {
  u32x2_t r;
  r[0] = cvt_pk_bf16(v[4 * q], v[4 * q + 1]);
  r[1] = cvt_pk_bf16(v[4 * q + 2], v[4 * q + 3]);
  return r;
}

// Per-wavefront LDS staging of output blocks for full-line stores: 32 rows of
// 128 bytes, 16-byte chunk c of row r at slot c ^ (r & 7) (the row-wise reads
// back are bank-conflict free).  A store instruction then writes 8 rows x 128
// contiguous bytes instead of 32 rows x 16 bytes: the L2 takes one request per
// line either way, so partial-line stores cost 4x the requests.
constexpr int kEpiStageBytes = 4096;
typedef __attribute__((address_space(3))) char lds_char_t;

__device__ __forceinline__ lds_char_t* stage_slot(lds_char_t* st, int row, int byte) {
  return st + row * 128 + ((((byte >> 4) ^ (row & 7))) << 4) + (byte & 15);
}
__device__ __forceinline__ void stage_put(lds_char_t* st, int row, int byte, u32x2_t v) {
  *(__attribute__((address_space(3))) u32x2_t*)stage_slot(st, row, byte) = v;
}
__device__ __forceinline__ void stage_put(lds_char_t* st, int row, int byte, u32x4_t v) {
  *(__attribute__((address_space(3))) u32x4_t*)stage_slot(st, row, byte) = v;
}
// chunk (16 bytes) c of row r
__device__ __forceinline__ u32x4_t stage_get(lds_char_t* st, int row, int c) {
  return *(__attribute__((address_space(3))) const u32x4_t*)stage_slot(st, row, c * 16);
}

// Stage two 32 x 32 bf16 blocks (output rows j = lane & 31, 64 columns) of one
// wavefront: afterwards row r of the stage holds columns 0..63 of block row r.
__device__ __forceinline__ void stage_bf16_pair(lds_char_t* st, const f32x16_t& lo,
                                                const f32x16_t& hi, int lane) {
  const int row = lane & 31, h4 = 4 * (lane >> 5);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    stage_put(st, row, (8 * q + h4) * 2, pack4_bf16_v(lo, q));
    stage_put(st, row, (32 + 8 * q + h4) * 2, pack4_bf16_v(hi, q));
  }
}

template <class Epi>
struct DmaEpi;

// Bytes an EpiRowBF16 output spans.
__host__ __device__ inline int64_t epi_row_bf16_bytes(const EpiRowBF16& e) {
  if (e.blen > 0) return (int64_t)((e.i_valid + e.blen - 1) / e.blen) * e.bstride * 2;
  return (int64_t)e.j_valid * e.ldc * 2;
}

template <>
struct DmaEpi<EpiRowBF16> {
  i32x4_t rsrc;
  int64_t ldc, bstride;
  int i_valid, j_valid, blen;
  __device__ __forceinline__ DmaEpi(const EpiRowBF16& e, const GemmArgs&)
      : rsrc(uniform_rsrc(e.c, epi_row_bf16_bytes(e))), ldc(e.ldc), bstride(e.bstride),
        i_valid(e.i_valid), j_valid(e.j_valid), blen(e.blen) {}
  // element offset of column i (in a batch-aligned tile) at row 0
  __device__ __forceinline__ int64_t col(int i) const {
    return blen > 0 ? (int64_t)(i / blen) * bstride + i % blen : i;
  }
  __device__ __forceinline__ int store_block(int i, int j, int, int lane,
                                             const f32x16_t& v) const {
    const int il = i + 4 * (lane >> 5);
    const uint32_t off = (uint32_t)((int64_t)j * ldc + col(il)) * 2u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool ok = j < j_valid && il + 8 * q < i_valid;
      buf_store_b64(pack4_bf16_v(v, q), ok ? off + 16u * q : kDmaOob, rsrc);
    }
    return 4;
  }
  // the wavefront's MI x MJ blocks at (i0 + 32 a, j0 + 32 b), through the stage
  template <int MI, int MJ>
  __device__ __forceinline__ int store_tile(const f32x16_t (&acc)[MI][MJ], int i0, int j0, int,
                                            int lane, lds_char_t* st) const {
    static_assert(MI % 2 == 0, "blocks are staged in pairs along i");
#pragma unroll
    for (int b = 0; b < MJ; ++b)
#pragma unroll
      for (int a2 = 0; a2 < MI / 2; ++a2) {
        stage_bf16_pair(st, acc[2 * a2][b], acc[2 * a2 + 1][b], lane);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 8 * r + (lane >> 3), c = lane & 7;
          const int j = j0 + 32 * b + row, i = i0 + 64 * a2 + 8 * c;
          const bool ok = j < j_valid && i < i_valid;
          buf_store_b128(stage_get(st, row, c),
                         ok ? (uint32_t)((int64_t)j * ldc + col(i)) * 2u : kDmaOob, rsrc);
        }
      }
    return MJ * (MI / 2) * 4;
  }
};

template <>
struct DmaEpi<EpiRowF32Split> {
  i32x4_t rsrc;
  int64_t ldc, split_stride;
  int i_valid, j_valid;
  __device__ __forceinline__ DmaEpi(const EpiRowF32Split& e, const GemmArgs& g)
      : rsrc(uniform_rsrc(e.c, (int64_t)g.splits * e.split_stride * 4)), ldc(e.ldc),
        split_stride(e.split_stride), i_valid(e.i_valid), j_valid(e.j_valid) {}
  __device__ __forceinline__ int store_block(int i, int j, int split, int lane,
                                             const f32x16_t& v) const {
    const int il = i + 4 * (lane >> 5);
    const uint32_t off = (uint32_t)((int64_t)split * split_stride + (int64_t)j * ldc + il) * 4u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool ok = j < j_valid && il + 8 * q < i_valid;
      // (a whole-vector bit_cast: bit_cast of single vector elements reads
      // element 0 with this compiler)
      const f32x4_t f = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
      buf_store_b128_partial(__builtin_bit_cast(u32x4_t, f), ok ? off + 32u * q : kDmaOob, rsrc);
    }
    return 4;
  }
  template <int MI, int MJ>
  __device__ __forceinline__ int store_tile(const f32x16_t (&acc)[MI][MJ], int i0, int j0,
                                            int split, int lane, lds_char_t* st) const {
    const int row_w = lane & 31, h4 = 4 * (lane >> 5);
#pragma unroll
    for (int b = 0; b < MJ; ++b)
#pragma unroll
      for (int a = 0; a < MI; ++a) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4_t f = {acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2],
                             acc[a][b][4 * q + 3]};
          stage_put(st, row_w, (8 * q + h4) * 4, __builtin_bit_cast(u32x4_t, f));
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 8 * r + (lane >> 3), c = lane & 7;
          const int j = j0 + 32 * b + row, i = i0 + 32 * a + 4 * c;
          const bool ok = j < j_valid && i < i_valid;
          const uint32_t off =
              (uint32_t)((int64_t)split * split_stride + (int64_t)j * ldc + i) * 4u;
          buf_store_b128_partial(stage_get(st, row, c), ok ? off : kDmaOob, rsrc);
        }
      }
    return MJ * MI * 4;
  }
};

// Value blocks go to the head-major values, logit blocks to the logit rows; a
// block that straddles the two (or, with D not a multiple of 32, several heads)
// issues the value and the logit stores.
template <>
struct DmaEpi<EpiProjectHM> {
  i32x4_t rsrc_v, rsrc_l;
  int H, D, T, Lp, n_logit_end, m_valid;
  __device__ __forceinline__ DmaEpi(const EpiProjectHM& e, const GemmArgs&)
      : rsrc_v(uniform_rsrc(e.values, (int64_t)e.m_valid * e.H * e.D * 2)),
        rsrc_l(uniform_rsrc(e.logits, (int64_t)e.m_valid * e.Lp * 2)), H(e.H), D(e.D), T(e.T),
        Lp(e.Lp), n_logit_end(e.n_logit_end), m_valid(e.m_valid) {}
  // n: wave-uniform first feature of the block; m: this lane's token
  __device__ __forceinline__ int store_block(int n, int m, int, int lane,
                                             const f32x16_t& v) const {
    const int HD = H * D;
    const bool mok = m < m_valid;
    const int b = m / T, t = m - b * T;
    const int nl = n + 4 * (lane >> 5);
    if (D % 32 == 0 && n + 32 <= HD) {
      const int h = n / D;
      const uint32_t off =
          (uint32_t)(((((int64_t)b * H + h) * T + t) * D) + (nl - h * D)) * 2u;
#pragma unroll
      for (int q = 0; q < 4; ++q) buf_store_b64(pack4_bf16_v(v, q), mok ? off + 16u * q : kDmaOob, rsrc_v);
      return 4;
    }
    int count = 0;
    if (n < HD) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nq = nl + 8 * q;
        const int h = nq / D, d = nq - h * D;
        const bool ok = mok && nq < HD;
        const uint32_t off = (uint32_t)((((int64_t)b * H + h) * T + t) * D + d) * 2u;
        buf_store_b64(pack4_bf16_v(v, q), ok ? off : kDmaOob, rsrc_v);
      }
      count += 4;
    }
    if (n + 32 > HD && n < n_logit_end) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nq = nl + 8 * q;
        const bool ok = mok && nq >= HD && nq < n_logit_end;
        const uint32_t off = (uint32_t)((int64_t)m * Lp + (nq - HD)) * 2u;
        buf_store_b64(pack4_bf16_v(v, q), ok ? off : kDmaOob, rsrc_l);
      }
      count += 4;
    }
    return count;
  }
  // value blocks in pairs inside one head go through the stage (one token's 64
  // channels = 128 contiguous bytes of values); other pairs use store_block
  template <int MI, int MJ>
  __device__ __forceinline__ int store_tile(const f32x16_t (&acc)[MI][MJ], int i0, int j0,
                                            int split, int lane, lds_char_t* st) const {
    static_assert(MI % 2 == 0, "blocks are staged in pairs along i");
    const int HD = H * D;
    int count = 0;
#pragma unroll
    for (int b = 0; b < MJ; ++b)
#pragma unroll
      for (int a2 = 0; a2 < MI / 2; ++a2) {
        const int n0 = i0 + 64 * a2;
        if (D % 64 == 0 && n0 + 64 <= HD) {
          stage_bf16_pair(st, acc[2 * a2][b], acc[2 * a2 + 1][b], lane);
          const int h = n0 / D, d0 = n0 - h * D;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = 8 * r + (lane >> 3), c = lane & 7;
            const int m = j0 + 32 * b + row;
            const int bb = m / T, t = m - bb * T;
            const uint32_t off =
                (uint32_t)((((int64_t)bb * H + h) * T + t) * D + d0 + 8 * c) * 2u;
            buf_store_b128(stage_get(st, row, c), m < m_valid ? off : kDmaOob, rsrc_v);
          }
          count += 4;
        } else {
          const int m = j0 + 32 * b + (lane & 31);
          count += store_block(n0, m, split, lane, acc[2 * a2][b]);
          count += store_block(n0 + 32, m, split, lane, acc[2 * a2 + 1][b]);
        }
      }
    return count;
  }
};

// MFMA operand fragment (8 consecutive k of one row) for k16 sub-step ks (0..3)
// of a stage.
template <int R, int L>
__device__ __forceinline__ bf16x8_t dma_read_frag(const bf16_t* stage, int row_base, int ks,
                                                  int lane) {
  typedef __attribute__((address_space(3))) const char lds_char;
  lds_char* base = (lds_char*)stage;
  if (L == OP_KC) {
    const int r = row_base + (lane & 31);
    const int c = 2 * ks + (lane >> 5);
    const u32x4_t q = *(__attribute__((address_space(3))) const u32x4_t*)(
        base + r * kDmaRowBytes + (dma_kc_slot(r, c) << 4));
    return __builtin_bit_cast(bf16x8_t, q);
  } else {
    const int g = lane >> 4, s = lane & 15;
    const int row = row_base + (g & 1) * 16 + 4 * (s & 3);
    const int k = ks * 16 + (g >> 1) * 8 + (s >> 2);
    const int c = row >> 3, within = (row & 7) * 2;
    typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
    lds_char* p0 = base + k * (R * 2) + ((c ^ (4 * (k & 3))) << 4) + within;
    lds_char* p1 = p0 + 4 * (R * 2);  // k + 4: same swizzle (k & 3 unchanged)
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p0);
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p1);
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    const i16x8_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8_t, v);
  }
}

// Work items of a persistent launch: item k of this workgroup is
// blockIdx.x + k gridDim.x of the (tile, split) items, XCD-contiguous.
template <int BI, int BJ>
struct GridItems {
  __device__ __forceinline__ void decode(const GemmArgs& g, GemmCursor& c) const {
    gemm_decode<BI, BJ>(g, c);
  }
};

// LDS of one direct-to-LDS GEMM workgroup: NST stages of each operand tile and
// a per-wavefront epilogue staging area (the launches declare it once and may
// run several GEMMs through it one after another).
template <int BI, int BJ, int NW>
struct DmaLds {
  static constexpr int kPB = BI * kDmaBK * 2, kQB = BJ * kDmaBK * 2;  // stage bytes per operand
  __attribute__((aligned(1024))) bf16_t p[kDmaStages][kPB / 2];
  __attribute__((aligned(1024))) bf16_t q[kDmaStages][kQB / 2];
  __attribute__((aligned(16))) char epi[NW][kEpiStageBytes];
};

// Persistent over (tile, split) work items like gemm_bf16_kernel, stepping the
// reduction in kDmaBK slices through two LDS stages; the items are those
// Items::decode gives this workgroup, in order.
template <int BI, int BJ, int WGI, int WGJ, int PL, int QL, class Epi, class Items>
__device__ __forceinline__ void gemm_dma_run(const GemmArgs& g, const Epi& epi, const Items& items,
                                             DmaLds<BI, BJ, WGI * WGJ>& lds) {
  constexpr int NW = WGI * WGJ;
  constexpr int WI = BI / WGI, WJ = BJ / WGJ;
  constexpr int MI = WI / 32, MJ = WJ / 32;
  static_assert(MI >= 1 && MJ >= 1 && WI % 32 == 0 && WJ % 32 == 0, "bad wave tile");
  constexpr int PB = BI * kDmaBK * 2, QB = BJ * kDmaBK * 2;  // stage bytes per operand
  constexpr int KS = kDmaBK / 16;                             // MFMA k16 sub-steps per step
  // The loads are issued by the last NWL wavefronts only (with 8 wavefronts,
  // one per SIMD).  A wavefront that issues a burst of direct-to-LDS loads
  // stalls until the texture unit has taken them, and cannot issue MFMAs
  // meanwhile; the other wavefront of its SIMD, which issues none, keeps the
  // matrix core busy.  Measured on MI355X at the d12 forward shape: 123 ->
  // 110 us (with the single-add load offsets) against every wavefront loading.
  constexpr int NWL = NW >= 2 ? NW / 2 : 1;
  using OpP = DmaOperand<BI, PL, NWL>;
  using OpQ = DmaOperand<BJ, QL, NWL>;

  constexpr int NST = kDmaStages;
  constexpr int kLoads = OpP::kPerWave + OpQ::kPerWave;  // vm instructions per k-step
  static_assert(PB == DmaLds<BI, BJ, NW>::kPB && QB == DmaLds<BI, BJ, NW>::kQB, "stage sizes");
  auto& lds_p = lds.p;
  auto& lds_q = lds.q;
  auto& lds_epi = lds.epi;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wi = wave % WGI, wj = wave / WGI;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wi_u = wave_u % WGI, wj_u = wave_u / WGI;

  f32x16_t acc[MI][MJ];
#pragma unroll
  for (int a = 0; a < MI; ++a)
#pragma unroll
    for (int b = 0; b < MJ; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

  OpP op_p;
  OpQ op_q;

  // cursors count k-steps of kDmaBK; reuse GemmCursor with nk in those units
  auto decode = [&](GemmCursor& c) {
    items.decode(g, c);
    if (c.valid) c.nk = (c.ke - c.kb + kDmaBK - 1) / kDmaBK;
  };
  auto advance = [&](GemmCursor& c) {
    if (++c.kt >= c.nk) {
      ++c.k;
      decode(c);
    }
  };
  const bool loader = wave_u >= NW - NWL;
  const int lw = wave_u - (NW - NWL);  // index among the loaders
  const int my_loads = loader ? kLoads : 0;
  auto issue = [&](const GemmCursor& c, int stage) {
    if (!loader) return;
    if (c.kt == 0) {
      op_p.setup(g.P, g.K, c.i0, c.ke, lw, lane);
      op_q.setup(g.Q, g.K, c.j0, c.ke, lw, lane);
    }
    const int k0 = c.kb + c.kt * kDmaBK;
    op_p.issue(lds_addr(&lds_p[stage][0]), k0, lw);
    op_q.issue(lds_addr(&lds_q[stage][0]), k0, lw);
  };

  GemmCursor lc, cc;
  lc.k = 0;
  decode(lc);
  cc = lc;
  if (!cc.valid) return;
  const DmaEpi<Epi> de(epi, g);
  // vmcnt bookkeeping over the last NST - 1 steps j (oldest first): st[] the
  // store instructions of step j's epilogue, tot[] everything step j issued
  // (the loads of step j + NST - 1, then those stores).  The prologue's loads of
  // steps 0 .. NST - 2 count as issued in steps 1 - NST .. -1.
  int st[NST - 1], tot[NST - 1];
#pragma unroll
  for (int i = 0; i < NST - 1; ++i) {
    st[i] = 0;
    tot[i] = 0;
    if (lc.valid) {
      issue(lc, i);
      advance(lc);
      tot[i] = my_loads;
    }
  }
  // instructions younger than the loads of step k + 1, at the end of step k
  auto younger = [&]() {
    int n = st[0];
#pragma unroll
    for (int i = 1; i < NST - 1; ++i) n += tot[i];
    return n;
  };
  wait_vmcnt_rt(younger());  // step 0 (nothing stored yet: st[0] = 0)
  __builtin_amdgcn_s_barrier();
  lds_fence();

  // Rotated k-step loop.  A step's last k16 sub-step runs after the barrier
  // that ends the step -- its fragments are in registers by then -- so its
  // MFMAs cover the barrier skew and the next step's first fragment reads
  // (the stage that barrier frees is refilled at the same time).  One pass:
  //   loads of step k + NST - 1; sub-step 0 reads of step k, with the last
  //   sub-step's MFMAs of step k - 1; the epilogue if step k - 1 ended a tile;
  //   sub-steps 0 .. KS - 2 of step k, reading sub-step t + 1 during t;
  //   wait for the loads of step k + 1; barrier.
  // The rotation keeps a sub-step's fragments live across the barrier and the
  // next step's load set-up; with row-contiguous operands (two reads and more
  // addresses per fragment) that exceeds the 256 registers of two wavefronts
  // per SIMD, and those kernels keep the plain loop below.
  constexpr bool kRotate = PL == OP_KC && QL == OP_KC;
  static_assert(KS % 2 == 0, "the last sub-step must use fragment set 1");
  constexpr int RD = MI * (PL == OP_KC ? 1 : 2) + MJ * (QL == OP_KC ? 1 : 2);  // LDS reads per sub-step
  constexpr int NM = MI * MJ;
  bf16x8_t fp[2][MI], fq[2][MJ];
  auto read_sub = [&](auto setc, int stg, int t) {
    constexpr int set = decltype(setc)::value;
    const bf16_t* sp = &lds_p[stg][0];
    const bf16_t* sq = &lds_q[stg][0];
#pragma unroll
    for (int a = 0; a < MI; ++a) fp[set][a] = dma_read_frag<BI, PL>(sp, wi * WI + a * 32, t, lane);
#pragma unroll
    for (int b = 0; b < MJ; ++b) fq[set][b] = dma_read_frag<BJ, QL>(sq, wj * WJ + b * 32, t, lane);
  };
  auto mfma_sub = [&](auto setc) {
    constexpr int set = decltype(setc)::value;
#pragma unroll
    for (int a = 0; a < MI; ++a)
#pragma unroll
      for (int b = 0; b < MJ; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fp[set][a], fq[set][b], acc[a][b], 0, 0, 0);
  };
  // Left to itself the scheduler issues each read right before the MFMA that
  // consumes it, and every MFMA group then waits for the LDS: one MFMA, then
  // its share of the reads, for each MFMA of a sub-step.
  auto interleave = [&]() {
    static_for<NM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr int n = RD / NM + (i < RD % NM ? 1 : 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x100, n, 0);
    });
  };
  auto record = [&](int loads, int stores) {
#pragma unroll
    for (int i = 0; i < NST - 2; ++i) {
      st[i] = st[i + 1];
      tot[i] = tot[i + 1];
    }
    st[NST - 2] = stores;
    tot[NST - 2] = loads + stores;
  };

  auto wait_next = [&]() {
    const int n = younger();
    if (n == 0)
      wait_vmcnt<0>();
    else
      wait_vmcnt_rt(n);
  };
  auto epilogue = [&](int ti0, int tj0, int tsplit) {
    const int stores = de.template store_tile<MI, MJ>(acc, ti0 + wi_u * WI, tj0 + wj_u * WJ, tsplit,
                                                      lane, (lds_char_t*)&lds_epi[wave_u][0]);
#pragma unroll
    for (int a = 0; a < MI; ++a)
#pragma unroll
      for (int b = 0; b < MJ; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
    return stores;
  };

  int stage = 0;
  if constexpr (!kRotate) {
    while (cc.valid) {
      // the stage of step k + NST - 1 was last read in step k - 1, which every
      // wavefront has finished (barrier below): refill it
      int loads = 0;
      if (lc.valid) {
        issue(lc, stage == 0 ? NST - 1 : stage - 1);
        advance(lc);
        loads = my_loads;
      }
      // the first sub-step's reads, then in each sub-step the next one's reads
      // spread between its MFMAs
      read_sub(std::integral_constant<int, 0>{}, stage, 0);
      static_for<KS>([&](auto tc) {
        constexpr int t = decltype(tc)::value;
        if constexpr (t + 1 < KS) read_sub(std::integral_constant<int, (t + 1) & 1>{}, stage, t + 1);
        mfma_sub(std::integral_constant<int, t & 1>{});
      });
      __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
      static_for<KS - 1>([&](auto) { interleave(); });
      static_for<NM>([&](auto) { __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); });
      int stores = 0;
      if (cc.kt == cc.nk - 1) stores = epilogue(cc.i0, cc.j0, cc.split);
      advance(cc);
      record(loads, stores);
      // the next step's loads have landed
      if (cc.valid) wait_next();
      __builtin_amdgcn_s_barrier();
      lds_fence();
      stage = stage == NST - 1 ? 0 : stage + 1;
    }
    wait_vmcnt<0>();
    return;
  }
  {
    int loads = 0;
    if (lc.valid) {
      issue(lc, NST - 1);
      advance(lc);
      loads = my_loads;
    }
    record(loads, 0);
  }
  read_sub(std::integral_constant<int, 0>{}, 0, 0);
  while (true) {
    static_for<KS - 1>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      read_sub(std::integral_constant<int, (t + 1) & 1>{}, stage, t + 1);
      mfma_sub(std::integral_constant<int, t & 1>{});
    });
    static_for<KS - 1>([&](auto) { interleave(); });
    const bool tile_end = cc.kt == cc.nk - 1;
    const int ti0 = cc.i0, tj0 = cc.j0, tsplit = cc.split;
    advance(cc);
    // every fragment read of this stage is done before the barrier lets the
    // stage be refilled, and the next step's loads have landed (instructions
    // issued after them: the previous epilogue's stores, if any)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (cc.valid) wait_next();
    __builtin_amdgcn_s_barrier();
    lds_fence();
    stage = stage == NST - 1 ? 0 : stage + 1;
    int loads = 0;
    if (lc.valid) {
      issue(lc, stage == 0 ? NST - 1 : stage - 1);
      advance(lc);
      loads = my_loads;
    }
    // after the last step the reads fetch stale stage data, never used
    read_sub(std::integral_constant<int, 0>{}, stage, 0);
    mfma_sub(std::integral_constant<int, 1>{});
    interleave();
    int stores = 0;
    if (tile_end) stores = epilogue(ti0, tj0, tsplit);
    record(loads, stores);
    if (!cc.valid) break;
  }
  wait_vmcnt<0>();
}

template <int BI, int BJ, int WGI, int WGJ, int PL, int QL, class Epi>
__global__ void __launch_bounds__(WGI * WGJ * 64)
gemm_dma_kernel(const GemmArgs g, const Epi epi) {
  __shared__ DmaLds<BI, BJ, WGI * WGJ> lds;
  gemm_dma_run<BI, BJ, WGI, WGJ, PL, QL>(g, epi, GridItems<BI, BJ>{}, lds);
}

// ---------------------------------------------------------------------------
// The projection backward's two GEMMs in one persistent launch.  When grad_x's
// tiles do not fill their last round of the grid (384 tiles on 256 CUs at
// d12, 192 at B = 16), workgroups [n_late, G) sit idle while [0, n_late) run
// their last tile.  Here every workgroup runs its grad_x tiles and then one
// piece of grad_weight's split reduction, the workgroups that finished grad_x
// a tile earlier taking the longer pieces:
// each of grad_weight's nt output tiles keeps S partial slots (the layout
// dw_reduce4_kernel sums), filled by e "early" pieces of a k-steps followed by
// S - e "late" pieces of b = a - delta k-steps, the last of which ends the
// reduction.  Tiles [0, x) have e1 early pieces, tiles [x, nt) e2 = e1 - 1, so
// that the early pieces number exactly the early workgroups.
// ---------------------------------------------------------------------------
struct DwPlan {
  int n_late;      // workgroups running one grad_x tile more than the rest
  int nt, S, x;    // grad_weight output tiles, slots per tile, tiles with e1 early pieces
  int e1, a1, b1;  // tiles [0, x): early pieces, their k-steps, late pieces' k-steps
  int e2, a2, b2;  // tiles [x, nt)
  int ksteps;      // k-steps of the whole reduction
};

// Which piece a workgroup takes: the early pieces in (slot, tile) order, and
// likewise the late ones, are dealt to the early (late) workgroups XCD by XCD
// (workgroup b runs on XCD b % 8), so the pieces an XCD holds mostly share
// their k-range and read the same rows of both operands through its L2.
// Measured at d12: 567 MB read from HBM against 808 MB when consecutive
// workgroups take consecutive pieces of one tile (about the same time, 214
// against 213 us), and 238 us when the (slot, tile) order is dealt round the
// XCDs instead.
template <int BI, int BJ>
struct DwPlanItems {
  DwPlan p;
  __device__ __forceinline__ void decode(const GemmArgs& g, GemmCursor& c) const {
    c.valid = false;
    if (c.k != 0) return;  // one piece per workgroup
    const int b = blockIdx.x;
    const int G = gridDim.x;
    const bool xcd = G % 8 == 0 && p.n_late % 8 == 0;
    int t, slot, k0, k1;
    if (b >= p.n_late) {  // early: one grad_x tile fewer before this piece
      const int w = b - p.n_late, n = G - p.n_late;
      const int i = xcd ? (w % 8) * (n / 8) + w / 8 : w;
      int s;
      if (i < p.e2 * p.nt) {
        s = i / p.nt;
        t = i % p.nt;
      } else {
        s = p.e2;
        t = i - p.e2 * p.nt;
        if (t >= p.x) return;
      }
      const int a = t < p.x ? p.a1 : p.a2;
      slot = s;
      k0 = s * a;
      k1 = k0 + a;
    } else {  // late
      const int i = xcd ? (b % 8) * (p.n_late / 8) + b / 8 : b;
      const int l1 = p.S - p.e1;  // late pieces of a tile with e1 early ones (one fewer than e2's)
      int j;
      if (i < l1 * p.nt) {
        j = i / p.nt;
        t = i % p.nt;
      } else {
        j = l1;
        t = p.x + (i - l1 * p.nt);
        if (t >= p.nt) return;
      }
      const bool c1 = t < p.x;
      const int e = c1 ? p.e1 : p.e2, a = c1 ? p.a1 : p.a2, lb = c1 ? p.b1 : p.b2;
      slot = e + j;
      k0 = e * a + j * lb;
      k1 = j == p.S - e - 1 ? p.ksteps : k0 + lb;
    }
    c.valid = true;
    c.i0 = (t % g.tiles_i) * BI;
    c.j0 = (t / g.tiles_i) * BJ;
    c.split = slot;
    c.kb = k0 * kDmaBK;
    c.ke = min(k1 * kDmaBK, g.K);
    c.kt = 0;
  }
};

template <class EpiX, class EpiW>
__global__ void __launch_bounds__(512)
gemm_dma_bwd_fused_kernel(const GemmArgs gx, const EpiX ex, const GemmArgs gw, const EpiW ew,
                          const DwPlan plan) {
  __shared__ DmaLds<256, 256, 8> lds;
  gemm_dma_run<256, 256, 2, 4, OP_RC, OP_KC>(gx, ex, GridItems<256, 256>{}, lds);
  __syncthreads();  // the LDS stages and staging areas are reused
  gemm_dma_run<256, 256, 2, 4, OP_RC, OP_RC>(gw, ew, DwPlanItems<256, 256>{plan}, lds);
}

}  // namespace ltv
