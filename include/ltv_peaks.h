/* Roofline microbenchmarks of libltv_peaks.so (bench.py --workload peaks).
 *
 * Measurement infrastructure, not part of the filter's C ABI
 * (nanochat_filter_amd.h) and with no counterpart in the reference, whose
 * headline peaks are MI355X's published figures; these measure what the box
 * itself reaches in the access and instruction shapes of this library's
 * kernels.  All pointers are device memory; every call only enqueues work on
 * `stream` and returns 0, or 1 for invalid arguments, 3 for a launch error.
 */
#ifndef LTV_PEAKS_H
#define LTV_PEAKS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* `blocks` workgroups of 4 wavefronts, each wavefront running `iters` rounds
 * (rounded up to a multiple of 4) of 8 independent v_mfma_f32_32x32x16_bf16
 * (32,768 FLOP each); operand bits
 * change from one MFMA to the next, or are all zero with zero_operands != 0.
 * out: blocks * 256 floats (one result per lane, so nothing is dead code). */
int ltv_peak_mfma(float* out, int blocks, int iters, int zero_operands, void* stream);

/* Stream n16 16-byte vectors of each of the `nr` (0..3) source arrays and,
 * with write != 0, write their XOR (nr = 0: a pattern) to `dst` (n16 vectors);
 * a read-only stream (write = 0, nr >= 1) keeps its loads live through a store
 * to dst[0] that happens only if the XOR of everything a thread read equals
 * `never`.  slice16 = 0: grid-stride over the arrays with `blocks` workgroups;
 * slice16 > 0: workgroup w streams vectors [w slice16, (w + 1) slice16)
 * (blocks * slice16 >= n16 required).  nontemporal != 0 marks every load and
 * store streaming. */
int ltv_peak_stream(const void* const* srcs, int nr, void* dst, int write, int nontemporal,
                    int64_t n16, int64_t slice16, int blocks, uint32_t never, void* stream);

/* The projection GEMM's k-step without its epilogue, `steps` steps on each of
 * `blocks` workgroups of 8 wavefronts (one per CU at 256): 64 KB of
 * direct-to-LDS loads per step from `src` (src_bytes a power of two, at least
 * 1 MiB; row offsets wrap inside it) issued one step ahead by 4 wavefronts,
 * 256 v_mfma_f32_32x32x16_bf16 on random bits, fragment reads from LDS, one
 * barrier per step.  mode: 5 loads only, 6 MFMAs only, 7 loads + MFMAs,
 * 30 MFMAs + 3 fragment reads per 4 MFMAs (read one group ahead and XORed
 * into the operands), 31 all three, 58 / 59 as 30 / 31 with the reads going
 * to a sink (no MFMA waits on them), 94 / 95 as 30 / 31 with the reads two
 * groups ahead.  out: blocks * 512 floats. */
int ltv_peak_overlap(const void* src, uint32_t src_bytes, float* out, int blocks, int steps,
                     int mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LTV_PEAKS_H */
