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

#ifdef __cplusplus
}
#endif

#endif /* LTV_PEAKS_H */
