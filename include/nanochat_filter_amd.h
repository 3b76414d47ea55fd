/*
 * nanochat_filter_amd.h -- C ABI of the MI355X (gfx950) LTV combined-QKV
 * filter path: the fused QKV projection and the gated EWMA scan, forward and
 * backward.
 *
 * Conventions for every entry point:
 *   - All tensor arguments are raw device pointers plus element strides
 *     (int64, in elements of the tensor's own dtype).  Shapes are plain ints.
 *     The scan entry points take any batch and head strides; their time and
 *     channel strides must be non-negative (LTV_ERR_UNSUPPORTED otherwise).
 *   - `dtype` selects the I/O element type: LTV_DTYPE_F32 or LTV_DTYPE_BF16
 *     (bf16 as raw 16-bit patterns).  State and arithmetic are always fp32;
 *     `logit_bias` / `grad_logit_bias` are always fp32.
 *   - `stream` is a hipStream_t (NULL = default stream).  Every call only
 *     enqueues work on that stream; none synchronises the host.
 *   - Outputs are caller-allocated; the library never allocates device memory.
 *     Temporary device memory is passed in as `workspace` (size from the
 *     matching *_workspace_size query).
 *   - Return value: LTV_OK, or an LTV_ERR_* code with a message available from
 *     ltv_last_error() (per host thread).
 *
 * Reference interfaces replaced (paths relative to aioaneid/nanochat-filter):
 *   pybind11 module `cpp_ewma_cuda` (cpp_ewma/src/bindings.cpp) functions
 *   ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_{forward,backward}
 *   and fused_linear_transpose{,_backward}, which the torch.library ops in
 *   nanochat/ops/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py
 *   and nanochat/ops/fused_linear_transpose.py call.
 */
#ifndef NANOCHAT_FILTER_AMD_H
#define NANOCHAT_FILTER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LTV_DTYPE_F32 0
#define LTV_DTYPE_BF16 1

#define LTV_OK 0
#define LTV_ERR_INVALID_ARG 1
#define LTV_ERR_UNSUPPORTED 2
#define LTV_ERR_HIP 3
#define LTV_ERR_WORKSPACE 4

/* Version of this ABI (bumped on any signature change or addition): 11. */
int ltv_abi_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* ltv_last_error(void);

/* ------------------------------------------------------------------------
 * Gated EWMA scan, reference layout.
 *
 * combined : (B, T, F) with F = H*(D+Da), H = NH + 2*NKVH, D = Da*r, any
 *            strides; per-head features [values D | logits Da]
 * inits    : (B, H, D), any strides
 * logit_bias: (H, Da) fp32, contiguous
 * out_q    : (B, NH, T, D), out_k / out_v : (B, NKVH, T, D), any strides
 *
 * Replaces ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward
 * (cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward.cu:532-552,
 *  called from nanochat/ops/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py:35-71).
 * The reference's tuning arguments (scan/r threads, r items) are launch
 * shapes of its CUDA kernel and have no counterpart here.
 * ---------------------------------------------------------------------- */
int ltv_hm_scan_forward(int dtype, const void* combined, const int64_t combined_strides[3],
                        const void* inits, const int64_t inits_strides[3],
                        const float* logit_bias, void* out_q, const int64_t out_q_strides[4],
                        void* out_k, const int64_t out_k_strides[4], void* out_v,
                        const int64_t out_v_strides[4], int B, int T, int NH, int NKVH, int Da,
                        int r, int use_sigmoid, void* stream);

/* ------------------------------------------------------------------------
 * ltv_hm_scan_forward with a chain workspace: the same scan and results,
 * computed by workgroups that each own one chunk of T and hand the state at
 * the chunk's end to the next chunk through `chain_workspace` (one pass over
 * HBM, with parallelism over T as well as over (b, head); long sequences at
 * small batch are the case it is for).
 *
 * chain_workspace: 256-byte aligned device memory of at least
 *   ltv_hm_scan_forward_chain_workspace_size(...) bytes, ALL ZERO before the
 *   first call.  Every call leaves it all zero again, so one zeroed buffer
 *   serves all later calls on one stream, in a captured HIP graph too; calls
 *   that overlap in time (other streams) need buffers of their own.
 *   NULL selects the kernel of ltv_hm_scan_forward.  The chained kernel is
 *   used where it is the faster one: fewer than 1,024 (b, head, channel slab)
 *   sequences of at least 8 chunks (T > 3,584; r = 1: T > 1,792), 16-byte
 *   channel vectors, gate groups of whole lanes or r = 1;
 *   elsewhere the size query returns 0 and a workspace passed is not
 *   touched.  (LTV_SCAN_CHAIN_CFG="CL,L,NW" forces it, "0" turns it off.)
 *   Failure: a chunk's wait for its carry is bounded (about a second); past
 *   it, or with a workspace that was not zero at the launch, the kernel still
 *   exits normally, but the outputs of that call are invalid.  It then sets
 *   the workspace's second 32-bit word to the error code (1: a wait ran out,
 *   2: the workspace was not zero) and stores the code into the library's
 *   host mailbox, which ltv_chain_take_error() reads without synchronising
 *   the device.  After an error the workspace must be zeroed again.  (A wait
 *   that runs out leaves no late carry behind: the reader marks the word
 *   abandoned and the late publisher clears it.)
 *
 * Replaces the same reference forward as ltv_hm_scan_forward; the workspace
 * has no counterpart there (the reference walks T serially per block,
 * cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward.cu:157-220).
 * ---------------------------------------------------------------------- */
size_t ltv_hm_scan_forward_chain_workspace_size(int dtype, int B, int T, int NH, int NKVH, int Da,
                                                int r);

int ltv_hm_scan_forward_ws(int dtype, const void* combined, const int64_t combined_strides[3],
                           const void* inits, const int64_t inits_strides[3],
                           const float* logit_bias, void* out_q, const int64_t out_q_strides[4],
                           void* out_k, const int64_t out_k_strides[4], void* out_v,
                           const int64_t out_v_strides[4], void* chain_workspace,
                           size_t chain_workspace_bytes, int B, int T, int NH, int NKVH, int Da,
                           int r, int use_sigmoid, void* stream);

/* ------------------------------------------------------------------------
 * Error mailbox of the chained kernels (ltv_hm_scan_forward_ws,
 * ltv_hm_scan_backward_ws and the look-back *_split_ws variants): returns the
 * error code (1 or 2, see ltv_hm_scan_forward_ws) that a chained launch has
 * reported since the previous call, or 0, and clears it.  Reads mapped host
 * memory: no device synchronisation, so a launch still running is seen by a
 * later call.  Synchronise the stream first to check one call.
 *
 * No reference counterpart: the reference's scans launch no kernel that
 * waits on another workgroup; its launch checks are
 * cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward.cu:452,465,495,504
 * (C10_CUDA_KERNEL_LAUNCH_CHECK), which this library's status codes replace.
 * ---------------------------------------------------------------------- */
int ltv_chain_take_error(void);

/* Test control of the chained kernels' waits, for failure-handling tests that
 * must not hang: spin_max = polls before a wait gives up (0 restores the
 * default bound), no_publish != 0 makes every chained launch publish no carry,
 * so every wait runs out after spin_max polls and every kernel still exits
 * normally.  Applies to launches made after the call.  No reference
 * counterpart. */
int ltv_chain_set_test_controls(int spin_max, int no_publish);

/* Windows per lane of the short-window look-back backward (the kernel behind
 * ltv_hm_look_back_scan_backward[_split] for windows with a warm-up of at most
 * 8 steps shorter than P and Q).  With wpl > 1 a lane walks wpl consecutive
 * windows last to first and hands each one's chain value and warm-up to the
 * window before it, so u and the upstream gradients are read once per step;
 * the results are bitwise those of wpl = 1.  0 (the default) picks the
 * smallest wpl whose wavefronts fit one round of the device.  A tuning and
 * test control, applied to launches made after the call (overrides
 * LTV_SCAN_LB_WPL); returns LTV_ERR_INVALID_ARG for wpl < 0.  No reference
 * counterpart (the reference's look-back kernels take no such parameter:
 * cpp_ewma/src/ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward.cu). */
int ltv_lb_set_windows_per_lane(int wpl);

/* Workspace bytes needed by ltv_hm_scan_backward / ltv_hm_scan_backward_split. */
size_t ltv_hm_scan_backward_workspace_size(int dtype, int B, int T, int NH, int NKVH, int Da,
                                           int r);

/* ------------------------------------------------------------------------
 * Backward of ltv_hm_scan_forward.
 *
 * hq/hk/hv       : the forward outputs (any strides)
 * grad_hq/hk/hv  : upstream gradients, shaped like the outputs (any strides)
 * grad_combined  : (B, T, F), any strides (fully overwritten)
 * grad_inits     : (B, H, D), any strides (overwritten)
 * grad_logit_bias: (H, Da) fp32 contiguous (overwritten, not accumulated)
 * (grad_inits with batch stride 0 and B > 1 receives the sum over the batch,
 *  as described at ltv_hm_look_back_scan_backward_split_ws.)
 *
 * Replaces ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward
 * (cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward.cu:882-976,
 *  called from nanochat/ops/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py:145-193).
 * The reference zero-fills grad_logit_bias and atomically accumulates; this
 * entry point writes it once, deterministically.
 * ---------------------------------------------------------------------- */
int ltv_hm_scan_backward(int dtype, const void* combined, const int64_t combined_strides[3],
                         const void* inits, const int64_t inits_strides[3],
                         const float* logit_bias, const void* hq, const int64_t hq_strides[4],
                         const void* hk, const int64_t hk_strides[4], const void* hv,
                         const int64_t hv_strides[4], const void* grad_hq,
                         const int64_t grad_hq_strides[4], const void* grad_hk,
                         const int64_t grad_hk_strides[4], const void* grad_hv,
                         const int64_t grad_hv_strides[4], void* grad_combined,
                         const int64_t grad_combined_strides[3], void* grad_inits,
                         const int64_t grad_inits_strides[3], float* grad_logit_bias,
                         void* workspace, size_t workspace_bytes, int B, int T, int NH, int NKVH,
                         int Da, int r, int use_sigmoid, void* stream);

/* ------------------------------------------------------------------------
 * ltv_hm_scan_backward with a chain workspace: the same gradients, computed
 * by workgroups that each own one tile-long chunk of T, last chunk first, and
 * hand the gradient carry at the chunk's start to the chunk before it through
 * `chain_workspace` (one pass over HBM, parallel over T as well as over
 * (b, head)).  grad_combined and grad_inits are bitwise those of the
 * unchunked tile kernel with the same steps per lane; grad_logit_bias sums
 * per-chunk partials (a different fp32 association, fixed from call to call).
 *
 * chain_workspace: the contract of ltv_hm_scan_forward_ws's, sized by
 *   ltv_hm_scan_backward_chain_workspace_size(...) (one zeroed buffer can serve
 *   the chained forward and backward on one stream: each call leaves it
 *   zeroed).  NULL selects the kernels of ltv_hm_scan_backward.  The chained
 *   kernel is used below 256 (b, head) sequences with 16-byte channel
 *   vectors, gate groups of whole lanes (at most 16 per head) or r = 1, and
 *   at least two chunks; elsewhere the size query returns 0 and a workspace
 *   passed is not touched.  (LTV_SCAN_BWD_CHAIN_CFG="L,NW" forces it, "0"
 *   turns it off.)  `workspace` is sized by ltv_hm_scan_backward_workspace_size
 *   as before (it covers either kernel's dbias partials).
 *
 * Replaces the same reference backward as ltv_hm_scan_backward; the chain
 * workspace has no counterpart there (the reference walks T serially per
 * block, cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward.cu:882-976).
 * ---------------------------------------------------------------------- */
size_t ltv_hm_scan_backward_chain_workspace_size(int dtype, int B, int T, int NH, int NKVH,
                                                 int Da, int r);

int ltv_hm_scan_backward_ws(int dtype, const void* combined, const int64_t combined_strides[3],
                            const void* inits, const int64_t inits_strides[3],
                            const float* logit_bias, const void* hq, const int64_t hq_strides[4],
                            const void* hk, const int64_t hk_strides[4], const void* hv,
                            const int64_t hv_strides[4], const void* grad_hq,
                            const int64_t grad_hq_strides[4], const void* grad_hk,
                            const int64_t grad_hk_strides[4], const void* grad_hv,
                            const int64_t grad_hv_strides[4], void* grad_combined,
                            const int64_t grad_combined_strides[3], void* grad_inits,
                            const int64_t grad_inits_strides[3], float* grad_logit_bias,
                            void* workspace, size_t workspace_bytes, void* chain_workspace,
                            size_t chain_workspace_bytes, int B, int T, int NH, int NKVH, int Da,
                            int r, int use_sigmoid, void* stream);

/* ------------------------------------------------------------------------
 * Same scan with the value and logit slots given as two separate 4-D views
 * (b, h, t, channel) instead of one interleaved (B, T, F) tensor.  This is
 * the form the projection below writes (values and logits in one row-major
 * (B*T, Fp) buffer, see ltv_qkv_project_forward) and is what the filter
 * module's fast path uses.  Same math and buffer contracts as above.
 * Counterpart in the reference: the same scan entry points (the reference has
 * only the interleaved layout).
 * ---------------------------------------------------------------------- */
int ltv_hm_scan_forward_split(int dtype, const void* values, const int64_t values_strides[4],
                              const void* logits, const int64_t logits_strides[4],
                              const void* inits, const int64_t inits_strides[3],
                              const float* logit_bias, void* out_q,
                              const int64_t out_q_strides[4], void* out_k,
                              const int64_t out_k_strides[4], void* out_v,
                              const int64_t out_v_strides[4], int B, int T, int NH, int NKVH,
                              int Da, int r, int use_sigmoid, void* stream);

int ltv_hm_scan_backward_split(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    const float* logit_bias, const void* hq, const int64_t hq_strides[4], const void* hk,
    const int64_t hk_strides[4], const void* hv, const int64_t hv_strides[4],
    const void* grad_hq, const int64_t grad_hq_strides[4], const void* grad_hk,
    const int64_t grad_hk_strides[4], const void* grad_hv, const int64_t grad_hv_strides[4],
    void* grad_values, const int64_t grad_values_strides[4], void* grad_logits,
    const int64_t grad_logits_strides[4], void* grad_inits, const int64_t grad_inits_strides[3],
    float* grad_logit_bias, void* workspace, size_t workspace_bytes, int B, int T, int NH,
    int NKVH, int Da, int r, int use_sigmoid, void* stream);

/* ------------------------------------------------------------------------
 * Look-back scan: the same recurrence restarted in chunk windows.
 *
 * Chunk 0 covers steps [0, min(P, T)); chunk c >= 1 covers
 * [P + (c - 1) Q, min(P + c Q, T)).  Each chunk [st, hi) runs the recurrence
 * from the inits, starting K - 1 steps early at lo = max(0, st - (K - 1)) (the
 * warm-up), and writes only its own outputs [st, hi).  P >= T is the full
 * recurrence of ltv_hm_scan_forward (the reference passes P = 2147483647,
 * Q = K = 1 for it).  Any P >= 0, Q >= 1, K >= 1 is accepted (the reference's
 * CUDA dispatch builds a fixed list of (P, Q, K)).
 *
 * The backward is the exact gradient of that forward, as autograd gives it for
 * the reference's Python loop (nanochat/ops/ltv_reference_ops.py:37-124): a
 * step inside later chunks' warm-ups receives one contribution per chunk that
 * reads it, and every chunk adds to grad_inits.  Same buffer contracts as
 * ltv_hm_scan_backward; the workspace size depends on P, Q, K.  With several
 * chunk windows and gate groups outside the tile kernel's patterns (r neither a
 * multiple of V -- 8 for bf16, 4 for fp32 -- with Da <= 16, nor dividing V),
 * one thread per channel walks the windows, with two fp32 (B, H, T, D)
 * workspaces more.
 *
 * Replace ltv_look_back_fused_concat_head_major_register_cast_{blelloch,sequential}_scan_cuda_{forward,backward}
 * (cpp_ewma/src/ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward.cu:466-509,
 *  …_blelloch_scan_cuda_backward.cu:809-927 and the sequential pair, called from
 *  nanochat/ops/ltv_cuda_look_back_fused_concat_head_major_register_cast_{blelloch,sequential}_scan.py).
 * The reference's CUDA backward kernels for more than one chunk differ from the
 * autograd of its Python loop (its tests stay at T <= P); this one follows the
 * Python loop.
 * ---------------------------------------------------------------------- */
int ltv_hm_look_back_scan_forward(int dtype, const void* combined,
                                  const int64_t combined_strides[3], const void* inits,
                                  const int64_t inits_strides[3], const float* logit_bias,
                                  void* out_q, const int64_t out_q_strides[4], void* out_k,
                                  const int64_t out_k_strides[4], void* out_v,
                                  const int64_t out_v_strides[4], int B, int T, int NH, int NKVH,
                                  int Da, int r, int P, int Q, int K, int use_sigmoid,
                                  void* stream);

size_t ltv_hm_look_back_scan_backward_workspace_size(int dtype, int B, int T, int NH, int NKVH,
                                                     int Da, int r, int P, int Q, int K);

int ltv_hm_look_back_scan_backward(
    int dtype, const void* combined, const int64_t combined_strides[3], const void* inits,
    const int64_t inits_strides[3], const float* logit_bias, const void* hq,
    const int64_t hq_strides[4], const void* hk, const int64_t hk_strides[4], const void* hv,
    const int64_t hv_strides[4], const void* grad_hq, const int64_t grad_hq_strides[4],
    const void* grad_hk, const int64_t grad_hk_strides[4], const void* grad_hv,
    const int64_t grad_hv_strides[4], void* grad_combined, const int64_t grad_combined_strides[3],
    void* grad_inits, const int64_t grad_inits_strides[3], float* grad_logit_bias,
    void* workspace, size_t workspace_bytes, int B, int T, int NH, int NKVH, int Da, int r, int P,
    int Q, int K, int use_sigmoid, void* stream);

/* Split-layout forms (value and logit slots as two 4-D views, as in
 * ltv_hm_scan_forward_split). */
int ltv_hm_look_back_scan_forward_split(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    const float* logit_bias, void* out_q, const int64_t out_q_strides[4], void* out_k,
    const int64_t out_k_strides[4], void* out_v, const int64_t out_v_strides[4], int B, int T,
    int NH, int NKVH, int Da, int r, int P, int Q, int K, int use_sigmoid, void* stream);

/* ltv_hm_look_back_scan_forward_split with the chain workspace of
 * ltv_hm_scan_forward_ws (same contract), used when there is one window (P >= T);
 * with several windows the workspace is not touched.
 * inits_dtype: the dtype of `inits` -- `dtype`, or LTV_DTYPE_F32 with bf16
 *   values: fp32 inits (the parameter itself, e.g. (H, D) with batch stride 0)
 *   rounded to bf16 when read, exactly the reference's
 *   `init_param.expand(B, H, D).to(bfloat16)` before its kernel, without the
 *   cast's copy.  The fp32 form needs the full recurrence (P >= T), or
 *   look-back windows the short-window kernels take (Q <= 64, warm-up
 *   K - 1 <= min(Q, 16), gate groups of 8 x 2^k channels or dividing 8). */
int ltv_hm_look_back_scan_forward_split_ws(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    int inits_dtype, const float* logit_bias, void* out_q, const int64_t out_q_strides[4],
    void* out_k,
    const int64_t out_k_strides[4], void* out_v, const int64_t out_v_strides[4],
    void* chain_workspace, size_t chain_workspace_bytes, int B, int T, int NH, int NKVH, int Da,
    int r, int P, int Q, int K, int use_sigmoid, void* stream);

int ltv_hm_look_back_scan_backward_split(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    const float* logit_bias, const void* hq, const int64_t hq_strides[4], const void* hk,
    const int64_t hk_strides[4], const void* hv, const int64_t hv_strides[4],
    const void* grad_hq, const int64_t grad_hq_strides[4], const void* grad_hk,
    const int64_t grad_hk_strides[4], const void* grad_hv, const int64_t grad_hv_strides[4],
    void* grad_values, const int64_t grad_values_strides[4], void* grad_logits,
    const int64_t grad_logits_strides[4], void* grad_inits, const int64_t grad_inits_strides[3],
    float* grad_logit_bias, void* workspace, size_t workspace_bytes, int B, int T, int NH,
    int NKVH, int Da, int r, int P, int Q, int K, int use_sigmoid, void* stream);

/* ltv_hm_look_back_scan_backward_split with the chain workspace of
 * ltv_hm_scan_backward_ws (same contract), used when there is one window
 * (P >= T); with several windows the chain workspace is not touched.
 * inits_dtype: as in ltv_hm_look_back_scan_forward_split_ws; grad_inits has
 *   the same dtype.  With fp32 inits and bf16 values each sequence's inits
 *   gradient is the bf16 value widened to fp32 (the cast's backward).
 * grad_inits with batch stride 0 (e.g. the (H, D) parameter's gradient):
 *   receives the sum over the batch -- each sequence's gradient rounded to
 *   the values' dtype, summed in fp32 in batch order, stored in inits_dtype --
 *   which is what the broadcast's backward computes (the reference sums the
 *   expanded inits' gradient over B).  Needs the full recurrence and gate
 *   groups the tile kernels take (r a multiple of 8 bf16 / 4 fp32 channels
 *   with Da <= 16, or r dividing it), or look-back windows the short-window
 *   kernels take (as for fp32 inits); the sum is formed by the launch that
 *   reduces grad_logit_bias, in `workspace`.
 * grad_logits_pad: 0 .. 64 logit slots past the last head's last gate that
 *   are set to zero in every (b, t) row, slot q = H Da + p at
 *   b s0 + t s2 + q s3 of the grad_logits view (needs s1 = Da s3): the
 *   padding columns F .. round_up(F, 8) - 1 of a (B T, Fp) grad_combined,
 *   which ltv_qkv_project_backward_input_zero_padded then need not zero. */
int ltv_hm_look_back_scan_backward_split_ws(
    int dtype, const void* values, const int64_t values_strides[4], const void* logits,
    const int64_t logits_strides[4], const void* inits, const int64_t inits_strides[3],
    int inits_dtype, const float* logit_bias, const void* hq, const int64_t hq_strides[4],
    const void* hk,
    const int64_t hk_strides[4], const void* hv, const int64_t hv_strides[4],
    const void* grad_hq, const int64_t grad_hq_strides[4], const void* grad_hk,
    const int64_t grad_hk_strides[4], const void* grad_hv, const int64_t grad_hv_strides[4],
    void* grad_values, const int64_t grad_values_strides[4], void* grad_logits,
    const int64_t grad_logits_strides[4], int grad_logits_pad, void* grad_inits,
    const int64_t grad_inits_strides[3], float* grad_logit_bias, void* workspace,
    size_t workspace_bytes, void* chain_workspace, size_t chain_workspace_bytes, int B, int T,
    int NH, int NKVH, int Da, int r, int P, int Q, int K, int use_sigmoid, void* stream);

/* ------------------------------------------------------------------------
 * Projection, reference layout: out[b] (F x T) = weight (F x K) . x[b]^T
 *
 * x (B, T, K), weight (F, K), out (B, F, T): all contiguous, all `dtype`.
 * bf16 with T a multiple of 256 and K of 8 (16-byte aligned buffers) runs on
 * bf16 MFMA (fp32 accumulation) and writes the (B, F, T) layout directly; fp32
 * and the other bf16 shapes run on fp32 MFMA (v_mfma_f32_32x32x2_f32, fp32
 * accumulation, any sizes and alignment).  x and weight may be NULL when
 * K = 0 (out is then zeros).
 * Replaces fused_linear_transpose (cpp_ewma/src/fused_linear_transpose_forward.cu:23-58,
 * called from nanochat/ops/fused_linear_transpose.py:20-40).
 * ---------------------------------------------------------------------- */
int ltv_linear_transpose_forward(int dtype, const void* x, const void* weight, void* out, int B,
                                 int T, int K, int F, void* stream);

/* Backward: grad_x (B, T, K) = grad_out^T-mapped . weight,
 * grad_weight (F, K) = sum_b grad_out[b] . x[b]  (both overwritten, in
 * `dtype`, fp32 accumulation).
 * grad_out is (B, F, T) contiguous, or its (B, T, F)-contiguous transpose
 * when grad_out_is_btf != 0 (the two layouts the reference accepts,
 * nanochat/ops/fused_linear_transpose.py:76-84).  Runs on fp32 MFMA, the
 * weight gradient in one pass per output tile.  Pointers of tensors with no
 * elements may be NULL.
 * Replaces fused_linear_transpose_backward
 * (cpp_ewma/src/fused_linear_transpose_backward.cu:22-132). */
int ltv_linear_transpose_backward(int dtype, const void* x, const void* weight,
                                  const void* grad_out, int grad_out_is_btf, void* grad_x,
                                  void* grad_weight, int B, int T, int K, int F, void* stream);

/* The same backward with a workspace for grad_weight's reduction over B T,
 * split into fp32 partials summed in a fixed order (deterministic): bf16 with
 * grad_out (B, F, T) contiguous, T a multiple of 256 and K of 8 (16-byte
 * aligned buffers) runs both GEMMs on bf16 MFMA; every other case on fp32
 * MFMA, its weight gradient split when the workspace holds
 * ltv_linear_transpose_backward_workspace_size bytes (0: no split, and the
 * workspace may be NULL).
 * Same contract and counterpart as ltv_linear_transpose_backward. */
size_t ltv_linear_transpose_backward_workspace_size(int dtype, int B, int T, int K, int F,
                                                    int grad_out_is_btf);
int ltv_linear_transpose_backward_ws(int dtype, const void* x, const void* weight,
                                     const void* grad_out, int grad_out_is_btf, void* grad_x,
                                     void* grad_weight, void* workspace, size_t workspace_bytes,
                                     int B, int T, int K, int F, void* stream);

/* ------------------------------------------------------------------------
 * Fused QKV projection for the filter module (bf16 MFMA, fp32 accumulate).
 *
 * The parameter c.weight is (F, C) with per-head interleaved rows
 * [h0 values (D) | h0 logits (Da) | h1 values | ...], F = H (D + Da)
 * (nanochat/ltv_combined_head_major_qkv_filter.py:11-66).
 *
 * ltv_qkv_packed_width(H, D, Da) = Fp: F rounded up to a multiple of 128.
 * ltv_qkv_logit_width(H, Da)     = Lp: H Da rounded up to a multiple of 8.
 *
 * ltv_qkv_pack_weight: weight (F, C) fp32 or bf16 contiguous ->
 *   wpack (Fp, C) bf16: rows [all values, head-major | all logits | zeros].
 *
 * ltv_qkv_project_forward: x (B T, C) bf16 contiguous ->
 *   values (B, H, T, D) bf16 contiguous (head-major: what the scan reads) and
 *   logits (B T, Lp) bf16 contiguous (column h Da + j = logit j of head h;
 *   columns >= H Da are written as zeros).  One kernel launch.
 *
 * ltv_qkv_project_backward: grad_combined (B T, Fp) bf16 row-major with column
 *   h D + d = gradient of value channel d of head h and column H D + h Da + j =
 *   gradient of logit j (columns >= F are scratch: their values are ignored and
 *   the grad_x computation may overwrite columns F .. round_up(F, 8) - 1 with
 *   zeros, since it reads grad_combined in 8-column chunks) ->
 *   grad_x (B T, C) bf16 and grad_weight (F, C) fp32 in the parameter's
 *   interleaved row order (both overwritten; deterministic).
 * Counterpart in the reference: fused_linear_transpose forward/backward as used
 * by nanochat/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter.py:35-41
 * (there the output is (B, F, T) and the scan reads it through a transposed view).
 * ---------------------------------------------------------------------- */
int ltv_qkv_packed_width(int H, int D, int Da);
int ltv_qkv_logit_width(int H, int Da);
int ltv_qkv_pack_weight(int weight_dtype, const void* weight, void* wpack, int H, int D,
                        int Da, int C, void* stream);
int ltv_qkv_project_forward(const void* x, const void* wpack, void* values, void* logits, int B,
                            int T, int C, int H, int D, int Da, void* stream);
size_t ltv_qkv_project_backward_workspace_size(int M, int C, int H, int D, int Da);
int ltv_qkv_project_backward(const void* x, const void* wpack, void* grad_combined,
                             void* grad_x, float* grad_weight, void* workspace,
                             size_t workspace_bytes, int M, int C, int H, int D, int Da,
                             void* stream);
/* ltv_qkv_project_backward for a grad_combined whose columns
 * F .. round_up(F, 8) - 1 are zero already (as for
 * ltv_qkv_project_backward_input_zero_padded): grad_combined is only read.
 * Both combined calls run grad_x and grad_weight's GEMM in one launch where
 * grad_x's 256 x 256 tiles do not fill their last round of the device's
 * compute units (d12: 384 tiles on 256; B = 16: 192): the compute units with
 * one grad_x tile fewer take longer pieces of grad_weight's split reduction
 * (LTV_GEMM_BWD_FUSED=0 runs the two GEMMs one after the other).  grad_x is bitwise that of ltv_qkv_project_backward_input;
 * grad_weight sums the same products in fp32 over other split boundaries.
 * Counterpart in the reference: fused_linear_transpose_backward.cu:22-132
 * (both gradients of one call). */
int ltv_qkv_project_backward_zero_padded(const void* x, const void* wpack,
                                         const void* grad_combined, void* grad_x,
                                         float* grad_weight, void* workspace,
                                         size_t workspace_bytes, int M, int C, int H, int D,
                                         int Da, void* stream);
/* The two halves of ltv_qkv_project_backward, as separate calls: grad_x
 * (one GEMM launch) and grad_weight (split-K GEMM plus a fixed-order reduction;
 * needs the workspace).  They mirror the grad_x and grad_weight loops of
 * cpp_ewma/src/fused_linear_transpose_backward.cu:67-94 and :96-131. */
int ltv_qkv_project_backward_input(const void* x, const void* wpack, void* grad_combined,
                                   void* grad_x, int M, int C, int H, int D, int Da,
                                   void* stream);
/* ltv_qkv_project_backward_input for a grad_combined whose columns
 * F .. round_up(F, 8) - 1 are zero already (the scan backward writes them
 * with grad_logits_pad = round_up(F, 8) - F): the same grad_x, without the
 * launch that zeroes them, and grad_combined is only read.  Counterpart in
 * the reference: the same grad_x GEMM (fused_linear_transpose_backward.cu:67-95). */
int ltv_qkv_project_backward_input_zero_padded(const void* x, const void* wpack,
                                               const void* grad_combined, void* grad_x, int M,
                                               int C, int H, int D, int Da, void* stream);
int ltv_qkv_project_backward_weight(const void* x, const void* grad_combined,
                                    float* grad_weight, void* workspace, size_t workspace_bytes,
                                    int M, int C, int H, int D, int Da, void* stream);

/* ----------------------------------------------------------------------
 * Decode (T = 1), fused: one launch computes the projection of the B new
 * tokens and one step of the recurrence from each head's previous output row.
 *   x          : (B, C) bf16, rows x_row_stride elements apart (a multiple of 8)
 *   wpack      : the packed bf16 weight from ltv_qkv_pack_weight
 *   prev_q/k/v : previous output rows (B, NH, D), (B, NKVH, D), (B, NKVH, D) bf16,
 *                channel stride 1; prev_strides = {q_b, q_h, k_b, k_h, v_b, v_h}
 *   logit_bias : (H, Da) fp32;  out : (B, H, D) bf16 contiguous (overwritten)
 * The values and gate logits are rounded to bf16 exactly where the projection
 * stores them, and the step is the scan's h + alpha (u - h), so a decode step
 * matches the same step of a full recompute up to fp32 summation order in the
 * projection.  Requires C % 16 == 0.
 * Counterpart in the reference: its decode runs the general filter forward
 * with T = 1 (nanochat/ltv_cuda_fused_concat_head_major_register_cast_blelloch_
 * scan_qkv_filter.py:24-73) on the KV cache's last rows
 * (nanochat/ltv_combined_qkv_computer_module.py:28-41).
 * ---------------------------------------------------------------------- */
int ltv_qkv_decode_step(const void* x, int64_t x_row_stride, const void* wpack,
                        const void* prev_q, const void* prev_k, const void* prev_v,
                        const int64_t prev_strides[6], const float* logit_bias, void* out, int B,
                        int C, int NH, int NKVH, int D, int Da, int use_sigmoid, void* stream);

/* ltv_qkv_decode_step that also stores the new rows to rows_q/k/v (shaped
 * like prev_q/k/v, channel stride 1; rows_strides as prev_strides) -- e.g. the
 * KV cache's last-row buffers, which may be the prev rows themselves: every
 * previous element is read before it is overwritten, by the thread that
 * writes it.  `out` is written as well.  Counterpart in the reference: the
 * decode step above followed by the computer module's copy of the last
 * output rows into the cache (nanochat/ltv_combined_qkv_computer_module.py:28-41,
 * nanochat/kv_cache.py:212), done by the kernel's stores. */
int ltv_qkv_decode_step_rows(const void* x, int64_t x_row_stride, const void* wpack,
                             void* prev_q, void* prev_k, void* prev_v,
                             const int64_t prev_strides[6], const float* logit_bias, void* out,
                             void* rows_q, void* rows_k, void* rows_v,
                             const int64_t rows_strides[6], int B, int C, int NH, int NKVH, int D,
                             int Da, int use_sigmoid, void* stream);

/* ----------------------------------------------------------------------
 * Allocation-free form of ltv_hm_scan_backward: the same arguments without
 * the workspace, the same kernels and results (bitwise).  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It calls no hipMalloc/hipFree and no allocating library
 * routine; the workspace is a device array built into the library, one per
 * GPU, held until the process ends.
 *   Limit: the backward's workspace (ltv_hm_scan_backward_workspace_size) must
 *   fit in ltv_hm_scan_backward_noalloc_max_workspace() bytes (32 MiB: d12,
 *   B = 8 x T = 8192 prefill and smaller fit); larger shapes get
 *   LTV_ERR_WORKSPACE.
 *   Concurrency: every call on one GPU shares that GPU's array, so calls that
 *   overlap on one GPU (other streams, other host threads) race; calls in
 *   one stream are ordered.  The stream must belong to the current device.
 * ---------------------------------------------------------------------- */
size_t ltv_hm_scan_backward_noalloc_max_workspace(void);
int ltv_hm_scan_backward_noalloc(int dtype, const void* combined,
                                 const int64_t combined_strides[3], const void* inits,
                                 const int64_t inits_strides[3], const float* logit_bias,
                                 const void* hq, const int64_t hq_strides[4], const void* hk,
                                 const int64_t hk_strides[4], const void* hv,
                                 const int64_t hv_strides[4], const void* grad_hq,
                                 const int64_t grad_hq_strides[4], const void* grad_hk,
                                 const int64_t grad_hk_strides[4], const void* grad_hv,
                                 const int64_t grad_hv_strides[4], void* grad_combined,
                                 const int64_t grad_combined_strides[3], void* grad_inits,
                                 const int64_t grad_inits_strides[3], float* grad_logit_bias,
                                 int B, int T, int NH, int NKVH, int Da, int r, int use_sigmoid,
                                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOCHAT_FILTER_AMD_H */
