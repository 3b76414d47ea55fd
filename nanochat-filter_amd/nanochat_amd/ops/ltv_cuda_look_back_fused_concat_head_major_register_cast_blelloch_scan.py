"""CUDA-dispatch implementations and autograd of the look-back scan ops.

Behavioural mirror of the reference's
``nanochat/ops/ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan.py``
(forward kernel ``:32-78``, functional op ``:81-152``, backward kernel
``:155-213``, autograd ``:216-318``): same schemas, same buffer ownership
(Python allocates every output; kernels only write), the tuning arguments
validated against the reference's accepted sets.  The work is done by the
gfx950 library through ``ltv_hm_look_back_scan_forward`` /
``ltv_hm_look_back_scan_backward``.

Two differences, both deliberate:
  * any chunking P >= 0, Q >= 1, K >= 1 runs (the reference's CUDA dispatch
    accepts a fixed list of (P, Q, K) and raises for the rest);
  * with more than one chunk window the backward is the exact gradient of the
    forward -- the autograd of the reference's Python loop
    (``nanochat/ops/ltv_reference_ops.py:37-124``), where a step read by later
    chunks' warm-ups collects their contributions.  The reference's CUDA
    backward kernels differ from that loop once T > P (its tests stay at
    T <= P, where the two agree).

The sequential op of the reference
(``ltv_cuda_look_back_fused_concat_head_major_register_cast_sequential_scan.py``)
computes the same function; its implementations are in the sibling module and
share the helpers below.
"""

import torch

from nanochat_amd import _native as N
from nanochat_amd.ops.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan import (
    _check_common,
    _check_tuning,
    _R_ITEMS,
    _R_THREADS,
)


def _s4(t):
    return N.strides(t, 4)


def _check_pqk(P, Q, K):
    if P < 0 or Q < 1 or K < 1:
        raise RuntimeError(f"look-back chunking needs P >= 0, Q >= 1, K >= 1 (P={P} Q={Q} K={K})")


def _check_r_tuning(r_threads, r_items):
    if r_threads not in _R_THREADS:
        raise RuntimeError(f"Unsupported r_threads: {r_threads}")
    if r_items not in _R_ITEMS:
        raise RuntimeError(f"Unsupported r_items: {r_items}")


def run_forward(combined, inits, logit_bias, out_q, out_k, out_v, B, T, NH, NKVH, da, r, P, Q, K,
                use_sigmoid):
    _check_pqk(P, Q, K)
    B_, T_, H, D = _check_common(combined, inits, logit_bias, NH, NKVH, da, r)
    if (B_, T_) != (B, T):
        raise RuntimeError(f"B={B}, T={T} do not match combined.shape={tuple(combined.shape)}")
    rc = N.lib().ltv_hm_look_back_scan_forward(
        N.dtype_code(combined.dtype),
        combined.data_ptr(), N.strides(combined, 3),
        inits.data_ptr(), N.strides(inits, 3),
        logit_bias.data_ptr(),
        out_q.data_ptr(), _s4(out_q),
        out_k.data_ptr(), _s4(out_k),
        out_v.data_ptr(), _s4(out_v),
        B, T, NH, NKVH, da, r, P, Q, K, int(bool(use_sigmoid)),
        N.stream_of(combined),
    )
    N.check(rc, "ltv_hm_look_back_scan_forward")


def run_backward(combined, inits, logit_bias, hq, hk, hv, grad_hq, grad_hk, grad_hv,
                 grad_combined, grad_inits, grad_logit_bias, NH, NKVH, da, r, P, Q, K,
                 use_sigmoid):
    _check_pqk(P, Q, K)
    B, T, H, D = _check_common(combined, inits, logit_bias, NH, NKVH, da, r)
    if grad_logit_bias.dtype != torch.float32 or not grad_logit_bias.is_contiguous():
        raise RuntimeError("grad_logit_bias must be a contiguous float32 tensor")
    dt = N.dtype_code(combined.dtype)
    lib = N.lib()
    ws_bytes = lib.ltv_hm_look_back_scan_backward_workspace_size(dt, B, T, NH, NKVH, da, r,
                                                                 P, Q, K)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=combined.device)
    rc = lib.ltv_hm_look_back_scan_backward(
        dt,
        combined.data_ptr(), N.strides(combined, 3),
        inits.data_ptr(), N.strides(inits, 3),
        logit_bias.data_ptr(),
        hq.data_ptr(), _s4(hq), hk.data_ptr(), _s4(hk), hv.data_ptr(), _s4(hv),
        grad_hq.data_ptr(), _s4(grad_hq), grad_hk.data_ptr(), _s4(grad_hk),
        grad_hv.data_ptr(), _s4(grad_hv),
        grad_combined.data_ptr(), N.strides(grad_combined, 3),
        grad_inits.data_ptr(), N.strides(grad_inits, 3),
        grad_logit_bias.data_ptr(),
        ws.data_ptr(), ws_bytes,
        B, T, NH, NKVH, da, r, P, Q, K, int(bool(use_sigmoid)),
        N.stream_of(combined),
    )
    N.check(rc, "ltv_hm_look_back_scan_backward")


def allocate_outputs(combined, NH, NKVH, da, r):
    B, T, _ = combined.shape
    D = da * r
    return tuple(
        torch.empty((B, nh, T, D), device=combined.device, dtype=combined.dtype)
        for nh in (NH, NKVH, NKVH)
    )


def allocate_grads(combined, inits, logit_bias, hq, hk, hv, grad_hq, grad_hk, grad_hv):
    """Gradient buffers as the reference allocates them, plus zeros for outputs
    that took no part in the loss (autograd passes None for those)."""
    grad_hq = torch.zeros_like(hq) if grad_hq is None else grad_hq
    grad_hk = torch.zeros_like(hk) if grad_hk is None else grad_hk
    grad_hv = torch.zeros_like(hv) if grad_hv is None else grad_hv
    grad_combined = torch.empty_like(combined)
    grad_inits = torch.empty_like(inits, memory_format=torch.contiguous_format)
    grad_logit_bias = torch.zeros_like(logit_bias, memory_format=torch.contiguous_format)
    return grad_hq, grad_hk, grad_hv, grad_combined, grad_inits, grad_logit_bias


# ---------------- FORWARD ----------------


@torch.library.impl(
    "nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward_kernel",
    "CUDA",
)
def forward_kernel(
    combined,
    inits,
    logit_bias,
    out_q,
    out_k,
    out_v,
    B,
    T,
    NH,
    NKVH,
    da,
    r,
    P,
    Q,
    K,
    scan_threads_forward,
    r_threads_forward,
    r_items_forward,
    use_sigmoid,
):
    _check_tuning(scan_threads_forward, r_threads_forward, r_items_forward)
    run_forward(combined, inits, logit_bias, out_q, out_k, out_v, B, T, NH, NKVH, da, r, P, Q,
                K, use_sigmoid)


@torch.library.impl(
    "nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_op",
    "CUDA",
)
def forward_op(
    combined,
    inits,
    logit_bias,
    NH,
    NKVH,
    da,
    r,
    P,
    Q,
    K,
    scan_threads_forward,
    r_threads_forward,
    r_items_forward,
    scan_threads_backward,
    r_threads_backward,
    r_items_backward,
    use_sigmoid: bool,
):
    B, T, _ = combined.shape
    assert combined.dtype == inits.dtype
    out_q, out_k, out_v = allocate_outputs(combined, NH, NKVH, da, r)
    torch.ops.nanochat_cuda.ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward_kernel(
        combined, inits, logit_bias, out_q, out_k, out_v, B, T, NH, NKVH, da, r, P, Q, K,
        scan_threads_forward, r_threads_forward, r_items_forward, use_sigmoid,
    )
    return out_q, out_k, out_v


# ---------------- BACKWARD ----------------


@torch.library.impl(
    "nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward_kernel",
    "CUDA",
)
def backward_kernel(
    combined,
    inits,
    logit_bias,
    hq,
    hk,
    hv,
    grad_hq,
    grad_hk,
    grad_hv,
    grad_combined,
    grad_inits,
    grad_logit_bias,
    NH,
    NKVH,
    da,
    r,
    P,
    Q,
    K,
    scan_threads_backward,
    r_threads_backward,
    r_items_backward,
    use_sigmoid: bool,
):
    _check_tuning(scan_threads_backward, r_threads_backward, r_items_backward)
    run_backward(combined, inits, logit_bias, hq, hk, hv, grad_hq, grad_hk, grad_hv,
                 grad_combined, grad_inits, grad_logit_bias, NH, NKVH, da, r, P, Q, K,
                 use_sigmoid)


def _setup(ctx, inputs, output):
    (combined, inits, logit_bias, NH, NKVH, da, r, P, Q, K, _stf, _rtf, _rif,
     scan_threads_backward, r_threads_backward, r_items_backward, use_sigmoid) = inputs
    hq, hk, hv = output
    ctx.save_for_backward(combined, inits, logit_bias, hq, hk, hv)
    ctx.args = (NH, NKVH, da, r, P, Q, K, scan_threads_backward, r_threads_backward,
                r_items_backward, use_sigmoid)


def backward(ctx, grad_hq, grad_hk, grad_hv):
    combined, inits, logit_bias, hq, hk, hv = ctx.saved_tensors
    grad_hq, grad_hk, grad_hv, grad_combined, grad_inits, grad_logit_bias = allocate_grads(
        combined, inits, logit_bias, hq, hk, hv, grad_hq, grad_hk, grad_hv)
    torch.ops.nanochat_cuda.ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward_kernel(
        combined, inits, logit_bias, hq, hk, hv, grad_hq, grad_hk, grad_hv,
        grad_combined, grad_inits, grad_logit_bias, *ctx.args,
    )
    # grads for the 3 tensors, None for the 14 scalars
    return (grad_combined, grad_inits, grad_logit_bias) + (None,) * 14


torch.library.register_autograd(
    "nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_op",
    backward,
    setup_context=_setup,
)
