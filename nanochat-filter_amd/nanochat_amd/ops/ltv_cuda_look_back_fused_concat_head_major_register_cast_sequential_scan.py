"""The sequential look-back scan ops.

Behavioural mirror of the reference's
``nanochat/ops/ltv_cuda_look_back_fused_concat_head_major_register_cast_sequential_scan.py``
(forward kernel ``:32-77``, functional op ``:79-148``, backward kernel
``:150-207``, autograd ``:209-304``).  The reference's sequential and Blelloch
kernels compute the same function (its Python oracle delegates one to the other,
``nanochat/ops/ltv_reference_ops.py:125-158``), so both op families run the same
gfx950 kernels; only the signatures differ (no scan-thread arguments here).
"""

import torch

from nanochat_amd.ops.ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan import (
    _check_r_tuning,
    allocate_grads,
    allocate_outputs,
    run_backward,
    run_forward,
)


@torch.library.impl(
    "nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_forward_kernel",
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
    r_threads_forward,
    r_items_forward,
    use_sigmoid,
):
    _check_r_tuning(r_threads_forward, r_items_forward)
    run_forward(combined, inits, logit_bias, out_q, out_k, out_v, B, T, NH, NKVH, da, r, P, Q,
                K, use_sigmoid)


@torch.library.impl(
    "nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_op",
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
    r_threads_forward,
    r_items_forward,
    r_threads_backward,
    r_items_backward,
    use_sigmoid: bool,
):
    B, T, _ = combined.shape
    assert combined.dtype == inits.dtype
    out_q, out_k, out_v = allocate_outputs(combined, NH, NKVH, da, r)
    torch.ops.nanochat_cuda.ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_forward_kernel(
        combined, inits, logit_bias, out_q, out_k, out_v, B, T, NH, NKVH, da, r, P, Q, K,
        r_threads_forward, r_items_forward, use_sigmoid,
    )
    return out_q, out_k, out_v


@torch.library.impl(
    "nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_backward_kernel",
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
    r_threads_backward,
    r_items_backward,
    use_sigmoid: bool,
):
    _check_r_tuning(r_threads_backward, r_items_backward)
    run_backward(combined, inits, logit_bias, hq, hk, hv, grad_hq, grad_hk, grad_hv,
                 grad_combined, grad_inits, grad_logit_bias, NH, NKVH, da, r, P, Q, K,
                 use_sigmoid)


def _setup(ctx, inputs, output):
    (combined, inits, logit_bias, NH, NKVH, da, r, P, Q, K, _rtf, _rif,
     r_threads_backward, r_items_backward, use_sigmoid) = inputs
    hq, hk, hv = output
    ctx.save_for_backward(combined, inits, logit_bias, hq, hk, hv)
    ctx.args = (NH, NKVH, da, r, P, Q, K, r_threads_backward, r_items_backward, use_sigmoid)


def backward(ctx, grad_hq, grad_hk, grad_hv):
    combined, inits, logit_bias, hq, hk, hv = ctx.saved_tensors
    grad_hq, grad_hk, grad_hv, grad_combined, grad_inits, grad_logit_bias = allocate_grads(
        combined, inits, logit_bias, hq, hk, hv, grad_hq, grad_hk, grad_hv)
    torch.ops.nanochat_cuda.ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_backward_kernel(
        combined, inits, logit_bias, hq, hk, hv, grad_hq, grad_hk, grad_hv,
        grad_combined, grad_inits, grad_logit_bias, *ctx.args,
    )
    # grads for the 3 tensors, None for the 12 scalars
    return (grad_combined, grad_inits, grad_logit_bias) + (None,) * 12


torch.library.register_autograd(
    "nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_op",
    backward,
    setup_context=_setup,
)
