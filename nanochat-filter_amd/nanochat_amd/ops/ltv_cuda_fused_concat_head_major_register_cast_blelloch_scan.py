"""CUDA-dispatch implementations and autograd of the head-major LTV scan op.

Behavioural mirror of the reference's
``nanochat/ops/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py``
(forward kernel ``:31-71``, functional op ``:74-135``, backward kernel
``:141-193``, autograd ``:196-289``): same schemas, same buffer ownership
(Python allocates every output; kernels only write), same argument checks.
The work is done by the gfx950 library through
``ltv_hm_scan_forward`` / ``ltv_hm_scan_backward`` (their ``_ws`` forms, with the chain
workspace of the chained scans).
"""

import torch

from nanochat_amd import _native as N

# Launch-shape arguments the reference's CUDA dispatch accepts
# (cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_common.cuh:9-30,
#  ltv_fused_concat_head_major_register_cast_scan_cuda_common.cuh:58-108).  They
# do not steer the HIP kernels, but out-of-set values are rejected the same way.
_SCAN_THREADS = (1, 8, 32)
_R_THREADS = (2, 8, 32)
_R_ITEMS = (1, 4, 8)


def _check_tuning(scan_threads, r_threads, r_items):
    if scan_threads not in _SCAN_THREADS:
        raise RuntimeError(f"Unsupported scan_threads: {scan_threads}")
    if r_threads not in _R_THREADS:
        raise RuntimeError(f"Unsupported r_threads: {r_threads}")
    if r_items not in _R_ITEMS:
        raise RuntimeError(f"Unsupported r_items: {r_items}")


def _check_common(combined, inits, logit_bias, NH, NKVH, da, r):
    N.require_device(combined, inits, logit_bias)
    if combined.dim() != 3:
        raise RuntimeError(f"combined must be (B, T, F), got shape {tuple(combined.shape)}")
    B, T, F = combined.shape
    H = NH + 2 * NKVH
    D = da * r
    if F != H * (D + da):
        raise RuntimeError(
            f"combined feature size {F} != (NH + 2*NKVH) * (D + da) = {H * (D + da)}")
    if tuple(inits.shape) != (B, H, D):
        raise RuntimeError(f"inits must be {(B, H, D)}, got {tuple(inits.shape)}")
    if logit_bias.dtype != torch.float32 or not logit_bias.is_contiguous() \
            or logit_bias.numel() != H * da:
        raise RuntimeError("logit_bias must be a contiguous float32 tensor of shape (H, da)")
    return B, T, H, D


def _s4(t):
    return N.strides(t, 4)


# ---------------- FORWARD ----------------


@torch.library.impl(
    "nanochat_cuda::ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward_kernel",
    "CUDA",
)
def forward_kernel(
    combined,
    inits,
    logit_bias,
    out_q,
    out_k,
    out_v,
    T,
    NH,
    NKVH,
    da,
    r,
    scan_threads_forward,
    r_threads_forward,
    r_items_forward,
    use_sigmoid,
):
    _check_tuning(scan_threads_forward, r_threads_forward, r_items_forward)
    B, T_, H, D = _check_common(combined, inits, logit_bias, NH, NKVH, da, r)
    if T_ != T:
        raise RuntimeError(f"T={T} does not match combined.shape[1]={T_}")
    lib = N.lib()
    cw = N.chain_workspace_for(combined.dtype, combined.device, B, T, NH, NKVH, da, r)
    rc = lib.ltv_hm_scan_forward_ws(
        N.dtype_code(combined.dtype),
        combined.data_ptr(), N.strides(combined, 3),
        inits.data_ptr(), N.strides(inits, 3),
        logit_bias.data_ptr(),
        out_q.data_ptr(), _s4(out_q),
        out_k.data_ptr(), _s4(out_k),
        out_v.data_ptr(), _s4(out_v),
        cw.ptr, cw.nbytes,
        B, T, NH, NKVH, da, r, int(bool(use_sigmoid)),
        N.stream_of(combined),
    )
    N.check(rc, "ltv_hm_scan_forward_ws")
    N.chain_done(cw)


@torch.library.impl(
    "nanochat_cuda::ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op",
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
    scan_threads_forward,
    r_threads_forward,
    r_items_forward,
    scan_threads_backward,
    r_threads_backward,
    r_items_backward,
    use_sigmoid: bool,
):
    B, T, _ = combined.shape
    D = da * r

    assert combined.dtype == inits.dtype

    out_q = torch.empty((B, NH, T, D), device=combined.device, dtype=combined.dtype)
    out_k = torch.empty((B, NKVH, T, D), device=combined.device, dtype=combined.dtype)
    out_v = torch.empty((B, NKVH, T, D), device=combined.device, dtype=combined.dtype)

    torch.ops.nanochat_cuda.ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward_kernel(
        combined,
        inits,
        logit_bias,
        out_q,
        out_k,
        out_v,
        T,
        NH,
        NKVH,
        da,
        r,
        scan_threads_forward,
        r_threads_forward,
        r_items_forward,
        use_sigmoid,
    )
    return out_q, out_k, out_v


# ---------------- BACKWARD ----------------


@torch.library.impl(
    "nanochat_cuda::ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward_kernel",
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
    scan_threads_backward,
    r_threads_backward,
    r_items_backward,
    use_sigmoid: bool,
):
    _check_tuning(scan_threads_backward, r_threads_backward, r_items_backward)
    B, T, H, D = _check_common(combined, inits, logit_bias, NH, NKVH, da, r)
    if grad_logit_bias.dtype != torch.float32 or not grad_logit_bias.is_contiguous():
        raise RuntimeError("grad_logit_bias must be a contiguous float32 tensor")
    dt = N.dtype_code(combined.dtype)
    lib = N.lib()
    ws_bytes = lib.ltv_hm_scan_backward_workspace_size(dt, B, T, NH, NKVH, da, r)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=combined.device)
    cw = N.chain_workspace_for(combined.dtype, combined.device, B, T, NH, NKVH, da, r,
                               backward=True)
    rc = lib.ltv_hm_scan_backward_ws(
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
        ws.data_ptr(), ws_bytes, cw.ptr, cw.nbytes,
        B, T, NH, NKVH, da, r, int(bool(use_sigmoid)),
        N.stream_of(combined),
    )
    N.check(rc, "ltv_hm_scan_backward_ws")
    N.chain_done(cw)


def _setup(ctx, inputs, output):
    (
        combined,
        inits,
        logit_bias,
        NH,
        NKVH,
        da,
        r,
        scan_threads_forward,
        r_threads_forward,
        r_items_forward,
        scan_threads_backward,
        r_threads_backward,
        r_items_backward,
        use_sigmoid,
    ) = inputs
    hq, hk, hv = output
    ctx.save_for_backward(combined, inits, logit_bias, hq, hk, hv)
    ctx.NH = NH
    ctx.NKVH = NKVH
    ctx.da = da
    ctx.r = r
    ctx.scan_threads_backward = scan_threads_backward
    ctx.r_threads_backward = r_threads_backward
    ctx.r_items_backward = r_items_backward
    ctx.use_sigmoid = use_sigmoid


def backward(ctx, grad_hq, grad_hk, grad_hv):
    combined, inits, logit_bias, hq, hk, hv = ctx.saved_tensors
    # outputs that did not take part in the loss arrive as None
    grad_hq = torch.zeros_like(hq) if grad_hq is None else grad_hq
    grad_hk = torch.zeros_like(hk) if grad_hk is None else grad_hk
    grad_hv = torch.zeros_like(hv) if grad_hv is None else grad_hv

    grad_combined = torch.empty_like(combined)
    grad_inits = torch.empty_like(inits, memory_format=torch.contiguous_format)
    grad_logit_bias = torch.zeros_like(logit_bias, memory_format=torch.contiguous_format)

    torch.ops.nanochat_cuda.ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward_kernel(
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
        ctx.NH,
        ctx.NKVH,
        ctx.da,
        ctx.r,
        ctx.scan_threads_backward,
        ctx.r_threads_backward,
        ctx.r_items_backward,
        ctx.use_sigmoid,
    )

    return (grad_combined, grad_inits, grad_logit_bias) + (None,) * 11


torch.library.register_autograd(
    "nanochat_cuda::ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op",
    backward,
    setup_context=_setup,
)
