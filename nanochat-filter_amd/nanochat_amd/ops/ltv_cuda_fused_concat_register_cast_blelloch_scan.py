"""The scan op over the legacy projection layout
``combined (B, T, H (D + Da)) = [q values | k values | v values | gate logits]``.

Behavioural mirror of the reference's
``nanochat/ops/ltv_cuda_fused_concat_register_cast_blelloch_scan.py`` (forward
kernel ``:28-63``, functional op ``:66-123``, backward kernel ``:126-173``,
autograd ``:176-255``): the gate logits arrive with the bias already added, so
the op takes none; the backward writes ``grad_combined`` (values and logits),
``grad_inits``, and for ``r > 1`` also the fp32 ``grad_logits (B, T, H, Da)``
the reference's kernel fills.  Any strides.

The gfx950 library scans this layout through its split entry points: head h's
values are the 4-D view (b, h, t, d) -> column ``h D + d`` and its logits the
view (b, h, t, j) -> column ``H D + h Da + j`` of ``combined``, with a zero bias.

The launch-shape arguments (``chunk_size``, ``bank_count``: the reference's
block threads and items per thread) do not steer the HIP kernels and are not
validated: the reference's dispatch for this op builds a single shape (32, 1)
and then rejects it (``cpp_ewma/src/ltv_fused_concat_register_cast_blelloch_scan_cuda.cu:48-68, 611``),
so it accepts none.
"""

import ctypes

import torch

from nanochat_amd import _native as N


def _arr(s):
    return (ctypes.c_int64 * len(s))(*s)


def _views(t, H, D, Da):
    """Value and logit 4-D stride arrays (b, h, t, channel) and the logit pointer."""
    sb, st, se = t.stride()
    vals = _arr((sb, D * se, st, se))
    lgs = _arr((sb, Da * se, st, se))
    return vals, t.data_ptr() + H * D * se * t.element_size(), lgs


def _check(combined, inits, NH, NKVH, da, r):
    N.require_device(combined, inits)
    if combined.dim() != 3:
        raise RuntimeError(f"combined must be (B, T, F), got {tuple(combined.shape)}")
    B, T, F = combined.shape
    H, D = NH + 2 * NKVH, da * r
    if F != H * (D + da):
        raise RuntimeError(f"combined feature size {F} != (NH + 2*NKVH) * (D + da) = {H * (D + da)}")
    if tuple(inits.shape) != (B, H, D):
        raise RuntimeError(f"inits must be {(B, H, D)}, got {tuple(inits.shape)}")
    return B, T, H, D


@torch.library.impl(
    "nanochat_cuda::ltv_fused_concat_register_cast_blelloch_scan_cuda_forward_kernel", "CUDA"
)
def forward_kernel(combined, inits, out_q, out_k, out_v, T, NH, NKVH, da, r, block_threads,
                   items_per_thread, use_sigmoid):
    B, T_, H, D = _check(combined, inits, NH, NKVH, da, r)
    if T_ != T:
        raise RuntimeError(f"T={T} does not match combined.shape[1]={T_}")
    zero_bias = torch.zeros(H * da, dtype=torch.float32, device=combined.device)
    vals, lg_ptr, lgs = _views(combined, H, D, da)
    rc = N.lib().ltv_hm_scan_forward_split(
        N.dtype_code(combined.dtype), combined.data_ptr(), vals, lg_ptr, lgs,
        inits.data_ptr(), N.strides(inits, 3), zero_bias.data_ptr(),
        out_q.data_ptr(), N.strides(out_q, 4), out_k.data_ptr(), N.strides(out_k, 4),
        out_v.data_ptr(), N.strides(out_v, 4),
        B, T, NH, NKVH, da, r, int(bool(use_sigmoid)), N.stream_of(combined))
    N.check(rc, "ltv_hm_scan_forward_split")


@torch.library.impl("nanochat_cuda::ltv_fused_concat_register_cast_blelloch_scan_cuda_op", "CUDA")
def forward_op(combined, inits, NH, NKVH, da, r, block_threads=128, items_per_thread=8,
               use_sigmoid: bool = False):
    B, T, _ = combined.shape
    D = da * r
    assert combined.dtype == inits.dtype
    outs = [torch.empty((B, nh, T, D), device=combined.device, dtype=combined.dtype)
            for nh in (NH, NKVH, NKVH)]
    torch.ops.nanochat_cuda.ltv_fused_concat_register_cast_blelloch_scan_cuda_forward_kernel(
        combined, inits, *outs, T, NH, NKVH, da, r, block_threads, items_per_thread, use_sigmoid)
    return tuple(outs)


@torch.library.impl(
    "nanochat_cuda::ltv_fused_concat_register_cast_blelloch_scan_cuda_backward_kernel", "CUDA"
)
def backward_kernel(combined, inits, hq, hk, hv, grad_hq, grad_hk, grad_hv, grad_combined,
                    grad_inits, grad_logits, NH, NKVH, da, r, block_threads, items_per_thread,
                    use_sigmoid: bool):
    B, T, H, D = _check(combined, inits, NH, NKVH, da, r)
    dt = N.dtype_code(combined.dtype)
    lib = N.lib()
    zero_bias = torch.zeros(H * da, dtype=torch.float32, device=combined.device)
    grad_bias = torch.empty(H * da, dtype=torch.float32, device=combined.device)  # unused
    ws_bytes = lib.ltv_hm_scan_backward_workspace_size(dt, B, T, NH, NKVH, da, r)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=combined.device)
    vals, lg_ptr, lgs = _views(combined, H, D, da)
    gvals, glg_ptr, glgs = _views(grad_combined, H, D, da)
    s4 = lambda t: N.strides(t, 4)  # noqa: E731
    rc = lib.ltv_hm_scan_backward_split(
        dt, combined.data_ptr(), vals, lg_ptr, lgs,
        inits.data_ptr(), N.strides(inits, 3), zero_bias.data_ptr(),
        hq.data_ptr(), s4(hq), hk.data_ptr(), s4(hk), hv.data_ptr(), s4(hv),
        grad_hq.data_ptr(), s4(grad_hq), grad_hk.data_ptr(), s4(grad_hk),
        grad_hv.data_ptr(), s4(grad_hv),
        grad_combined.data_ptr(), gvals, glg_ptr, glgs,
        grad_inits.data_ptr(), N.strides(grad_inits, 3), grad_bias.data_ptr(),
        ws.data_ptr(), ws_bytes, B, T, NH, NKVH, da, r, int(bool(use_sigmoid)),
        N.stream_of(combined))
    N.check(rc, "ltv_hm_scan_backward_split")
    if r > 1:
        # the reference's kernel leaves the logit gradients (fp32) in grad_logits
        HD = H * D
        grad_logits.view(B, T, H * da).copy_(grad_combined[:, :, HD:HD + H * da])


def _setup(ctx, inputs, output):
    combined, inits, NH, NKVH, da, r, block_threads, items_per_thread, use_sigmoid = inputs
    ctx.save_for_backward(combined, inits, *output)
    ctx.args = (NH, NKVH, da, r, block_threads, items_per_thread, use_sigmoid)


def backward(ctx, grad_hq, grad_hk, grad_hv):
    combined, inits, hq, hk, hv = ctx.saved_tensors
    NH, NKVH, da, r = ctx.args[:4]
    B, T, _ = combined.shape
    H = NH + 2 * NKVH
    grad_hq = torch.zeros_like(hq) if grad_hq is None else grad_hq
    grad_hk = torch.zeros_like(hk) if grad_hk is None else grad_hk
    grad_hv = torch.zeros_like(hv) if grad_hv is None else grad_hv
    grad_combined = torch.empty(combined.shape, dtype=combined.dtype, device=combined.device)
    grad_inits = torch.empty_like(inits, memory_format=torch.contiguous_format)
    if r > 1:
        grad_logits = torch.zeros(B, T, H, da, dtype=torch.float32, device=combined.device)
    else:
        grad_logits = torch.empty(1, dtype=torch.float32, device=combined.device)
    torch.ops.nanochat_cuda.ltv_fused_concat_register_cast_blelloch_scan_cuda_backward_kernel(
        combined, inits, hq, hk, hv, grad_hq, grad_hk, grad_hv, grad_combined, grad_inits,
        grad_logits, *ctx.args)
    # (the logit columns of grad_combined are already written by the kernel)
    return grad_combined, grad_inits, None, None, None, None, None, None, None


torch.library.register_autograd(
    "nanochat_cuda::ltv_fused_concat_register_cast_blelloch_scan_cuda_op", backward,
    setup_context=_setup)
