"""CUDA-dispatch implementations and autograd of ``fused_linear_transpose``.

Behavioural mirror of the reference's ``nanochat/ops/fused_linear_transpose.py``
(``:20-134``): ``out[b] (F x T) = weight (F x K) @ x[b]^T`` with contiguous
inputs, a zero-initialised (B, F, T) output from the functional op, and a
backward that accepts grad_out either contiguous or as the transposed view of a
(B, T, F)-contiguous tensor.  The work runs in the gfx950 library
(``ltv_linear_transpose_forward`` / ``ltv_linear_transpose_backward_ws``): bf16
MFMA kernels where the layout allows, else the strided fp32-MFMA GEMM.
"""

import torch

from nanochat_amd import _native as N


@torch.library.impl("nanochat_cuda::fused_linear_transpose", "CUDA")
def fused_linear_transpose(x, weight, out):
    if not x.is_contiguous() or not weight.is_contiguous() or not out.is_contiguous():
        raise RuntimeError(
            "fused_linear_transpose requires contiguous x, weight, and out tensors"
        )
    N.require_device(x, weight, out)
    if x.dtype != weight.dtype or out.dtype != x.dtype:
        raise RuntimeError(
            f"fused_linear_transpose requires one dtype for x, weight and out, got "
            f"{x.dtype}, {weight.dtype}, {out.dtype}")
    B, T, K = x.shape
    F = weight.size(0)
    if weight.size(1) != K or tuple(out.shape) != (B, F, T):
        raise RuntimeError(
            f"shape mismatch: x {tuple(x.shape)}, weight {tuple(weight.shape)}, "
            f"out {tuple(out.shape)}")
    with N.span("linear_transpose_fwd"):
        rc = N.lib().ltv_linear_transpose_forward(
            N.dtype_code(x.dtype), x.data_ptr(), weight.data_ptr(), out.data_ptr(),
            B, T, K, F, N.stream_of(x))
    N.check(rc, "ltv_linear_transpose_forward")
    return None


@torch.library.impl("nanochat_cuda::fused_linear_transpose_cuda_op", "CUDA")
def fused_linear_transpose_cuda_op(x, weight):
    B, T, K = x.shape
    F = weight.size(0)
    # the kernel writes every element (the reference zero-fills first, a 152 MB
    # memset at d12); an empty reduction (K == 0) still gets zeros
    alloc = torch.zeros if K == 0 else torch.empty
    out = alloc((B, F, T), dtype=x.dtype, device=x.device)
    torch.ops.nanochat_cuda.fused_linear_transpose(x, weight, out)
    return out


def _is_transposed_grad_out(grad_out):
    return (
        grad_out.stride(1) == 1
        and grad_out.stride(2) == grad_out.size(1)
        and grad_out.stride(0) == grad_out.size(1) * grad_out.size(2)
    )


@torch.library.impl("nanochat_cuda::fused_linear_transpose_backward_kernel", "CUDA")
def fused_linear_transpose_backward_kernel(x, weight, grad_out, grad_x, grad_weight):
    if (
        not x.is_contiguous()
        or not weight.is_contiguous()
        or not (grad_out.is_contiguous() or _is_transposed_grad_out(grad_out))
    ):
        raise RuntimeError(
            "fused_linear_transpose_backward_kernel requires contiguous x and weight, "
            "and either contiguous or transposed grad_out. Found strides: "
            f"x={x.stride()}, weight={weight.stride()}, grad_out={grad_out.stride()}"
        )
    N.require_device(x, weight, grad_out, grad_x, grad_weight)
    if not (grad_x.is_contiguous() and grad_weight.is_contiguous()):
        raise RuntimeError("grad_x and grad_weight must be contiguous")
    dt = x.dtype
    if weight.dtype != dt or grad_out.dtype != dt or grad_x.dtype != dt or grad_weight.dtype != dt:
        raise RuntimeError("fused_linear_transpose backward requires one dtype for all tensors")
    B, T, K = x.shape
    F = weight.size(0)
    is_btf = 1 if (not grad_out.is_contiguous()) else 0
    lib = N.lib()
    # the weight gradient's reduction over B T is split into fp32 partials,
    # which need a workspace (0 bytes: no split)
    ws_bytes = lib.ltv_linear_transpose_backward_workspace_size(N.dtype_code(dt), B, T, K, F, is_btf)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    with N.span("linear_transpose_bwd"):
        rc = lib.ltv_linear_transpose_backward_ws(
            N.dtype_code(dt), x.data_ptr(), weight.data_ptr(), grad_out.data_ptr(), is_btf,
            grad_x.data_ptr(), grad_weight.data_ptr(), ws.data_ptr(), ws_bytes, B, T, K, F,
            N.stream_of(x))
    N.check(rc, "ltv_linear_transpose_backward_ws")
    return None


def _fused_linear_transpose_setup(ctx, inputs, output):
    x, weight = inputs
    ctx.save_for_backward(x, weight)


def _fused_linear_transpose_backward(ctx, grad_out):
    x, weight = ctx.saved_tensors
    # the kernel reads grad_out as (B, F, T) or as its transposed (B, T, F)
    # view; autograd can hand over other layouts (an expanded zero gradient
    # under AOT tracing, say), which are made contiguous here rather than
    # refused as the reference does -- every layout it accepts is unchanged
    if not (grad_out.is_contiguous() or _is_transposed_grad_out(grad_out)):
        grad_out = grad_out.contiguous()
    if (
        not x.is_contiguous()
        or not weight.is_contiguous()
        or not (grad_out.is_contiguous() or _is_transposed_grad_out(grad_out))
    ):
        raise RuntimeError(
            "fused_linear_transpose backward requires contiguous x and weight, "
            "and either contiguous or transposed grad_out. Found strides: "
            f"x={x.stride()}, weight={weight.stride()}, grad_out={grad_out.stride()}"
        )
    # overwritten by the kernels; empty reductions (F == 0 for grad_x, B T == 0
    # for grad_weight) still get zeros
    B, T, _ = x.shape
    F = weight.size(0)
    grad_x = (torch.zeros_like if F == 0 else torch.empty_like)(
        x, memory_format=torch.contiguous_format)
    grad_weight = (torch.zeros_like if B * T == 0 else torch.empty_like)(
        weight, memory_format=torch.contiguous_format)
    torch.ops.nanochat_cuda.fused_linear_transpose_backward_kernel(
        x, weight, grad_out, grad_x, grad_weight
    )
    return grad_x, grad_weight


torch.library.register_autograd(
    "nanochat_cuda::fused_linear_transpose_cuda_op",
    _fused_linear_transpose_backward,
    setup_context=_fused_linear_transpose_setup,
)
