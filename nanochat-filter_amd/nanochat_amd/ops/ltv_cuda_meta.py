"""Fake (meta) implementations so the path traces under torch.compile.

Shape/dtype rules of the reference's ``nanochat/ops/ltv_cuda_meta.py``
(``:155-252`` for the scan, ``:341-377`` for fused_linear_transpose).
"""

import torch


@torch.library.register_fake(
    "nanochat_cuda::ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op"
)
def _scan_op_fake(combined, inits, logit_bias, NH, NKVH, da, r, *tuning_and_flag):
    B, T, _ = combined.shape
    D = da * r
    mk = lambda h: combined.new_empty((B, h, T, D))  # noqa: E731
    return mk(NH), mk(NKVH), mk(NKVH)


@torch.library.register_fake(
    "nanochat_cuda::ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward_kernel"
)
def _scan_fwd_kernel_fake(*args):
    return None


@torch.library.register_fake(
    "nanochat_cuda::ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward_kernel"
)
def _scan_bwd_kernel_fake(*args):
    return None


@torch.library.register_fake("nanochat_cuda::fused_linear_transpose")
def _flt_fake(x, weight, out):
    return None


@torch.library.register_fake("nanochat_cuda::fused_linear_transpose_cuda_op")
def _flt_op_fake(x, weight):
    B, T, _ = x.shape
    return x.new_empty((B, weight.size(0), T))


@torch.library.register_fake("nanochat_cuda::fused_linear_transpose_backward_kernel")
def _flt_bwd_fake(x, weight, grad_out, grad_x, grad_weight):
    return None


# Look-back ops (reference nanochat/ops/ltv_cuda_meta.py:380-580): outputs
# (B, NH|NKVH, T, D) like the full-recurrence op; the kernels return nothing.
def _look_back_op_fake(combined, inits, logit_bias, NH, NKVH, da, r, *pqk_tuning_and_flag):
    B, T, _ = combined.shape
    D = da * r
    mk = lambda h: combined.new_empty((B, h, T, D))  # noqa: E731
    return mk(NH), mk(NKVH), mk(NKVH)


for _variant in ("blelloch", "sequential"):
    _base = f"nanochat_cuda::ltv_look_back_fused_concat_head_major_register_cast_{_variant}_scan_cuda"
    torch.library.register_fake(f"{_base}_op")(_look_back_op_fake)
    torch.library.register_fake(f"{_base}_forward_kernel")(lambda *args: None)
    torch.library.register_fake(f"{_base}_backward_kernel")(lambda *args: None)


# Legacy-layout scan op (reference nanochat/ops/ltv_cuda_meta.py:76-150).
@torch.library.register_fake("nanochat_cuda::ltv_fused_concat_register_cast_blelloch_scan_cuda_op")
def _legacy_op_fake(combined, inits, NH, NKVH, da, r, chunk_size, bank_count, use_sigmoid):
    B, T, _ = combined.shape
    D = da * r
    mk = lambda h: combined.new_empty((B, h, T, D))  # noqa: E731
    return mk(NH), mk(NKVH), mk(NKVH)


torch.library.register_fake(
    "nanochat_cuda::ltv_fused_concat_register_cast_blelloch_scan_cuda_forward_kernel")(
    lambda *args: None)
torch.library.register_fake(
    "nanochat_cuda::ltv_fused_concat_register_cast_blelloch_scan_cuda_backward_kernel")(
    lambda *args: None)
