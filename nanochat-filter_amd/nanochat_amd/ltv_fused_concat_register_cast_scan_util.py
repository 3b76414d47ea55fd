"""dtype policy and tunables of the LTV filter
(reference ``nanochat/ltv_fused_concat_register_cast_scan_util.py:7-70``).

``CUDA_SUPPORTS_NATIVE_BF16`` is true on gfx950 (bf16 MFMA and conversions are
native).  The ``_*_FORWARD`` / ``_*_BACKWARD`` values are the reference's launch
shapes for its CUDA kernels; they keep their environment variables and
defaults so scripts that set them still run, and the ops validate them against
the reference's accepted sets, but they do not steer the HIP kernels (those pick
their own launch shapes from the tensor shapes).
"""

import torch

from nanochat_amd.ltv.ltv_filter import LtvInitValues
from nanochat_amd.train_utils import env_int


CUDA_SUPPORTS_NATIVE_BF16 = torch.cuda.is_available() and torch.cuda.is_bf16_supported(
    including_emulation=False
)


def should_run_cuda_ltv_in_fp32(tensor: torch.Tensor) -> bool:
    return (
        not CUDA_SUPPORTS_NATIVE_BF16
        and tensor.dtype == torch.bfloat16
        and tensor.is_cuda
    )


def should_run_ltv_in_fp32(device_type: str) -> bool:
    """True only when autocast asks for float32 on this device, or for bf16 on a
    CUDA device without native bf16."""
    if torch.is_autocast_enabled(device_type):
        autocast_dtype = torch.get_autocast_dtype(device_type)
        if device_type == "cuda":
            if autocast_dtype == torch.float32:
                return True
            if autocast_dtype == torch.bfloat16 and not CUDA_SUPPORTS_NATIVE_BF16:
                return True
        return False
    return False


def resolve_inits_original_dtype(B, init_param, previous_values: LtvInitValues):
    """Initial states (B, H, D): the cached previous q/k/v rows when given,
    otherwise the learned ``init_param`` broadcast over the batch."""
    if previous_values.q is not None:
        return torch.cat([previous_values.q, previous_values.k, previous_values.v], dim=1)
    return init_param.unsqueeze(0).expand(B, -1, -1)


_SCAN_THREADS_FORWARD = env_int(
    "LTV_CUDA_FUSED_CONCAT_HEAD_MAJOR_REGISTER_CAST_SCAN_THREADS_FORWARD", 8
)
_R_THREADS_FORWARD = env_int(
    "LTV_CUDA_FUSED_CONCAT_HEAD_MAJOR_REGISTER_CAST_R_THREADS_FORWARD", 8
)
_R_ITEMS_FORWARD = env_int(
    "LTV_CUDA_FUSED_CONCAT_HEAD_MAJOR_REGISTER_CAST_R_ITEMS_FORWARD", 4
)
_SCAN_THREADS_BACKWARD = env_int(
    "LTV_CUDA_FUSED_CONCAT_HEAD_MAJOR_REGISTER_CAST_SCAN_THREADS_BACKWARD", 32
)
_R_THREADS_BACKWARD = env_int(
    "LTV_CUDA_FUSED_CONCAT_HEAD_MAJOR_REGISTER_CAST_R_THREADS_BACKWARD", 2
)
_R_ITEMS_BACKWARD = env_int(
    "LTV_CUDA_FUSED_CONCAT_HEAD_MAJOR_REGISTER_CAST_R_ITEMS_BACKWARD", 8
)
