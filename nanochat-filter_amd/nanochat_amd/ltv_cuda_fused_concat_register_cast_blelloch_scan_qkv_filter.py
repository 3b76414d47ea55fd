"""The legacy-layout combined filter on the gfx950 scan (reference
``nanochat/ltv_cuda_fused_concat_register_cast_blelloch_scan_qkv_filter.py:26-81``).

Dataflow as the reference: ``combined = c(x)`` in the layout
``[q values | k values | v values | gate logits]``, the 1-D ``logit_bias`` added
to the logit columns in place, then the scan op
``nanochat_cuda::ltv_fused_concat_register_cast_blelloch_scan_cuda_op`` on
``combined`` (no bias argument).  The scan reads the value and logit slots as
two strided views of ``combined`` (head ``h``'s values start at column ``h D``
in this layout too, its logits at ``H D + h Da``), so no copy is made.
"""

import torch

import nanochat_amd.ops  # noqa: F401  (registers the ops)
from nanochat_amd.ltv.ltv_filter import LtvInitValues
from nanochat_amd.ltv_combined_qkv_filter import LtvCombinedQkvFilter
from nanochat_amd.ltv_fused_concat_register_cast_scan_util import (
    resolve_inits_original_dtype,
    should_run_cuda_ltv_in_fp32,
)
from nanochat_amd.train_utils import env_int

# the reference's launch-shape tunables for this op (accepted, not used: the
# gfx950 scan picks its own launch shape)
_BLOCK_THREADS = env_int("LTV_CUDA_FUSED_CONCAT_REGISTER_CAST_BLELLOCH_SCAN_BLOCK_THREADS", 32)
_ITEMS_PER_THREAD = env_int("LTV_CUDA_FUSED_CONCAT_REGISTER_CAST_BLELLOCH_SCAN_ITEMS_PER_THREAD", 1)


class LtvCudaFusedConcatRegisterCastBlellochScanQkvFilter(LtvCombinedQkvFilter):
    def forward(self, x, previous_values: LtvInitValues):
        B = x.size(0)
        combined = self.c(x)
        q_size, kv_size, kv_size2, logit_size = self.split_sections
        logit_start = q_size + kv_size + kv_size2
        combined[..., logit_start:logit_start + logit_size].add_(self.logit_bias)
        inits = (resolve_inits_original_dtype(B, self.init_param, previous_values)
                 .contiguous().to(dtype=combined.dtype))
        run_ltv_in_fp32 = should_run_cuda_ltv_in_fp32(combined)
        kernel_combined = combined.float() if run_ltv_in_fp32 else combined
        kernel_inits = inits.float() if run_ltv_in_fp32 else inits
        hq, hk, hv = torch.ops.nanochat_cuda.ltv_fused_concat_register_cast_blelloch_scan_cuda_op(
            kernel_combined, kernel_inits, self.n_head, self.n_kv_head, self.num_alpha_groups,
            self.r, _BLOCK_THREADS, _ITEMS_PER_THREAD, True)
        if run_ltv_in_fp32:
            hq, hk, hv = hq.to(combined.dtype), hk.to(combined.dtype), hv.to(combined.dtype)
        return hq.transpose(1, 2), hk.transpose(1, 2), hv.transpose(1, 2)
