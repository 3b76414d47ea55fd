"""Look-back QKV filter with a plain ``nn.Linear`` projection and the
sequential-scan look-back op (reference
``nanochat/ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_qkv_filter.py:41-90``).

Same constructor (the op is injected) and the reference dataflow: ``self.c(x)``
in the natural (B, T, F) layout, then the op.  With this package's
``ltv_cuda_look_back_..._sequential_scan`` in bf16 it takes the same fused path
as the Blelloch filter (the two ops compute the same function).
"""

from collections.abc import Callable

import torch

from nanochat_amd.gpt_config import ChunksAndHistory
from nanochat_amd.ltv_fused_concat_register_cast_scan_util import (
    _R_ITEMS_BACKWARD,
    _R_ITEMS_FORWARD,
    _R_THREADS_BACKWARD,
    _R_THREADS_FORWARD,
    should_run_ltv_in_fp32,
)
from nanochat_amd.ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
    look_back_fused_forward,
)
from nanochat_amd.ltv_look_back_head_major_qkv_filter_base import LtvLookBackHeadMajorQkvFilter
from nanochat_amd.ops import ltv_hm_fast as hm_fast
from nanochat_amd.ops.ltv_cuda_ops import (
    ltv_cuda_look_back_fused_concat_head_major_register_cast_sequential_scan,
)

# (combined, inits, logit_bias, NH, NKVH, da, r, P, Q, K, r threads and items
#  forward and backward, use_sigmoid) -> (hq, hk, hv), each (B, H, T, D)
SequentialLookBackOp = Callable[..., tuple[torch.Tensor, torch.Tensor, torch.Tensor]]


class LtvLookBackFusedConcatHeadMajorRegisterCastSequentialScanQkvFilter(
    LtvLookBackHeadMajorQkvFilter
):
    def __init__(self, n_head: int, n_kv_head: int, head_dim: int, r: int,
                 layer_spec: ChunksAndHistory, sequential_look_back_op: SequentialLookBackOp):
        super().__init__(n_head, n_kv_head, head_dim, r, layer_spec)
        self.sequential_look_back_op = sequential_look_back_op

    def forward(self, x: torch.Tensor, resolved_inits: torch.Tensor, full_recurrence: bool):
        if (self.sequential_look_back_op is
                ltv_cuda_look_back_fused_concat_head_major_register_cast_sequential_scan
                and x.is_cuda and x.dtype == torch.bfloat16
                and not should_run_ltv_in_fp32(x.device.type)
                and hm_fast.fast_path_ok(x.size(2), self.head_dim)):
            return look_back_fused_forward(self, x, resolved_inits, full_recurrence)
        return super().forward(x, resolved_inits, full_recurrence)

    def _project(self, x: torch.Tensor) -> torch.Tensor:
        # in x's dtype, the weight rounded to it
        return torch.nn.functional.linear(x, self.c.weight.to(x.dtype)).contiguous()

    def _look_back_op(self, combined, inits, logit_bias, full_recurrence: bool):
        P, Q, K = self.chunking(full_recurrence)
        hq, hk, hv = self.sequential_look_back_op(
            combined, inits, logit_bias, self.n_head, self.n_kv_head, self.num_alpha_groups,
            self.r, P, Q, K,
            _R_THREADS_FORWARD, _R_ITEMS_FORWARD, _R_THREADS_BACKWARD, _R_ITEMS_BACKWARD,
            True,  # use_sigmoid
        )
        return hq.transpose(1, 2), hk.transpose(1, 2), hv.transpose(1, 2)
