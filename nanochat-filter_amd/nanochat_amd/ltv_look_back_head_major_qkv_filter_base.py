"""Base of the look-back QKV filters (reference
``nanochat/ltv_look_back_head_major_qkv_filter_base.py:12-87``).

The head-major combined projection of ``LtvCombinedHeadMajorQkvFilter``
followed by the look-back scan: the recurrence restarts in the chunks of the
layer's ``ChunksAndHistory`` (p, q, k), or runs unchunked when the caller asks
for the full recurrence (the KV-cache path).  ``forward(x, resolved_inits,
full_recurrence) -> (q, k, v)`` with q (B, T, NH, D), k and v (B, T, NKVH, D).

dtype policy (reference ``:53-87``): the projection and scan run in float32
when ``should_run_ltv_in_fp32`` says so (autocast asking for float32), else in
the dtype of ``x``; results are returned in the projection's dtype.
"""

from abc import ABC, abstractmethod

import torch

from nanochat_amd.gpt_config import UNBOUNDED_P, ChunksAndHistory
from nanochat_amd.ltv_combined_head_major_qkv_filter import LtvCombinedHeadMajorQkvFilter
from nanochat_amd.ltv_fused_concat_register_cast_scan_util import should_run_ltv_in_fp32

__all__ = ["LtvLookBackHeadMajorQkvFilter", "UNBOUNDED_P"]


class LtvLookBackHeadMajorQkvFilter(LtvCombinedHeadMajorQkvFilter, ABC):
    def __init__(self, n_head: int, n_kv_head: int, head_dim: int, r: int,
                 layer_spec: ChunksAndHistory):
        super().__init__(n_head, n_kv_head, head_dim, r)
        self.layer_spec = layer_spec

    def chunking(self, full_recurrence: bool) -> tuple[int, int, int]:
        """(P, Q, K) the scan runs with."""
        if full_recurrence:
            return UNBOUNDED_P, 1, 1
        return self.layer_spec.p, self.layer_spec.q, self.layer_spec.k

    @abstractmethod
    def _project(self, x: torch.Tensor) -> torch.Tensor:
        """x (B, T, C) -> the combined (B, T, F) tensor (any strides)."""

    @abstractmethod
    def _look_back_op(self, combined: torch.Tensor, inits: torch.Tensor,
                      logit_bias: torch.Tensor, full_recurrence: bool):
        """The scan: -> hq, hk, hv as (B, T, H, D) views."""

    def forward(self, x: torch.Tensor, resolved_inits: torch.Tensor, full_recurrence: bool):
        run_ltv_in_fp32 = should_run_ltv_in_fp32(x.device.type)
        combined = self._project(x.float() if run_ltv_in_fp32 else x)
        logit_bias = self.logit_bias.contiguous()
        inits = resolved_inits.to(dtype=combined.dtype).contiguous()
        hq, hk, hv = self._look_back_op(
            combined,
            inits.float() if run_ltv_in_fp32 else inits,
            logit_bias.float() if run_ltv_in_fp32 else logit_bias,
            full_recurrence,
        )
        if run_ltv_in_fp32:
            hq, hk, hv = hq.to(combined.dtype), hk.to(combined.dtype), hv.to(combined.dtype)
        return hq, hk, hv
