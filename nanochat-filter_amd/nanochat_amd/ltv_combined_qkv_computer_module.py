"""Adapter from the combined filter to ``CausalSelfAttention``'s
``qkv_computer(x, kv_cache)`` protocol (reference
``nanochat/ltv_combined_qkv_computer_module.py:12-61``).

With a KV cache that holds this layer's last q/k/v rows, those rows are the
filter's initial states; after the call the last output rows are stored back,
so decoding one token at a time continues the recurrence.
"""

import logging
from typing import Optional

import torch.nn as nn

from nanochat_amd.kv_cache import KVCache
from nanochat_amd.ltv.ltv_filter import LtvInitValues
from nanochat_amd.ltv_combined_qkv_filter_base import LtvCombinedQkvFilterBase

logger = logging.getLogger(__name__)


class LtvCombinedQkvComputerModule(nn.Module):
    def __init__(self, layer_idx: int, ltv_filter: LtvCombinedQkvFilterBase):
        super().__init__()
        self.ltv_filter = ltv_filter
        self.layer_idx = layer_idx

    def forward(self, x, kv_cache: Optional[object]):
        if kv_cache and kv_cache.has_last_qkv(self.layer_idx):
            last = kv_cache.last_qkv
            previous_values = LtvInitValues(
                q=last.q.special[self.layer_idx],
                k=last.k.special[self.layer_idx],
                v=last.v.special[self.layer_idx],
            )
        else:
            previous_values = LtvInitValues(None, None, None)

        # A filter that can store its new last rows itself (the fused decode
        # step) writes them straight into the cache's row buffers -- the rows
        # it read as previous_values -- which is what update_last_qkv below
        # would copy there (the cache already holds this layer's rows, so its
        # bookkeeping has nothing to change).  Only for KVCache, whose row
        # buffers are its own (a cache that kept references to earlier outputs
        # would see them overwritten).
        decode_into = getattr(self.ltv_filter, "decode_into_rows", None)
        if (decode_into is not None and previous_values.q is not None
                and isinstance(kv_cache, KVCache)):
            out = decode_into(x, previous_values,
                              (previous_values.q, previous_values.k, previous_values.v))
            if out is not None:
                return out

        q, k, v = self.ltv_filter(x, previous_values)

        if kv_cache:
            kv_cache.update_last_qkv(
                self.layer_idx, q=q[:, -1, :, :], k=k[:, -1, :, :], v=v[:, -1, :, :]
            )
        return q, k, v

    def init_weights(
        self, alpha_mlp_bias_init: float, weight_s: float, bias_s: float, init_s: float
    ):
        self.ltv_filter.init_weights(
            alpha_mlp_bias_init=alpha_mlp_bias_init,
            weight_s=weight_s,
            bias_s=bias_s,
            init_s=init_s,
        )

    def get_matrix_linear_params(self):
        return self.ltv_filter.get_matrix_linear_params()

    def estimate_flops(self, sequence_len: int) -> int:
        return self.ltv_filter.estimate_flops(sequence_len)

    def ltv_parameter_count(self) -> int:
        return self.ltv_filter.ltv_parameter_count()
