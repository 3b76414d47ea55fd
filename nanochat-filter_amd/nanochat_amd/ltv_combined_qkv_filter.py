"""Combined filter with the legacy projection layout
``[all q values | all k values | all v values | all gate logits]`` (reference
``nanochat/ltv_combined_qkv_filter.py:11-62``).

Parameters: ``c.weight (H (D + Da), C)`` in that row order, a 1-D
``logit_bias (H Da)`` added to the gate-logit columns, ``init_param (H, D)``.
``init_weights`` draws q, k, v values and the gate rows U(-weight_s, weight_s)
in that order, the bias U(alpha_mlp_bias_init -/+ bias_s), then the inits (same
RNG consumption as the reference).
"""

import torch
import torch.nn as nn

from nanochat_amd.ltv.ltv_fused_scan_filter import init_weights_of_init
from nanochat_amd.ltv_combined_qkv_filter_base import LtvCombinedQkvFilterBase


class LtvCombinedQkvFilter(LtvCombinedQkvFilterBase):
    def __init__(self, n_head: int, n_kv_head: int, head_dim: int, r: int):
        super().__init__(n_head, n_kv_head, head_dim, r)
        self.logit_bias = nn.Parameter(torch.empty(self.total_active_heads * self.num_alpha_groups))

    def init_weights(
        self, alpha_mlp_bias_init: float, weight_s: float, bias_s: float, init_s: float
    ):
        C = self.c.in_features
        HD = self.total_active_heads * self.head_dim
        blocks = [self.c.weight.new_empty(n * self.head_dim, C)
                  for n in (self.n_head, self.n_kv_head, self.n_kv_head)]
        for w in blocks:
            torch.nn.init.uniform_(w, -weight_s, weight_s)
        gates = self.c.weight.new_empty(self.c.weight.shape[0] - HD, C)
        torch.nn.init.uniform_(gates, -weight_s, weight_s)
        with torch.no_grad():
            self.c.weight.copy_(torch.cat(blocks + [gates], dim=0))
        torch.nn.init.uniform_(
            self.logit_bias, alpha_mlp_bias_init - bias_s, alpha_mlp_bias_init + bias_s
        )
        init_weights_of_init(self.init_param, self.n_head, self.n_kv_head, init_s)
