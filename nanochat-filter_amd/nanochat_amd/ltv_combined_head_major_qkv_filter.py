"""Head-major combined filter: per-head interleaved projection rows
``[head 0 values (D) | head 0 logits (Da) | head 1 values | ...]``.

Parameters and initialisation as the reference's
``nanochat/ltv_combined_head_major_qkv_filter.py:11-66``: the value rows of q,
k, v and the gate rows are drawn U(-weight_s, weight_s) in the order q, k, v,
gates, then interleaved per head; ``logit_bias`` (H, Da) ~
U(alpha_mlp_bias_init - bias_s, alpha_mlp_bias_init + bias_s); ``init_param``
via ``init_weights_of_init``.  Same RNG consumption order, so seeded inits match.
"""

import torch
import torch.nn as nn

from nanochat_amd.ltv.ltv_fused_scan_filter import init_weights_of_init
from nanochat_amd.ltv_combined_qkv_filter_base import LtvCombinedQkvFilterBase


class LtvCombinedHeadMajorQkvFilter(LtvCombinedQkvFilterBase):
    def __init__(self, n_head: int, n_kv_head: int, head_dim: int, r: int):
        super().__init__(n_head, n_kv_head, head_dim, r)
        self.logit_bias = nn.Parameter(
            torch.empty(self.total_active_heads, self.num_alpha_groups)
        )

    def init_weights(
        self, alpha_mlp_bias_init: float, weight_s: float, bias_s: float, init_s: float
    ):
        C = self.c.in_features
        H, D, Da = self.total_active_heads, self.head_dim, self.num_alpha_groups
        q_val = self.c.weight.new_empty(self.n_head * D, C)
        k_val = self.c.weight.new_empty(self.n_kv_head * D, C)
        v_val = self.c.weight.new_empty(self.n_kv_head * D, C)
        torch.nn.init.uniform_(q_val, -weight_s, weight_s)
        torch.nn.init.uniform_(k_val, -weight_s, weight_s)
        torch.nn.init.uniform_(v_val, -weight_s, weight_s)
        gate_w = self.c.weight.new_empty(H * Da, C)
        torch.nn.init.uniform_(gate_w, -weight_s, weight_s)

        per_head = torch.cat(
            [torch.cat([q_val, k_val, v_val], dim=0).view(H, D, C), gate_w.view(H, Da, C)],
            dim=1,
        )
        with torch.no_grad():
            self.c.weight.copy_(per_head.view(-1, C))

        torch.nn.init.uniform_(
            self.logit_bias, alpha_mlp_bias_init - bias_s, alpha_mlp_bias_init + bias_s
        )
        init_weights_of_init(self.init_param, self.n_head, self.n_kv_head, init_s)
