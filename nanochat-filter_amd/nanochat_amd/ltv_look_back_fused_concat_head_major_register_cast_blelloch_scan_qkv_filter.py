"""Look-back QKV filter with the fused linear-transpose projection and the
Blelloch-scan look-back op (reference
``nanochat/ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter.py:21-99``).

Same constructor: the projection (``transpose_op(x, W) -> (B, F, T)``) and the
scan (``look_back_op``, the reference's op signature) are injected, and the
filter runs them as the reference does -- with this package's
``fused_linear_transpose`` and ``ltv_cuda_look_back_..._blelloch_scan`` they
run on the gfx950 library.  For exactly that pair in bf16 the filter takes the
fused path instead: one ``nanochat_amd::qkv_filter`` call (bf16 MFMA projection
straight into the scan's head-major layout, then the look-back scan; autograd
through its fused backward), and for one-token inference steps of the full
recurrence (the KV-cache path) the fused decode kernel.  Same results to bf16
rounding; the layout the injected ops use is never materialised.
"""

from collections.abc import Callable

import torch

from nanochat_amd.gpt_config import ChunksAndHistory
from nanochat_amd.ltv_fused_concat_register_cast_scan_util import (
    _R_ITEMS_BACKWARD,
    _R_ITEMS_FORWARD,
    _R_THREADS_BACKWARD,
    _R_THREADS_FORWARD,
    _SCAN_THREADS_BACKWARD,
    _SCAN_THREADS_FORWARD,
    should_run_ltv_in_fp32,
)
from nanochat_amd.ltv_look_back_head_major_qkv_filter_base import LtvLookBackHeadMajorQkvFilter
from nanochat_amd.ops import ltv_hm_fast as hm_fast
from nanochat_amd.ops.ltv_cuda_ops import (
    fused_linear_transpose,
    ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan,
)

TransposeOp = Callable[[torch.Tensor, torch.Tensor], torch.Tensor]

# (combined, inits, logit_bias, NH, NKVH, da, r, P, Q, K, scan/r threads and
#  items forward and backward, use_sigmoid) -> (hq, hk, hv), each (B, H, T, D)
LookBackOp = Callable[..., tuple[torch.Tensor, torch.Tensor, torch.Tensor]]


class LtvLookBackFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter(
    LtvLookBackHeadMajorQkvFilter
):
    def __init__(self, n_head: int, n_kv_head: int, head_dim: int, r: int,
                 layer_spec: ChunksAndHistory, transpose_op: TransposeOp,
                 look_back_op: LookBackOp):
        super().__init__(n_head, n_kv_head, head_dim, r, layer_spec)
        self.transpose_op = transpose_op
        self.look_back_op = look_back_op

    def _uses_library_ops(self) -> bool:
        return (self.transpose_op is fused_linear_transpose and self.look_back_op is
                ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan)

    def forward(self, x: torch.Tensor, resolved_inits: torch.Tensor, full_recurrence: bool):
        """resolved_inits: (B, H, D), or (H, D) shared by every sequence (the
        init parameter itself, as the computer module passes it without a KV
        cache): the library then sums its gradient over the batch where the
        kernels can, else it is expanded to (B, H, D) here."""
        fused = (self._uses_library_ops() and x.is_cuda and x.dtype == torch.bfloat16
                 and not should_run_ltv_in_fp32(x.device.type)
                 and hm_fast.fast_path_ok(x.size(2), self.head_dim))
        if resolved_inits.dim() == 2 and not (fused and self.takes_shared_inits(x, full_recurrence)):
            resolved_inits = resolved_inits.unsqueeze(0).expand(x.size(0), -1, -1)
        if fused:
            return look_back_fused_forward(self, x, resolved_inits, full_recurrence)
        return super().forward(x, resolved_inits, full_recurrence)

    def takes_shared_inits(self, x: torch.Tensor, full_recurrence: bool) -> bool:
        """Whether the fused path takes (H, D) inits for this input and sums
        their gradient over the batch in the library (not the one-step decode,
        which reads per-sequence cache rows)."""
        if full_recurrence and x.size(1) == 1:
            return False
        P, Q, K = self.chunking(full_recurrence)
        return hm_fast.fp32_inits_ok(x.size(1), self.head_dim, self.r, P, Q, K)

    def _project(self, x: torch.Tensor) -> torch.Tensor:
        # the projection runs in x's dtype (the weight rounded to it)
        out_buf = self.transpose_op(x, self.c.weight.to(x.dtype))
        return out_buf.transpose(1, 2)  # (B, T, F) view of the (B, F, T) buffer

    def _look_back_op(self, combined, inits, logit_bias, full_recurrence: bool):
        P, Q, K = self.chunking(full_recurrence)
        hq, hk, hv = self.look_back_op(
            combined, inits, logit_bias, self.n_head, self.n_kv_head, self.num_alpha_groups,
            self.r, P, Q, K,
            _SCAN_THREADS_FORWARD, _R_THREADS_FORWARD, _R_ITEMS_FORWARD,
            _SCAN_THREADS_BACKWARD, _R_THREADS_BACKWARD, _R_ITEMS_BACKWARD,
            True,  # use_sigmoid
        )
        return hq.transpose(1, 2), hk.transpose(1, 2), hv.transpose(1, 2)


def look_back_fused_forward(filt: LtvLookBackHeadMajorQkvFilter, x: torch.Tensor,
                            resolved_inits: torch.Tensor, full_recurrence: bool):
    """bf16 fused path of a look-back filter: (q, k, v) as (B, T, H, D) views."""
    NH, NKVH, Da, D = filt.n_head, filt.n_kv_head, filt.num_alpha_groups, filt.head_dim
    H = NH + 2 * NKVH
    if (full_recurrence and x.size(1) == 1 and not torch.is_grad_enabled()
            and hm_fast.decode_ok(x.size(2), D)):
        inits = resolved_inits.to(torch.bfloat16)
        # one recurrence step from the cached rows: the fused decode kernel
        wpack = hm_fast.cached_packed_weight(filt, H, D, Da)
        out = hm_fast.decode_step(x, wpack, (inits[:, :NH], inits[:, NH:NH + NKVH],
                                             inits[:, NH + NKVH:]),
                                  filt.logit_bias.detach().float().contiguous(), NH, NKVH, Da,
                                  filt.r)
        return (out[:, :NH].unsqueeze(1), out[:, NH:NH + NKVH].unsqueeze(1),
                out[:, NH + NKVH:].unsqueeze(1))
    P, Q, K = filt.chunking(full_recurrence)
    if resolved_inits.dtype == torch.float32 and hm_fast.fp32_inits_ok(x.size(1), D, filt.r, P, Q, K):
        # the kernels round fp32 inits to bf16 as they read them and return
        # their gradient as the widened bf16 one -- what .to(bfloat16) and its
        # backward give, without the two conversion launches
        inits = resolved_inits
    else:
        inits = resolved_inits.to(torch.bfloat16).contiguous()
    hq, hk, hv, _, _, _ = hm_fast.qkv_filter_call(
        x.contiguous(), filt.c.weight, inits, filt.logit_bias.float().contiguous(),
        NH, NKVH, Da, filt.r, P, Q, K)
    return hq.transpose(1, 2), hk.transpose(1, 2), hv.transpose(1, 2)
