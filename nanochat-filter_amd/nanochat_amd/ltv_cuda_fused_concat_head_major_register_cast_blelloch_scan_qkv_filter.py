"""The drop-in LTV combined-QKV filter, running on the gfx950 HIP library.

Same class name, constructor, parameters and ``forward(x, previous_values) ->
(q, k, v)`` contract as the reference's
``nanochat/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter.py:21-73``:
q is (B, T, n_head, D) and k, v are (B, T, n_kv_head, D), each a transposed view
of a contiguous (B, H, T, D) buffer.

dtype policy (reference ``:24-49``): the filter computes in float32 when autocast
asks for float32, otherwise in the dtype of ``x``.
  * bf16: the fast path -- ``nanochat_amd::qkv_filter``: the bf16 MFMA
    projection (fp32 accumulation, the fp32 master weight cast to bf16 on the
    fly) writes values and logits straight into the head-major layout the
    scan streams, forward and backward in two fused ops.
  * fp32: the reference-layout ops ``fused_linear_transpose`` (B, F, T) and the
    ``nanochat_cuda`` scan op read through the transposed (B, T, F) view,
    exactly the reference's dataflow.
  * bf16 decode (one token per sequence, no autograd): one fused launch,
    ``ltv_qkv_decode_step``, from the previous rows the KV cache feeds back
    (or ``init_param``), with the packed bf16 weight reused across steps.
"""

import torch

import nanochat_amd.ops  # noqa: F401  (registers the ops)
from nanochat_amd.ltv.ltv_filter import LtvInitValues
from nanochat_amd.ltv_combined_head_major_qkv_filter import LtvCombinedHeadMajorQkvFilter
from nanochat_amd.ltv_fused_concat_register_cast_scan_util import (
    CUDA_SUPPORTS_NATIVE_BF16,
    resolve_inits_original_dtype,
    _SCAN_THREADS_FORWARD,
    _R_THREADS_FORWARD,
    _R_ITEMS_FORWARD,
    _SCAN_THREADS_BACKWARD,
    _R_THREADS_BACKWARD,
    _R_ITEMS_BACKWARD,
)
from nanochat_amd.ops import ltv_hm_fast as hm_fast
from nanochat_amd.ops.ltv_cuda_ops import (
    fused_linear_transpose,
    ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan,
)


class _BatchSharedInits(torch.autograd.Function):
    """``init_param`` (H, D) as the bf16 inits of every sequence: its bf16
    rounding broadcast to (B, H, D) as a view with batch stride 0, which the
    scan kernels read in place.  The gradient is the batch sum of the (B, H, D)
    bf16 inits gradient, accumulated in float32: what the cast's and the
    broadcast's backward compute (``init_param.expand(B, H, D).to(bfloat16)``),
    in one reduction instead of a cast, a (B, H, D) copy and a reduction.
    Used for gate shapes whose scan takes no (H, D) inits; for the others the
    parameter goes to the scan as it is (``_shared_inits_in_kernel``), which
    does the rounding and the batch sum itself."""

    @staticmethod
    def forward(ctx, init_param, B):
        ctx.param_dtype = init_param.dtype
        return init_param.to(torch.bfloat16).unsqueeze(0).expand(B, -1, -1)

    @staticmethod
    def backward(ctx, grad):
        return grad.sum(0, dtype=torch.float32).to(ctx.param_dtype), None


class LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter(
    LtvCombinedHeadMajorQkvFilter
):
    def __init__(self, n_head: int, n_kv_head: int, head_dim: int, r: int):
        super().__init__(n_head, n_kv_head, head_dim, r)
        # loading a checkpoint replaces c.weight's values: drop the decode
        # path's packed copy of it
        self.register_load_state_dict_post_hook(
            lambda module, incompatible_keys: hm_fast.invalidate_packed_weight(module))

    def invalidate_packed_weight(self):
        """Drop the decode path's packed bf16 copy of ``c.weight``.  Needed only
        after writing the weight through ``c.weight.data`` (which does not bump
        the parameter's version counter); optimizer steps, in-place updates of
        the parameter and ``load_state_dict`` are tracked."""
        hm_fast.invalidate_packed_weight(self)

    def _compute_dtype(self, x):
        autocast_dtype = torch.get_autocast_dtype("cuda")
        run_ltv_in_fp32 = (
            autocast_dtype == torch.float32 if CUDA_SUPPORTS_NATIVE_BF16 else True
        )
        return torch.float32 if run_ltv_in_fp32 else x.dtype

    def decode_into_rows(self, x, previous_values: LtvInitValues, rows):
        """``forward``'s fused T = 1 bf16 decode step from the cache's previous
        rows, which also stores the new last rows into ``rows`` (q, k, v, e.g.
        the KV cache's last-row buffers, which may be the previous rows
        themselves) in the same launch.  Returns (q, k, v) as ``forward`` does,
        or None where ``forward`` would not take that path (then nothing is
        written).  Also None unless every row buffer is a bf16 tensor on x's
        device with contiguous channels (stride(-1) == 1), as the kernel
        stores them: a cache filled by an fp32 prefill, say, then takes the
        general path and the module's own row update."""
        if (x.size(1) != 1 or torch.is_grad_enabled() or previous_values.q is None
                or any(t is None for t in rows)
                or self._compute_dtype(x) != torch.bfloat16
                or not hm_fast.decode_ok(x.size(2), self.head_dim)):
            return None
        if any(t.dtype != torch.bfloat16 or t.device != x.device or t.stride(-1) != 1
               for t in rows):
            return None
        return self._decode_bf16(x, previous_values, rows)

    def forward(self, x, previous_values: LtvInitValues):
        B, _, C = x.size()
        compute_dtype = self._compute_dtype(x)
        if compute_dtype == torch.bfloat16 and not hm_fast.fast_path_ok(C, self.head_dim):
            return self._forward_bf16_dataflow(x, previous_values)
        if (compute_dtype == torch.bfloat16 and x.size(1) == 1 and not torch.is_grad_enabled()
                and hm_fast.decode_ok(C, self.head_dim)):
            return self._decode_bf16(x, previous_values)
        if compute_dtype == torch.bfloat16:
            if previous_values.q is None and self._shared_inits_in_kernel():
                # the (H, D) parameter itself: the scan reads it for every
                # sequence, rounding fp32 to bf16, and returns its gradient
                # summed over the batch
                inits = self.init_param
            elif previous_values.q is None:
                inits = _BatchSharedInits.apply(self.init_param, B)
            else:
                inits = resolve_inits_original_dtype(B, self.init_param, previous_values).to(
                    dtype=torch.bfloat16).contiguous()
            return self._forward_bf16(x, inits)
        inits = resolve_inits_original_dtype(B, self.init_param, previous_values)
        if compute_dtype != torch.float32:
            raise TypeError(f"LTV filter computes in bfloat16 or float32, not {compute_dtype}")
        return self._forward_fp32(x, inits)

    def _shared_inits_in_kernel(self):
        return (self.init_param.dtype in (torch.float32, torch.bfloat16)
                and hm_fast.shared_inits_ok(self.head_dim, self.num_alpha_groups, self.r))

    def _forward_bf16(self, x, inits):
        """inits: (B, H, D) bf16, contiguous or the batch-shared view, or the
        (H, D) parameter (fp32 or bf16) shared by every sequence."""
        hq, hk, hv, _, _, _ = hm_fast.qkv_filter_call(
            x.to(torch.bfloat16).contiguous(),
            self.c.weight,
            inits,
            self.logit_bias.float().contiguous(),
            self.n_head,
            self.n_kv_head,
            self.num_alpha_groups,
            self.r,
        )
        return hq.transpose(1, 2), hk.transpose(1, 2), hv.transpose(1, 2)

    def _packed_weight(self):
        """The bf16 packed weight, reused until ``c.weight`` changes."""
        return hm_fast.cached_packed_weight(self, self.n_head + 2 * self.n_kv_head,
                                            self.head_dim, self.num_alpha_groups)

    def _decode_bf16(self, x, previous_values, rows=None):
        """T = 1 inference: one fused launch (projection of the new tokens and one
        recurrence step from the previous rows; the new rows also to ``rows``)."""
        B = x.size(0)
        NH, NKVH = self.n_head, self.n_kv_head
        if previous_values.q is not None:
            prev = (previous_values.q, previous_values.k, previous_values.v)
        else:
            ip = self.init_param.detach().to(torch.bfloat16)
            prev = (ip[:NH].unsqueeze(0).expand(B, -1, -1),
                    ip[NH:NH + NKVH].unsqueeze(0).expand(B, -1, -1),
                    ip[NH + NKVH:].unsqueeze(0).expand(B, -1, -1))
        bias = self.logit_bias
        if bias.dtype != torch.float32 or not bias.is_contiguous():
            bias = bias.detach().float().contiguous()
        out = hm_fast.decode_step(x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16),
                                  self._packed_weight(), prev, bias, NH, NKVH,
                                  self.num_alpha_groups, self.r, rows=rows)
        # (B, 1, nh, D) views of the new rows, in one split
        return out.unsqueeze(1).split((NH, NKVH, NKVH), dim=2)

    def _forward_bf16_dataflow(self, x, previous_values):
        """bf16 for the shapes the fused path does not take (C not a multiple
        of 8, D not of 4): the reference's dataflow in bf16 -- the projection
        into a (B, F, T) buffer with the weight rounded to bf16, then the scan
        through the transposed view."""
        bf = torch.bfloat16
        out_buf = fused_linear_transpose(x.to(bf).contiguous(), self.c.weight.to(bf).contiguous())
        kernel_combined = out_buf.transpose(1, 2)
        inits = resolve_inits_original_dtype(x.size(0), self.init_param, previous_values).to(
            dtype=bf).contiguous()
        hq, hk, hv = ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan(
            kernel_combined, inits, self.logit_bias.float().contiguous(), self.n_head,
            self.n_kv_head, self.num_alpha_groups, self.r,
            _SCAN_THREADS_FORWARD, _R_THREADS_FORWARD, _R_ITEMS_FORWARD,
            _SCAN_THREADS_BACKWARD, _R_THREADS_BACKWARD, _R_ITEMS_BACKWARD,
            True,  # use_sigmoid
        )
        return hq.transpose(1, 2), hk.transpose(1, 2), hv.transpose(1, 2)

    def _forward_fp32(self, x, inits):
        out_buf = fused_linear_transpose(x.float().contiguous(), self.c.weight.float().contiguous())
        kernel_combined = out_buf.transpose(1, 2)  # (B, T, F) view, strides (F*T, 1, T)
        hq, hk, hv = ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan(
            kernel_combined,
            inits.to(dtype=kernel_combined.dtype).contiguous(),
            self.logit_bias.float().contiguous(),
            self.n_head,
            self.n_kv_head,
            self.num_alpha_groups,
            self.r,
            _SCAN_THREADS_FORWARD,
            _R_THREADS_FORWARD,
            _R_ITEMS_FORWARD,
            _SCAN_THREADS_BACKWARD,
            _R_THREADS_BACKWARD,
            _R_ITEMS_BACKWARD,
            True,  # use_sigmoid
        )
        return hq.transpose(1, 2), hk.transpose(1, 2), hv.transpose(1, 2)
