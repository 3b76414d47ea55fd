"""torch.library schemas of the LTV combined-QKV path, plus functional wrappers.

Mirrors the reference's ``nanochat/ops/ltv_cuda_ops.py`` for the ops on this
path (schemas at ``:115-145`` and ``:242-250``; wrappers ``:256-299``), under
the same ``nanochat_cuda`` namespace so callers written against the reference
(``torch.ops.nanochat_cuda.<op>``) run unchanged.  The implementations are in
``fused_linear_transpose.py`` and
``ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py`` and call the
gfx950 HIP library through its C ABI.

The legacy-layout scan op (``:89-113``) is implemented in
``ltv_cuda_fused_concat_register_cast_blelloch_scan.py``; the look-back ops
(``:172-241``, wrappers ``:332-410``) in
``ltv_cuda_look_back_fused_concat_head_major_register_cast_{blelloch,sequential}_scan.py``.

The filter module's own fast path uses two further ops in the ``nanochat_amd``
namespace (``ltv_hm_fast.py``).
"""

import torch

lib = torch.library.Library("nanochat_cuda", "DEF")

lib.define(
    "ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "int NH, int NKVH, int da, int r, "
    "int scan_threads_forward, int r_threads_forward, int r_items_forward, "
    "int scan_threads_backward, int r_threads_backward, int r_items_backward, "
    "bool use_sigmoid"
    ") -> (Tensor, Tensor, Tensor)"
)

lib.define(
    "ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward_kernel("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "Tensor(a!) out_q, Tensor(b!) out_k, Tensor(c!) out_v, "
    "int T, int NH, int NKVH, int da, int r, "
    "int scan_threads_forward, int r_threads_forward, int r_items_forward, "
    "bool use_sigmoid"
    ") -> ()"
)

lib.define(
    "ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward_kernel("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "Tensor hq, Tensor hk, Tensor hv, "
    "Tensor grad_hq, Tensor grad_hk, Tensor grad_hv, "
    "Tensor(a!) grad_combined, Tensor(b!) grad_inits, Tensor(c!) grad_logit_bias, "
    "int NH, int NKVH, int da, int r, "
    "int scan_threads_backward, int r_threads_backward, int r_items_backward, "
    "bool use_sigmoid"
    ") -> ()"
)

# Legacy projection layout [q | k | v | logits] (bias pre-added), schemas of the
# reference's ops/ltv_cuda_ops.py:89-113.
lib.define(
    "ltv_fused_concat_register_cast_blelloch_scan_cuda_op("
    "Tensor combined, Tensor inits, "
    "int NH, int NKVH, int da, int r, int chunk_size, int bank_count, bool use_sigmoid"
    ") -> (Tensor, Tensor, Tensor)"
)

lib.define(
    "ltv_fused_concat_register_cast_blelloch_scan_cuda_forward_kernel("
    "Tensor combined, Tensor inits, "
    "Tensor(a!) out_q, Tensor(b!) out_k, Tensor(c!) out_v, "
    "int T, int NH, int NKVH, int da, int r, int chunk_size, int bank_count, bool use_sigmoid"
    ") -> ()"
)

lib.define(
    "ltv_fused_concat_register_cast_blelloch_scan_cuda_backward_kernel("
    "Tensor combined, Tensor inits, "
    "Tensor hq, Tensor hk, Tensor hv, "
    "Tensor grad_hq, Tensor grad_hk, Tensor grad_hv, "
    "Tensor(a!) grad_combined, Tensor(b!) grad_inits, "
    "Tensor(c!) grad_logits, "
    "int NH, int NKVH, int da, int r, int chunk_size, int bank_count, bool use_sigmoid"
    ") -> ()"
)

# Look-back variants (chunk restarts with a K - 1 step warm-up), schemas of the
# reference's ops/ltv_cuda_ops.py:172-241.
lib.define(
    "ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_op("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "int NH, int NKVH, int da, int r, "
    "int P, int Q, int K, "
    "int scan_threads_forward, int r_threads_forward, int r_items_forward, "
    "int scan_threads_backward, int r_threads_backward, int r_items_backward, "
    "bool use_sigmoid"
    ") -> (Tensor, Tensor, Tensor)"
)

lib.define(
    "ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_forward_kernel("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "Tensor(a!) out_q, Tensor(b!) out_k, Tensor(c!) out_v, "
    "int B, int T, int NH, int NKVH, int da, int r, "
    "int P, int Q, int K, "
    "int scan_threads_forward, int r_threads_forward, int r_items_forward, "
    "bool use_sigmoid"
    ") -> ()"
)

lib.define(
    "ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward_kernel("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "Tensor hq, Tensor hk, Tensor hv, "
    "Tensor grad_hq, Tensor grad_hk, Tensor grad_hv, "
    "Tensor(a!) grad_combined, Tensor(b!) grad_inits, Tensor(c!) grad_logit_bias, "
    "int NH, int NKVH, int da, int r, "
    "int P, int Q, int K, "
    "int scan_threads_backward, int r_threads_backward, int r_items_backward, "
    "bool use_sigmoid"
    ") -> ()"
)

lib.define(
    "ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_op("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "int NH, int NKVH, int da, int r, "
    "int P, int Q, int K, "
    "int r_threads_forward, int r_items_forward, "
    "int r_threads_backward, int r_items_backward, "
    "bool use_sigmoid"
    ") -> (Tensor, Tensor, Tensor)"
)

lib.define(
    "ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_forward_kernel("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "Tensor(a!) out_q, Tensor(b!) out_k, Tensor(c!) out_v, "
    "int B, int T, int NH, int NKVH, int da, int r, "
    "int P, int Q, int K, "
    "int r_threads_forward, int r_items_forward, "
    "bool use_sigmoid"
    ") -> ()"
)

lib.define(
    "ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_backward_kernel("
    "Tensor combined, Tensor inits, Tensor logit_bias, "
    "Tensor hq, Tensor hk, Tensor hv, "
    "Tensor grad_hq, Tensor grad_hk, Tensor grad_hv, "
    "Tensor(a!) grad_combined, Tensor(b!) grad_inits, Tensor(c!) grad_logit_bias, "
    "int NH, int NKVH, int da, int r, "
    "int P, int Q, int K, "
    "int r_threads_backward, int r_items_backward, "
    "bool use_sigmoid"
    ") -> ()"
)

lib.define("fused_linear_transpose(Tensor x, Tensor weight, Tensor(a!) out) -> ()")

lib.define("fused_linear_transpose_cuda_op(Tensor x, Tensor weight) -> Tensor")

lib.define(
    "fused_linear_transpose_backward_kernel("
    "Tensor x, Tensor weight, Tensor grad_out, Tensor(a!) grad_x, Tensor(b!) grad_weight"
    ") -> ()"
)


import nanochat_amd.ops.fused_linear_transpose  # noqa: E402,F401  (registers impls)
import nanochat_amd.ops.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan  # noqa: E402,F401
import nanochat_amd.ops.ltv_cuda_fused_concat_register_cast_blelloch_scan  # noqa: E402,F401
import nanochat_amd.ops.ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan  # noqa: E402,F401
import nanochat_amd.ops.ltv_cuda_look_back_fused_concat_head_major_register_cast_sequential_scan  # noqa: E402,F401
import nanochat_amd.ops.ltv_cuda_meta  # noqa: E402,F401


def fused_linear_transpose(x: torch.Tensor, weight: torch.Tensor):
    """Returns a new (B, F, T) contiguous tensor ``out[b] = weight @ x[b]^T``
    (reference wrapper ``ops/ltv_cuda_ops.py:256-263``)."""
    return torch.ops.nanochat_cuda.fused_linear_transpose_cuda_op(x, weight)


def ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan(
    combined: torch.Tensor,
    inits: torch.Tensor,
    logit_bias: torch.Tensor,
    NH: int,
    NKVH: int,
    da: int,
    r: int,
    scan_threads_forward: int,
    r_threads_forward: int,
    r_items_forward: int,
    scan_threads_backward: int,
    r_threads_backward: int,
    r_items_backward: int,
    use_sigmoid: bool,
):
    """Reference wrapper ``ops/ltv_cuda_ops.py:266-299``."""
    return torch.ops.nanochat_cuda.ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op(
        combined,
        inits,
        logit_bias,
        NH,
        NKVH,
        da,
        r,
        scan_threads_forward,
        r_threads_forward,
        r_items_forward,
        scan_threads_backward,
        r_threads_backward,
        r_items_backward,
        use_sigmoid,
    )


def ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan(
    combined: torch.Tensor,
    inits: torch.Tensor,
    logit_bias: torch.Tensor,
    NH: int,
    NKVH: int,
    da: int,
    r: int,
    P: int,
    Q: int,
    K: int,
    scan_threads_forward: int,
    r_threads_forward: int,
    r_items_forward: int,
    scan_threads_backward: int,
    r_threads_backward: int,
    r_items_backward: int,
    use_sigmoid: bool,
):
    """Reference wrapper ``ops/ltv_cuda_ops.py:332-371``."""
    return torch.ops.nanochat_cuda.ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_op(
        combined, inits, logit_bias, NH, NKVH, da, r, P, Q, K,
        scan_threads_forward, r_threads_forward, r_items_forward,
        scan_threads_backward, r_threads_backward, r_items_backward, use_sigmoid,
    )


def ltv_cuda_look_back_fused_concat_head_major_register_cast_sequential_scan(
    combined: torch.Tensor,
    inits: torch.Tensor,
    logit_bias: torch.Tensor,
    NH: int,
    NKVH: int,
    da: int,
    r: int,
    P: int,
    Q: int,
    K: int,
    r_threads_forward: int,
    r_items_forward: int,
    r_threads_backward: int,
    r_items_backward: int,
    use_sigmoid: bool,
):
    """Reference wrapper ``ops/ltv_cuda_ops.py:374-410``."""
    return torch.ops.nanochat_cuda.ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_op(
        combined, inits, logit_bias, NH, NKVH, da, r, P, Q, K,
        r_threads_forward, r_items_forward, r_threads_backward, r_items_backward, use_sigmoid,
    )
