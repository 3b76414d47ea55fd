"""Fast path of the filter module: bf16 MFMA projection straight into a
head-major split layout, and the scan over that layout.

Two ops in the ``nanochat_amd`` namespace, each with a fake implementation and
autograd:

``qkv_project(x, weight, H, D, Da) -> (combined, wpack)``
    x (B, T, C) bf16, weight (F, C) = the module's ``c.weight`` in its per-head
    interleaved row order (fp32 master or bf16).  ``wpack`` is the weight cast
    to bf16 with rows regrouped [values of all heads | logits | zero pad]
    (Fp rows); ``combined`` is (B, T, Fp) bf16 with column ``h*D + d`` = value
    channel d of head h and column ``H*D + h*Da + j`` = logit j of head h.
    Same product as the reference's ``fused_linear_transpose``
    (``cpp_ewma/src/fused_linear_transpose_forward.cu:23-58``), written in the
    layout the scan reads with 16-byte vectors.

``hm_scan(combined, inits, logit_bias, NH, NKVH, Da, r, use_sigmoid) -> (q, k, v)``
    The head-major gated EWMA scan of
    ``nanochat/ops/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py``
    over the split layout; outputs (B, NH|NKVH, T, D) contiguous.
"""

from __future__ import annotations

import torch

from nanochat_amd import _native as N


def packed_width(H: int, D: int, Da: int) -> int:
    F = H * D + H * Da
    return (F + 63) // 64 * 64


# ---------------------------------------------------------------------------
# projection
# ---------------------------------------------------------------------------
@torch.library.custom_op("nanochat_amd::qkv_project", mutates_args=())
def qkv_project(x: torch.Tensor, weight: torch.Tensor, H: int, D: int,
                Da: int) -> tuple[torch.Tensor, torch.Tensor]:
    N.require_device(x, weight)
    if x.dtype != torch.bfloat16:
        raise RuntimeError(f"qkv_project computes in bf16; x is {x.dtype}")
    if x.dim() != 3:
        raise RuntimeError(f"x must be (B, T, C), got {tuple(x.shape)}")
    B, T, C = x.shape
    F = H * (D + Da)
    if tuple(weight.shape) != (F, C):
        raise RuntimeError(f"weight must be {(F, C)}, got {tuple(weight.shape)}")
    x = x.contiguous()
    weight = weight.contiguous()
    Fp = packed_width(H, D, Da)
    lib = N.lib()
    st = N.stream_of(x)
    wpack = torch.empty((Fp, C), dtype=torch.bfloat16, device=x.device)
    with N.span("pack_weight"):
        rc = lib.ltv_qkv_pack_weight(N.dtype_code(weight.dtype), weight.data_ptr(),
                                     wpack.data_ptr(), H, D, Da, C, st)
    N.check(rc, "ltv_qkv_pack_weight")
    combined = torch.empty((B, T, Fp), dtype=torch.bfloat16, device=x.device)
    with N.span("qkv_project_fwd"):
        rc = lib.ltv_qkv_project_forward(x.data_ptr(), wpack.data_ptr(), combined.data_ptr(),
                                         B * T, C, Fp, st)
    N.check(rc, "ltv_qkv_project_forward")
    return combined, wpack


@qkv_project.register_fake
def _(x, weight, H, D, Da):
    B, T, C = x.shape
    Fp = packed_width(H, D, Da)
    return (x.new_empty((B, T, Fp), dtype=torch.bfloat16),
            x.new_empty((Fp, C), dtype=torch.bfloat16))


@torch.library.custom_op("nanochat_amd::qkv_project_backward", mutates_args=())
def qkv_project_backward(x: torch.Tensor, wpack: torch.Tensor, grad_combined: torch.Tensor,
                         H: int, D: int, Da: int) -> tuple[torch.Tensor, torch.Tensor]:
    B, T, C = x.shape
    M = B * T
    x = x.contiguous()
    grad_combined = grad_combined.contiguous()
    lib = N.lib()
    grad_x = torch.empty((B, T, C), dtype=torch.bfloat16, device=x.device)
    grad_w = torch.empty((H * (D + Da), C), dtype=torch.float32, device=x.device)
    ws_bytes = lib.ltv_qkv_project_backward_workspace_size(M, C, H, D, Da)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    with N.span("qkv_project_bwd"):
        rc = lib.ltv_qkv_project_backward(x.data_ptr(), wpack.data_ptr(),
                                          grad_combined.data_ptr(), grad_x.data_ptr(),
                                          grad_w.data_ptr(), ws.data_ptr(), ws_bytes,
                                          M, C, H, D, Da, N.stream_of(x))
    N.check(rc, "ltv_qkv_project_backward")
    return grad_x, grad_w


@qkv_project_backward.register_fake
def _(x, wpack, grad_combined, H, D, Da):
    B, T, C = x.shape
    return (x.new_empty((B, T, C), dtype=torch.bfloat16),
            x.new_empty((H * (D + Da), C), dtype=torch.float32))


def _project_setup(ctx, inputs, output):
    x, weight, H, D, Da = inputs
    _, wpack = output
    ctx.save_for_backward(x, wpack)
    ctx.shape = (H, D, Da)
    ctx.weight_dtype = weight.dtype


def _project_backward(ctx, grad_combined, grad_wpack):
    x, wpack = ctx.saved_tensors
    H, D, Da = ctx.shape
    if grad_combined is None:
        return None, None, None, None, None
    gx, gw = torch.ops.nanochat_amd.qkv_project_backward(x, wpack, grad_combined, H, D, Da)
    if ctx.weight_dtype != torch.float32:
        gw = gw.to(ctx.weight_dtype)
    return gx, gw, None, None, None


qkv_project.register_autograd(_project_backward, setup_context=_project_setup)


# ---------------------------------------------------------------------------
# scan over the split layout
# ---------------------------------------------------------------------------
def _split_views(combined: torch.Tensor, H: int, D: int, Da: int):
    """(B, T, Fp) -> (values view strides, logits pointer, logits strides) as (b, h, t, c)."""
    sb, st, sc = combined.stride()
    vals = (sb, D * sc, st, sc)
    lg_off = H * D * sc * combined.element_size()
    lgs = (sb, Da * sc, st, sc)
    return vals, lg_off, lgs


def _arr(s):
    import ctypes
    return (ctypes.c_int64 * len(s))(*s)


@torch.library.custom_op("nanochat_amd::hm_scan", mutates_args=())
def hm_scan(combined: torch.Tensor, inits: torch.Tensor, logit_bias: torch.Tensor, NH: int,
            NKVH: int, Da: int, r: int,
            use_sigmoid: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    N.require_device(combined, inits, logit_bias)
    B, T, Fp = combined.shape
    H = NH + 2 * NKVH
    D = Da * r
    if Fp < H * (D + Da):
        raise RuntimeError(f"combined width {Fp} < H*(D+Da) = {H * (D + Da)}")
    if inits.dtype != combined.dtype or tuple(inits.shape) != (B, H, D):
        raise RuntimeError("inits must be (B, H, D) in combined's dtype")
    if logit_bias.dtype != torch.float32 or not logit_bias.is_contiguous():
        raise RuntimeError("logit_bias must be contiguous float32")
    out = [torch.empty((B, nh, T, D), dtype=combined.dtype, device=combined.device)
           for nh in (NH, NKVH, NKVH)]
    vals, lg_off, lgs = _split_views(combined, H, D, Da)
    with N.span("scan_fwd"):
      rc = N.lib().ltv_hm_scan_forward_split(
        N.dtype_code(combined.dtype),
        combined.data_ptr(), _arr(vals), combined.data_ptr() + lg_off, _arr(lgs),
        inits.data_ptr(), N.strides(inits, 3), logit_bias.data_ptr(),
        out[0].data_ptr(), N.strides(out[0], 4), out[1].data_ptr(), N.strides(out[1], 4),
        out[2].data_ptr(), N.strides(out[2], 4),
        B, T, NH, NKVH, Da, r, int(bool(use_sigmoid)), N.stream_of(combined))
    N.check(rc, "ltv_hm_scan_forward_split")
    return out[0], out[1], out[2]


@hm_scan.register_fake
def _(combined, inits, logit_bias, NH, NKVH, Da, r, use_sigmoid):
    B, T, _ = combined.shape
    D = Da * r
    return tuple(combined.new_empty((B, nh, T, D)) for nh in (NH, NKVH, NKVH))


@torch.library.custom_op("nanochat_amd::hm_scan_backward", mutates_args=())
def hm_scan_backward(combined: torch.Tensor, inits: torch.Tensor, logit_bias: torch.Tensor,
                     hq: torch.Tensor, hk: torch.Tensor, hv: torch.Tensor,
                     gq: torch.Tensor, gk: torch.Tensor, gv: torch.Tensor, NH: int, NKVH: int,
                     Da: int, r: int,
                     use_sigmoid: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, T, Fp = combined.shape
    H = NH + 2 * NKVH
    D = Da * r
    grad_combined = torch.empty_like(combined)
    grad_inits = torch.empty((B, H, D), dtype=inits.dtype, device=inits.device)
    grad_bias = torch.empty((H, Da), dtype=torch.float32, device=combined.device)
    dt = N.dtype_code(combined.dtype)
    lib = N.lib()
    ws_bytes = lib.ltv_hm_scan_backward_workspace_size(dt, B, T, NH, NKVH, Da, r)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=combined.device)
    vals, lg_off, lgs = _split_views(combined, H, D, Da)
    gvals, glg_off, glgs = _split_views(grad_combined, H, D, Da)
    with N.span("scan_bwd"):
      rc = lib.ltv_hm_scan_backward_split(
        dt,
        combined.data_ptr(), _arr(vals), combined.data_ptr() + lg_off, _arr(lgs),
        inits.data_ptr(), N.strides(inits, 3), logit_bias.data_ptr(),
        hq.data_ptr(), N.strides(hq, 4), hk.data_ptr(), N.strides(hk, 4),
        hv.data_ptr(), N.strides(hv, 4),
        gq.data_ptr(), N.strides(gq, 4), gk.data_ptr(), N.strides(gk, 4),
        gv.data_ptr(), N.strides(gv, 4),
        grad_combined.data_ptr(), _arr(gvals), grad_combined.data_ptr() + glg_off, _arr(glgs),
        grad_inits.data_ptr(), N.strides(grad_inits, 3), grad_bias.data_ptr(),
        ws.data_ptr(), ws_bytes, B, T, NH, NKVH, Da, r, int(bool(use_sigmoid)),
        N.stream_of(combined))
    N.check(rc, "ltv_hm_scan_backward_split")
    return grad_combined, grad_inits, grad_bias


@hm_scan_backward.register_fake
def _(combined, inits, logit_bias, hq, hk, hv, gq, gk, gv, NH, NKVH, Da, r, use_sigmoid):
    B, T, _ = combined.shape
    H = NH + 2 * NKVH
    D = Da * r
    return (torch.empty_like(combined), inits.new_empty((B, H, D)),
            combined.new_empty((H, Da), dtype=torch.float32))


def _scan_setup(ctx, inputs, output):
    combined, inits, logit_bias, NH, NKVH, Da, r, use_sigmoid = inputs
    ctx.save_for_backward(combined, inits, logit_bias, *output)
    ctx.args = (NH, NKVH, Da, r, use_sigmoid)


def _scan_backward(ctx, gq, gk, gv):
    combined, inits, logit_bias, hq, hk, hv = ctx.saved_tensors
    gq = torch.zeros_like(hq) if gq is None else gq
    gk = torch.zeros_like(hk) if gk is None else gk
    gv = torch.zeros_like(hv) if gv is None else gv
    gc, gi, gb = torch.ops.nanochat_amd.hm_scan_backward(
        combined, inits, logit_bias, hq, hk, hv, gq, gk, gv, *ctx.args)
    return gc, gi, gb.view_as(logit_bias), None, None, None, None, None


hm_scan.register_autograd(_scan_backward, setup_context=_scan_setup)
