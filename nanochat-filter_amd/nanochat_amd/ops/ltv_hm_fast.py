"""Fast path of the filter module: the bf16 MFMA projection writes the scan's
head-major layout directly, and the gated EWMA scan runs over it.

Buffers (H = NH + 2 NKVH filtered heads, Da = D / r gate logits per head,
M = B T tokens):
  values  (B, H, T, D) bf16, contiguous   -- head-major, what the scan streams
  logits  (B, T, Lp)   bf16, contiguous   -- column h Da + j = logit j of head h
  grad_combined (B, T, Fp) bf16           -- the scan backward's output and the
            projection backward's input: column h D + d = d(value d of head h),
            column H D + h Da + j = d(logit j of head h), the rest padding
with Fp = ``packed_width`` and Lp = ``logit_width``.

Ops in the ``nanochat_amd`` namespace, each with a fake implementation:

``qkv_filter(x, weight, inits, logit_bias, NH, NKVH, Da, r, P, Q, K)``
    -> (q, k, v, values, logits, wpack).  q (B, NH, T, D), k and v
    (B, NKVH, T, D), contiguous.  inits (B, H, D) bf16, or the (H, D)
    parameter shared by every sequence (fp32 or bf16; ``shared_inits_ok``),
    whose gradient comes back summed over the batch.  The last three outputs are the intermediates
    the backward reads; callers use only q, k, v.  Same result as the
    reference's ``fused_linear_transpose`` (``cpp_ewma/src/fused_linear_transpose_forward.cu:23-58``)
    followed by its head-major scan
    (``nanochat/ops/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py``),
    with a bf16 copy of the weight as the MFMA operand.  Autograd through
    ``qkv_filter_backward``: the scan backward writes grad_combined, then the
    projection backward reads it (grad_x, and grad_weight in fp32).
    (P, Q, K) are the look-back chunking of
    ``nanochat/ops/ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan.py``;
    the default P = 2**31 - 1 is the full recurrence.

The helpers ``project``, ``project_backward``, ``scan_forward`` and
``scan_backward`` call the library directly; the tests use them to check each
stage on its own.  ``decode_step`` is the fused T = 1 inference step (one
launch: projection of the new tokens plus one recurrence step from the previous
rows), with ``pack_weight`` giving the weight operand it reuses across steps.
"""

from __future__ import annotations

import ctypes

import torch

from nanochat_amd import _native as N

UNBOUNDED_P = 2_147_483_647  # look-back P of the full recurrence (one chunk window)


def packed_width(H: int, D: int, Da: int) -> int:
    F = H * (D + Da)
    return (F + 127) // 128 * 128


def logit_width(H: int, Da: int) -> int:
    return (H * Da + 7) // 8 * 8


_ARR_CACHE: dict = {}


def _arr(s):
    """An int64 ctypes array of s.  The arrays of recurring stride tuples are
    kept (the library only reads them during the call), which saves their
    construction on every decode step."""
    key = tuple(s)
    a = _ARR_CACHE.get(key)
    if a is None:
        a = (ctypes.c_int64 * len(key))(*key)
        if len(_ARR_CACHE) < 4096:
            _ARR_CACHE[key] = a
    return a


# ---------------------------------------------------------------------------
# library calls
# ---------------------------------------------------------------------------
def project(x: torch.Tensor, weight: torch.Tensor, H: int, D: int, Da: int):
    """x (B, T, C) bf16, weight (F, C) fp32/bf16 -> (values, logits, wpack)."""
    N.require_device(x, weight)
    if x.dtype != torch.bfloat16:
        raise RuntimeError(f"the projection computes in bf16; x is {x.dtype}")
    if x.dim() != 3:
        raise RuntimeError(f"x must be (B, T, C), got {tuple(x.shape)}")
    B, T, C = x.shape
    F = H * (D + Da)
    if tuple(weight.shape) != (F, C):
        raise RuntimeError(f"weight must be {(F, C)}, got {tuple(weight.shape)}")
    x = x.contiguous()
    weight = weight.contiguous()
    Fp, Lp = packed_width(H, D, Da), logit_width(H, Da)
    lib = N.lib()
    st = N.stream_of(x)
    wpack = torch.empty((Fp, C), dtype=torch.bfloat16, device=x.device)
    with N.span("pack_weight"):
        rc = lib.ltv_qkv_pack_weight(N.dtype_code(weight.dtype), weight.data_ptr(),
                                     wpack.data_ptr(), H, D, Da, C, st)
    N.check(rc, "ltv_qkv_pack_weight")
    values = torch.empty((B, H, T, D), dtype=torch.bfloat16, device=x.device)
    logits = torch.empty((B, T, Lp), dtype=torch.bfloat16, device=x.device)
    with N.span("qkv_project_fwd"):
        rc = lib.ltv_qkv_project_forward(x.data_ptr(), wpack.data_ptr(), values.data_ptr(),
                                         logits.data_ptr(), B, T, C, H, D, Da, st)
    N.check(rc, "ltv_qkv_project_forward")
    return values, logits, wpack


def pack_weight(weight: torch.Tensor, H: int, D: int, Da: int) -> torch.Tensor:
    """weight (F, C) fp32/bf16 -> the packed bf16 (Fp, C) MFMA operand."""
    N.require_device(weight)
    F, C = weight.shape
    if F != H * (D + Da):
        raise RuntimeError(f"weight must have {H * (D + Da)} rows, got {F}")
    weight = weight.contiguous()
    wpack = torch.empty((packed_width(H, D, Da), C), dtype=torch.bfloat16, device=weight.device)
    with N.span("pack_weight"):
        rc = N.lib().ltv_qkv_pack_weight(N.dtype_code(weight.dtype), weight.data_ptr(),
                                         wpack.data_ptr(), H, D, Da, C, N.stream_of(weight))
    N.check(rc, "ltv_qkv_pack_weight")
    return wpack


def cached_packed_weight(module, H: int, D: int, Da: int) -> torch.Tensor:
    """The packed bf16 weight of ``module.c.weight``, kept on the module and
    rebuilt when the weight changes: in-place updates of the Parameter (an
    optimizer step, ``copy_`` under ``no_grad``) bump its version counter, and
    ``load_state_dict`` drops the cache.  Writes through ``weight.data`` do not
    bump the version; after one, call ``invalidate_packed_weight(module)``."""
    w = module.c.weight
    key = (w.data_ptr(), w._version, w.dtype, w.device)
    cached = getattr(module, "_wpack_cache", None)
    if cached is None or cached[0] != key:
        cached = (key, pack_weight(w.detach(), H, D, Da))
        module._wpack_cache = cached
    return cached[1]


def invalidate_packed_weight(module) -> None:
    """Drop the packed weight cached by ``cached_packed_weight``."""
    module._wpack_cache = None


def decode_step(x: torch.Tensor, wpack: torch.Tensor, prev, logit_bias: torch.Tensor, NH: int,
                NKVH: int, Da: int, r: int, use_sigmoid: bool = True, rows=None) -> torch.Tensor:
    """One fused decode step: x (B, C) or (B, 1, C) bf16, the packed weight, the
    previous output rows ``prev = (q (B, NH, D), k (B, NKVH, D), v (B, NKVH, D))``
    bf16 with channel stride 1 -> the new rows (B, H, D) bf16, contiguous.
    rows: three more (B, nh, D) bf16 tensors, channel stride 1, that receive the
    new rows as well -- e.g. the KV cache's last-row buffers, which may be the
    prev tensors themselves (the kernel reads each previous element before
    the same thread overwrites it)."""
    if x.dim() == 3:
        if x.shape[1] != 1:
            raise RuntimeError(f"decode_step takes one token per sequence, got x {tuple(x.shape)}")
        # (B, 1, C): token b's row starts b * stride(0) elements in, as in (B, C)
        B, _, C = x.shape
        x_rs, x_cs = x.stride(0), x.stride(2)
    else:
        B, C = x.shape
        x_rs, x_cs = x.stride(0), x.stride(1)
    N.require_device(x, wpack, logit_bias, *prev)
    if x.dtype != torch.bfloat16 or wpack.dtype != torch.bfloat16:
        raise RuntimeError("decode_step computes in bf16")
    D = Da * r
    H = NH + 2 * NKVH
    if x_cs != 1 or x_rs % 8 != 0:
        x = x.reshape(B, C).contiguous()
        x_rs = C
    prevs = []
    for t, nh in zip(prev, (NH, NKVH, NKVH)):
        if t.dtype != torch.bfloat16:
            t = t.to(torch.bfloat16)
        if tuple(t.shape) != (B, nh, D):
            raise RuntimeError(f"previous rows must be {(B, nh, D)}, got {tuple(t.shape)}")
        if t.stride(2) != 1:
            t = t.contiguous()
        prevs.append(t)
    if logit_bias.dtype != torch.float32 or not logit_bias.is_contiguous():
        raise RuntimeError("logit_bias must be contiguous float32")
    out = torch.empty((B, H, D), dtype=torch.bfloat16, device=x.device)
    strides = _arr([s for t in prevs for s in t.stride()[:2]])
    if rows is None:
        with N.span("qkv_decode"):
            rc = N.lib().ltv_qkv_decode_step(x.data_ptr(), x_rs, wpack.data_ptr(),
                                             prevs[0].data_ptr(), prevs[1].data_ptr(),
                                             prevs[2].data_ptr(), strides, logit_bias.data_ptr(),
                                             out.data_ptr(), B, C, NH, NKVH, D, Da,
                                             int(use_sigmoid), N.stream_of(x))
        N.check(rc, "ltv_qkv_decode_step")
        return out
    if all(a is b for a, b in zip(rows, prevs)):
        rstrides = strides  # the rows are the previous rows, checked above (the cache in place)
    else:
        for t, nh in zip(rows, (NH, NKVH, NKVH)):
            if (t.dtype != torch.bfloat16 or tuple(t.shape) != (B, nh, D) or t.stride(2) != 1
                    or t.device != x.device):
                raise RuntimeError(f"rows must be ({B}, {nh}, {D}) bf16 with channel stride 1 on "
                                   f"{x.device}, got {tuple(t.shape)} {t.dtype} {t.device}")
        rstrides = _arr([s for t in rows for s in t.stride()[:2]])
    with N.span("qkv_decode"):
        rc = N.lib().ltv_qkv_decode_step_rows(x.data_ptr(), x_rs, wpack.data_ptr(),
                                              prevs[0].data_ptr(), prevs[1].data_ptr(),
                                              prevs[2].data_ptr(), strides, logit_bias.data_ptr(),
                                              out.data_ptr(), rows[0].data_ptr(),
                                              rows[1].data_ptr(), rows[2].data_ptr(), rstrides,
                                              B, C, NH, NKVH, D, Da, int(use_sigmoid),
                                              N.stream_of(x))
    N.check(rc, "ltv_qkv_decode_step_rows")
    return out


def project_backward(x: torch.Tensor, wpack: torch.Tensor, grad_combined: torch.Tensor, H: int,
                     D: int, Da: int, pad_zeroed: bool = False):
    """grad_combined (B, T, Fp) -> (grad_x (B, T, C) bf16, grad_weight (F, C) fp32).
    pad_zeroed: columns F .. round_up(F, 8) - 1 of grad_combined are zero
    already (``scan_backward(..., zero_pad=True)``), so grad_x skips zeroing them."""
    B, T, C = x.shape
    M = B * T
    x = x.contiguous()
    grad_combined = grad_combined.contiguous()
    lib = N.lib()
    st = N.stream_of(x)
    grad_x = torch.empty((B, T, C), dtype=torch.bfloat16, device=x.device)
    grad_w = torch.empty((H * (D + Da), C), dtype=torch.float32, device=x.device)
    ws_bytes = lib.ltv_qkv_project_backward_workspace_size(M, C, H, D, Da)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    # both gradients in one call: the library runs the two GEMMs in one launch
    # where grad_x's tiles leave part of the device idle in their last round
    fn = (lib.ltv_qkv_project_backward_zero_padded if pad_zeroed
          else lib.ltv_qkv_project_backward)
    with N.span("qkv_project_bwd"):
        rc = fn(x.data_ptr(), wpack.data_ptr(), grad_combined.data_ptr(), grad_x.data_ptr(),
                grad_w.data_ptr(), ws.data_ptr(), ws_bytes, M, C, H, D, Da, st)
    N.check(rc, "ltv_qkv_project_backward")
    return grad_x, grad_w


def fast_path_ok(C: int, D: int) -> bool:
    """Whether the fused bf16 path (the head-major MFMA projection and its
    backward) takes this width and head size: C a multiple of 8 (16-byte rows
    of x and of the packed weight), D of 4.  The filters run other shapes
    through the reference dataflow (``fused_linear_transpose`` in bf16, then
    the scan op)."""
    return C % 8 == 0 and D % 4 == 0


def decode_ok(C: int, D: int) -> bool:
    """Whether the fused decode step takes this shape: the fused path's, with
    C a multiple of 16 (the step's k16 MFMA slices)."""
    return fast_path_ok(C, D) and C % 16 == 0


def shared_inits_ok(D: int, Da: int, r: int) -> bool:
    """Whether the bf16 scan takes one (H, D) set of inits for every sequence,
    fp32 or bf16, with the inits gradient summed over the batch by the
    library (gate groups the tile kernels reduce: r a multiple of 8 with at
    most 16 groups per head, or r dividing 8; 16-byte channel vectors)."""
    return D % 8 == 0 and ((r % 8 == 0 and Da <= 16) or 8 % r == 0)


def fp32_inits_ok(T: int, D: int, r: int, P: int, Q: int, K: int) -> bool:
    """Whether the bf16 scan takes (B, H, D) fp32 inits for this chunking: the
    full recurrence (P >= T) with gate groups the tile kernels reduce, or
    look-back windows the short-window kernels take (Q <= 64, a warm-up
    K - 1 <= min(Q, 16), gate groups of 8 2^k channels or dividing 8)."""
    if P >= T:  # the tile kernels' gate groups, as for shared inits
        return D % 8 == 0 and ((r % 8 == 0 and D // r <= 16) or 8 % r == 0)
    if Q > 64 or K - 1 > 16 or K - 1 > Q or D % 8:
        return False
    return (r % 8 == 0 and (r // 8) & (r // 8 - 1) == 0) or 8 % r == 0


def _inits_view(inits: torch.Tensor, values: torch.Tensor):
    """(strides (b, h, d), dtype code) of the inits: (B, H, D) per sequence,
    or (H, D) shared by every sequence (batch stride 0); the values' dtype,
    or fp32 with bf16 values (rounded to bf16 by the kernels)."""
    B, H, _, D = values.shape
    if inits.dim() == 2:
        if tuple(inits.shape) != (H, D):
            raise RuntimeError(f"shared inits must be {(H, D)}, got {tuple(inits.shape)}")
        st = (0, inits.stride(0), inits.stride(1))
    elif tuple(inits.shape) == (B, H, D):
        st = tuple(inits.stride())
    else:
        raise RuntimeError(f"inits must be {(B, H, D)} or {(H, D)}, got {tuple(inits.shape)}")
    if inits.dtype != values.dtype and not (inits.dtype == torch.float32
                                            and values.dtype == torch.bfloat16):
        raise RuntimeError(f"inits must be in the values' dtype, or float32 with bfloat16 "
                           f"values; got {inits.dtype} with {values.dtype}")
    return st, N.dtype_code(inits.dtype)


def scan_forward(values: torch.Tensor, logits: torch.Tensor, inits: torch.Tensor,
                 logit_bias: torch.Tensor, NH: int, NKVH: int, Da: int, r: int,
                 use_sigmoid: bool, P: int = UNBOUNDED_P, Q: int = 1, K: int = 1):
    """values (B, H, T, D); logits (B, T, >= H Da) with column h Da + j, or
    head-major (B, H, T, Da) -> out_q (B, NH, T, D), out_k, out_v (B, NKVH, T, D).
    inits: (B, H, D), or (H, D) for every sequence; fp32 inits with bf16 values
    are rounded to bf16 as they are read (the full recurrence only)."""
    N.require_device(values, logits, inits, logit_bias)
    B, H, T, D = values.shape
    if H != NH + 2 * NKVH or D != Da * r:
        raise RuntimeError("values shape does not match (NH, NKVH, Da, r)")
    ist, idt = _inits_view(inits, values)
    if logit_bias.dtype != torch.float32 or not logit_bias.is_contiguous():
        raise RuntimeError("logit_bias must be contiguous float32")
    out = [torch.empty((B, nh, T, D), dtype=values.dtype, device=values.device)
           for nh in (NH, NKVH, NKVH)]
    if logits.dim() == 4:  # head-major (B, H, T, Da)
        if tuple(logits.shape) != (B, H, T, Da) or logits.dtype != values.dtype:
            raise RuntimeError(f"head-major logits must be {(B, H, T, Da)} in the values' dtype")
        lgs = logits.stride()
    else:  # (B, T, >= H Da), column h Da + j
        sb, st_, sl = logits.stride()
        lgs = (sb, Da * sl, st_, sl)
    cw = (N.chain_workspace_for(values.dtype, values.device, B, T, NH, NKVH, Da, r)
          if P >= T else N._NO_CHAIN)
    with N.span("scan_fwd"):
        rc = N.lib().ltv_hm_look_back_scan_forward_split_ws(
            N.dtype_code(values.dtype),
            values.data_ptr(), N.strides(values, 4), logits.data_ptr(), _arr(lgs),
            inits.data_ptr(), _arr(ist), idt, logit_bias.data_ptr(),
            out[0].data_ptr(), N.strides(out[0], 4), out[1].data_ptr(), N.strides(out[1], 4),
            out[2].data_ptr(), N.strides(out[2], 4), cw.ptr, cw.nbytes,
            B, T, NH, NKVH, Da, r, P, Q, K, int(bool(use_sigmoid)), N.stream_of(values))
    N.check(rc, "ltv_hm_look_back_scan_forward_split_ws")
    N.chain_done(cw)
    return out[0], out[1], out[2]


def scan_backward(values, logits, inits, logit_bias, hq, hk, hv, gq, gk, gv, NH: int,
                  NKVH: int, Da: int, r: int, use_sigmoid: bool,
                  grad_combined: torch.Tensor, P: int = UNBOUNDED_P, Q: int = 1, K: int = 1,
                  zero_pad: bool = False):
    """Writes grad_combined (B, T, Fp); returns (grad_inits, grad_logit_bias).
    grad_inits is shaped like inits: with (H, D) inits it is the sum over the
    batch of every sequence's gradient (each rounded to the values' dtype,
    summed in fp32 in batch order), in the inits' dtype.  zero_pad: also set
    grad_combined's columns F .. round_up(F, 8) - 1 to zero (what
    ``project_backward(..., pad_zeroed=True)`` relies on)."""
    B, H, T, D = values.shape
    dt = N.dtype_code(values.dtype)
    lib = N.lib()
    ist, idt = _inits_view(inits, values)
    grad_inits = torch.empty(inits.shape, dtype=inits.dtype, device=inits.device)
    gist = ((0,) + tuple(grad_inits.stride())) if inits.dim() == 2 else tuple(grad_inits.stride())
    grad_bias = torch.empty((H, Da), dtype=torch.float32, device=values.device)
    ws_bytes = lib.ltv_hm_look_back_scan_backward_workspace_size(dt, B, T, NH, NKVH, Da, r,
                                                                 P, Q, K)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=values.device)
    sb, st_, sl = logits.stride()
    lgs = (sb, Da * sl, st_, sl)
    gsb, gst, gsc = grad_combined.stride()
    gvals = (gsb, D * gsc, gst, gsc)
    glgs = (gsb, Da * gsc, gst, gsc)
    glg_ptr = grad_combined.data_ptr() + H * D * gsc * grad_combined.element_size()
    F = H * (D + Da)
    pad = (-F) % 8 if zero_pad else 0
    cw = (N.chain_workspace_for(values.dtype, values.device, B, T, NH, NKVH, Da, r,
                                backward=True)
          if P >= T else N._NO_CHAIN)
    with N.span("scan_bwd"):
        rc = lib.ltv_hm_look_back_scan_backward_split_ws(
            dt,
            values.data_ptr(), N.strides(values, 4), logits.data_ptr(), _arr(lgs),
            inits.data_ptr(), _arr(ist), idt, logit_bias.data_ptr(),
            hq.data_ptr(), N.strides(hq, 4), hk.data_ptr(), N.strides(hk, 4),
            hv.data_ptr(), N.strides(hv, 4),
            gq.data_ptr(), N.strides(gq, 4), gk.data_ptr(), N.strides(gk, 4),
            gv.data_ptr(), N.strides(gv, 4),
            grad_combined.data_ptr(), _arr(gvals), glg_ptr, _arr(glgs), pad,
            grad_inits.data_ptr(), _arr(gist), grad_bias.data_ptr(),
            ws.data_ptr(), ws_bytes, cw.ptr, cw.nbytes, B, T, NH, NKVH, Da, r, P, Q, K,
            int(bool(use_sigmoid)), N.stream_of(values))
    N.check(rc, "ltv_hm_look_back_scan_backward_split_ws")
    N.chain_done(cw)
    return grad_inits, grad_bias


# ---------------------------------------------------------------------------
# the fused op
# ---------------------------------------------------------------------------
def _qkv_filter_impl(x, weight, inits, logit_bias, NH, NKVH, Da, r, P, Q, K):
    H = NH + 2 * NKVH
    D = Da * r
    values, logits, wpack = project(x, weight, H, D, Da)
    q, k, v = scan_forward(values, logits, inits, logit_bias, NH, NKVH, Da, r, True, P, Q, K)
    return q, k, v, values, logits, wpack


@torch.library.custom_op("nanochat_amd::qkv_filter", mutates_args=())
def qkv_filter(x: torch.Tensor, weight: torch.Tensor, inits: torch.Tensor,
               logit_bias: torch.Tensor, NH: int, NKVH: int, Da: int, r: int,
               P: int = UNBOUNDED_P, Q: int = 1,
               K: int = 1) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                    torch.Tensor, torch.Tensor]:
    return _qkv_filter_impl(x, weight, inits, logit_bias, NH, NKVH, Da, r, P, Q, K)


@qkv_filter.register_fake
def _(x, weight, inits, logit_bias, NH, NKVH, Da, r, P=UNBOUNDED_P, Q=1, K=1):
    B, T, C = x.shape
    H = NH + 2 * NKVH
    D = Da * r
    bf = torch.bfloat16
    return (x.new_empty((B, NH, T, D), dtype=bf), x.new_empty((B, NKVH, T, D), dtype=bf),
            x.new_empty((B, NKVH, T, D), dtype=bf), x.new_empty((B, H, T, D), dtype=bf),
            x.new_empty((B, T, logit_width(H, Da)), dtype=bf),
            x.new_empty((packed_width(H, D, Da), C), dtype=bf))


def _qkv_filter_backward_impl(x, wpack, values, logits, inits, logit_bias, hq, hk, hv, gq, gk,
                              gv, NH, NKVH, Da, r, P, Q, K):
    B, T, C = x.shape
    H = NH + 2 * NKVH
    D = Da * r
    grad_combined = torch.empty((B, T, packed_width(H, D, Da)), dtype=torch.bfloat16,
                                device=x.device)
    grad_inits, grad_bias = scan_backward(values, logits, inits, logit_bias, hq, hk, hv,
                                          gq.to(hq.dtype), gk.to(hk.dtype), gv.to(hv.dtype),
                                          NH, NKVH, Da, r, True, grad_combined, P, Q, K,
                                          zero_pad=True)
    grad_x, grad_w = project_backward(x, wpack, grad_combined, H, D, Da, pad_zeroed=True)
    return grad_x, grad_w, grad_inits, grad_bias


@torch.library.custom_op("nanochat_amd::qkv_filter_backward", mutates_args=())
def qkv_filter_backward(x: torch.Tensor, wpack: torch.Tensor, values: torch.Tensor,
                        logits: torch.Tensor, inits: torch.Tensor, logit_bias: torch.Tensor,
                        hq: torch.Tensor, hk: torch.Tensor, hv: torch.Tensor, gq: torch.Tensor,
                        gk: torch.Tensor, gv: torch.Tensor, NH: int, NKVH: int, Da: int,
                        r: int, P: int = UNBOUNDED_P, Q: int = 1,
                        K: int = 1) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                             torch.Tensor]:
    return _qkv_filter_backward_impl(x, wpack, values, logits, inits, logit_bias, hq, hk, hv,
                                     gq, gk, gv, NH, NKVH, Da, r, P, Q, K)


@qkv_filter_backward.register_fake
def _(x, wpack, values, logits, inits, logit_bias, hq, hk, hv, gq, gk, gv, NH, NKVH, Da, r,
      P=UNBOUNDED_P, Q=1, K=1):
    B, T, C = x.shape
    H = NH + 2 * NKVH
    D = Da * r
    return (x.new_empty((B, T, C), dtype=torch.bfloat16),
            x.new_empty((H * (D + Da), C), dtype=torch.float32),
            inits.new_empty(inits.shape), x.new_empty((H, Da), dtype=torch.float32))


def _filter_setup(ctx, inputs, output):
    x, weight, inits, logit_bias, *args = inputs  # NH, NKVH, Da, r, P, Q, K
    q, k, v, values, logits, wpack = output
    ctx.save_for_backward(x, wpack, values, logits, inits, logit_bias, q, k, v)
    ctx.args = tuple(args)
    ctx.weight_dtype = weight.dtype
    # values / logits / wpack are internal outputs: no zero gradients for them
    ctx.set_materialize_grads(False)


def _filter_grads(ctx, gq, gk, gv, backward_fn):
    """Input gradients from the saved tensors, through ``backward_fn`` (the
    library op or its implementation)."""
    x, wpack, values, logits, inits, logit_bias, q, k, v = ctx.saved_tensors
    # upstream grads keep their strides (typically the transposed (B, T, H, D)
    # views): the scan backward reads any layout, 16-byte vectors along D
    gq = torch.zeros_like(q) if gq is None else gq
    gk = torch.zeros_like(k) if gk is None else gk
    gv = torch.zeros_like(v) if gv is None else gv
    gx, gw, gi, gb = backward_fn(x, wpack, values, logits, inits, logit_bias, q, k, v, gq, gk, gv,
                                 *ctx.args)
    if ctx.weight_dtype != torch.float32:
        gw = gw.to(ctx.weight_dtype)
    return (gx, gw, gi, gb.view_as(logit_bias)) + (None,) * len(ctx.args)


def _filter_backward(ctx, gq, gk, gv, g_values, g_logits, g_wpack):
    return _filter_grads(ctx, gq, gk, gv, torch.ops.nanochat_amd.qkv_filter_backward)


qkv_filter.register_autograd(_filter_backward, setup_context=_filter_setup)


class _QkvFilterEager(torch.autograd.Function):
    """The op's forward and backward implementations under a plain autograd
    function: the same launches, without the library op's dispatch (default
    filling, the compiler guards, the registered-autograd wrapper), which took
    about as much host time per step as the launches themselves."""

    @staticmethod
    def forward(ctx, x, weight, inits, logit_bias, NH, NKVH, Da, r, P, Q, K):
        out = _qkv_filter_impl(x, weight, inits, logit_bias, NH, NKVH, Da, r, P, Q, K)
        _filter_setup(ctx, (x, weight, inits, logit_bias, NH, NKVH, Da, r, P, Q, K), out)
        ctx.mark_non_differentiable(*out[3:])
        return out

    @staticmethod
    def backward(ctx, gq, gk, gv, g_values, g_logits, g_wpack):
        return _filter_grads(ctx, gq, gk, gv, _qkv_filter_backward_impl)


def qkv_filter_call(x: torch.Tensor, weight: torch.Tensor, inits: torch.Tensor,
                    logit_bias: torch.Tensor, NH: int, NKVH: int, Da: int, r: int,
                    P: int = UNBOUNDED_P, Q: int = 1, K: int = 1):
    """``nanochat_amd::qkv_filter`` as the filter modules call it: the library
    op under ``torch.compile`` (its schema, fake impl and registered autograd),
    the same implementation through ``_QkvFilterEager`` in eager mode."""
    if torch.compiler.is_compiling():
        return torch.ops.nanochat_amd.qkv_filter(x, weight, inits, logit_bias, NH, NKVH, Da, r,
                                                 P, Q, K)
    return _QkvFilterEager.apply(x, weight, inits, logit_bias, NH, NKVH, Da, r, P, Q, K)
