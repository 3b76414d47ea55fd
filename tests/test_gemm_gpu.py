"""GPU parity of the projection.

* the reference-layout op ``fused_linear_transpose`` against torch.matmul in
  fp32 on the shapes of the reference's tests/test_fused_linear_transpose.py:32-86
  (fp32 tolerance 1e-4, bf16 5e-2 as there);
* the fast path ``nanochat_amd::qkv_project`` (bf16 MFMA) against a float64
  product of the same bf16-rounded operands, forward and backward, including the
  head-major split layout it writes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ltv_test_utils import assert_close, np_of

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ops():
    import nanochat_amd.ops  # noqa: F401
    return torch.ops


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("B,T,K,F", [(1, 16, 32, 128), (4, 128, 128, 256),
                                     (4, 1024, 1024, 3096), (2, 31, 63, 127)])
def test_fused_linear_transpose(dtype, B, T, K, F):
    ops = _ops()
    g = torch.Generator().manual_seed(B * T + K + F)
    x = (torch.randn(B, T, K, generator=g) / K ** 0.5).to(dtype).to(DEV).requires_grad_(True)
    w = (torch.randn(F, K, generator=g) / K ** 0.5).to(dtype).to(DEV).requires_grad_(True)
    xr = x.detach().float().requires_grad_(True)
    wr = w.detach().float().requires_grad_(True)
    ref = torch.matmul(wr, xr.transpose(-1, -2))  # plain torch fp32 reference
    go = torch.randn(ref.shape, generator=g).to(DEV)
    ref.backward(go)
    out = ops.nanochat_cuda.fused_linear_transpose_cuda_op(x, w)
    assert out.shape == (B, F, T) and out.is_contiguous() and out.dtype == dtype
    out.backward(go.to(dtype))
    tol = 5e-2 if dtype == torch.bfloat16 else 1e-4
    assert_close(np_of(out), np_of(ref), tol, "out")
    assert_close(np_of(x.grad), np_of(xr.grad), tol, "grad_x")
    assert_close(np_of(w.grad), np_of(wr.grad), tol, "grad_weight")


def test_fused_linear_transpose_accepts_btf_grad():
    ops = _ops()
    B, T, K, F = 2, 40, 24, 56
    x = torch.randn(B, T, K, device=DEV)
    w = torch.randn(F, K, device=DEV)
    go_btf = torch.randn(B, T, F, device=DEV)
    gx = torch.zeros_like(x)
    gw = torch.zeros_like(w)
    ops.nanochat_cuda.fused_linear_transpose_backward_kernel(x, w, go_btf.transpose(1, 2), gx, gw)
    go = go_btf.transpose(1, 2).double().cpu()
    assert_close(np_of(gx), (go.transpose(1, 2) @ w.double().cpu()).numpy(), 1e-4, "gx")
    assert_close(np_of(gw), torch.einsum("bft,btk->fk", go, x.double().cpu()).numpy(), 1e-4, "gw")


def _bf(t):
    return t.to(torch.bfloat16).double()


@pytest.mark.parametrize("B,T,C,NH,NKVH,D,Da", [
    (2, 256, 768, 6, 6, 128, 1),   # d12 widths
    (1, 100, 64, 1, 1, 16, 2),     # ragged M, small heads
    (3, 33, 128, 2, 1, 64, 64),    # per-channel gates (r = 1)
    (1, 300, 256, 3, 0, 12, 4),    # head width not a multiple of 8, no kv heads
])
def test_qkv_project_fast_path(B, T, C, NH, NKVH, D, Da):
    """bf16 MFMA projection: head-major values and row-major logits forward;
    grad_x and fp32 grad_weight (parameter row order) backward."""
    from nanochat_amd.ops import ltv_hm_fast as F_
    H = NH + 2 * NKVH
    F = H * (D + Da)
    Fp, Lp = F_.packed_width(H, D, Da), F_.logit_width(H, Da)
    g = torch.Generator().manual_seed(T + C)
    x = torch.randn(B, T, C, generator=g).to(torch.bfloat16)
    w = torch.randn(F, C, generator=g) / C ** 0.5  # fp32 master, cast to bf16 by the op
    values, logits, wpack = F_.project(x.to(DEV), w.to(DEV), H, D, Da)
    assert values.shape == (B, H, T, D) and logits.shape == (B, T, Lp)

    ref = (_bf(x) @ _bf(w).T).view(B, T, H, D + Da)  # interleaved order, float64
    assert_close(np_of(values), ref[..., :D].permute(0, 2, 1, 3).numpy(), 2e-2, "values")
    assert_close(np_of(logits)[..., : H * Da], ref[..., D:].reshape(B, T, H * Da).numpy(), 2e-2,
                 "logits")

    gc = torch.randn(B, T, Fp, generator=g).to(torch.bfloat16)
    gc[..., F:] = float("nan")  # padding columns must be ignored
    gx, gw = F_.project_backward(x.to(DEV), wpack, gc.to(DEV), H, D, Da)
    gc_i = torch.cat([gc[..., : H * D].view(B, T, H, D), gc[..., H * D: F].view(B, T, H, Da)],
                     dim=-1).reshape(B, T, F).double()
    want_gx = gc_i @ _bf(w)
    want_gw = torch.einsum("btf,btc->fc", gc_i, _bf(x))
    assert torch.isfinite(gx).all() and torch.isfinite(gw).all()
    assert gw.dtype == torch.float32
    assert_close(np_of(gx), want_gx.numpy(), 2e-2, "grad_x")
    assert_close(np_of(gw), want_gw.numpy(), 2e-2, "grad_weight")


@pytest.mark.parametrize("M", [1, 255, 257, 8192 + 64])
def test_projection_ragged_token_counts(M):
    """Token counts that leave partial 256-row tiles and partial dW splits."""
    from nanochat_amd.ops import ltv_hm_fast as F_
    H, D, Da, C = 3, 128, 1, 256
    F = H * (D + Da)
    Fp = F_.packed_width(H, D, Da)
    g = torch.Generator().manual_seed(M)
    x = torch.randn(1, M, C, generator=g).to(torch.bfloat16)
    w = torch.randn(F, C, generator=g) / C ** 0.5
    values, logits, wpack = F_.project(x.to(DEV), w.to(DEV), H, D, Da)
    ref = (_bf(x) @ _bf(w).T).view(1, M, H, D + Da)
    assert_close(np_of(values), ref[..., :D].permute(0, 2, 1, 3).numpy(), 2e-2, "values")
    gc = torch.randn(1, M, Fp, generator=g).to(torch.bfloat16)
    gx, gw = F_.project_backward(x.to(DEV), wpack, gc.to(DEV), H, D, Da)
    gc_i = torch.cat([gc[..., : H * D].view(1, M, H, D), gc[..., H * D: F].view(1, M, H, Da)],
                     dim=-1).reshape(1, M, F).double()
    assert_close(np_of(gx), (gc_i @ _bf(w)).numpy(), 2e-2, "grad_x")
    assert_close(np_of(gw), torch.einsum("btf,btc->fc", gc_i, _bf(x)).numpy(), 2e-2,
                 "grad_weight")


@pytest.mark.parametrize("B,T,K,F", [
    (32, 1024, 768, 2322),   # d12: the reference filter's projection at configs[2]
    (2, 256, 64, 100),       # one token tile per batch, F not a multiple of 8
    (3, 512, 136, 700),      # K a multiple of 8 but not of 64
])
def test_fused_linear_transpose_bf16_mfma(B, T, K, F):
    """bf16 reference-layout projection on the MFMA kernels (T a multiple of
    256, K of 8): out (B, F, T), grad_x and grad_weight against an fp32 torch
    product of the same bf16 operands, and against the fp32-MFMA kernel
    (ltv_linear_transpose_backward) -- both fp32-accumulated, so within
    accumulation-order rounding; the weight gradient twice bitwise equal
    (fixed-order split sum)."""
    from nanochat_amd import _native as N
    ops = _ops()
    lib = N.lib()
    assert lib.ltv_linear_transpose_backward_workspace_size(N.DTYPE_BF16, B, T, K, F, 0) > 0
    g = torch.Generator().manual_seed(B + T + K + F)
    x = (torch.randn(B, T, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(DEV)
    w = (torch.randn(F, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(DEV)
    go = torch.randn(B, F, T, generator=g).to(torch.bfloat16).to(DEV)
    xf, wf, gof = x.float(), w.float(), go.float()
    out = ops.nanochat_cuda.fused_linear_transpose_cuda_op(x, w)
    ref = torch.matmul(wf, xf.transpose(1, 2))
    assert_close(np_of(out), np_of(ref), 2e-2, "out")
    grads = []
    for _ in range(2):
        gx = torch.empty_like(x)
        gw = torch.empty_like(w)
        ops.nanochat_cuda.fused_linear_transpose_backward_kernel(x, w, go, gx, gw)
        grads.append((gx, gw))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    gx, gw = grads[0]
    want_gx = torch.matmul(gof.transpose(1, 2), wf)                        # (B, T, K)
    want_gw = torch.matmul(gof.reshape(B, F, T).permute(1, 0, 2).reshape(F, B * T),
                           xf.reshape(B * T, K))                          # (F, K)
    assert_close(np_of(gx), np_of(want_gx), 2e-2, "grad_x")
    assert_close(np_of(gw), np_of(want_gw), 2e-2, "grad_weight")
    # the fp32-MFMA kernel on the same operands
    sx, sw = torch.empty_like(x), torch.empty_like(w)
    N.check(lib.ltv_linear_transpose_backward(N.DTYPE_BF16, x.data_ptr(), w.data_ptr(),
                                              go.data_ptr(), 0, sx.data_ptr(), sw.data_ptr(),
                                              B, T, K, F, N.stream_of(x)), "fp32-MFMA backward")
    torch.cuda.synchronize()
    assert_close(np_of(gx), np_of(sx), 2e-2, "grad_x vs fp32-MFMA")
    assert_close(np_of(gw), np_of(sw), 2e-2, "grad_weight vs fp32-MFMA")
