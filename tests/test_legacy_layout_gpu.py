"""GPU parity of the legacy-layout scan op and filter
(``combined = [q values | k values | v values | gate logits]``, bias pre-added).

Mirrors the reference's tests/test_ltv_cuda_fused_concat_register_cast_blelloch_scan.py:
its integer generator (values ``(11b + 7t + 5h + d) % 7 - 3``, logits
``(b + t + h + j) % 2``, ``:95-128``) over every stride layout of ``combined`` and
T in {1, 2, 3, 31, 32, 33, 63, 64, 65, 127, 128, 129} without the sigmoid must
match exactly, forward and backward.  The expected values come from the CPU
oracle after a pure index permutation of the layout into the head-interleaved
one (``O.scan_forward`` / ``O.scan_backward`` with a zero bias: the bias is
already in the logits).  Sigmoid cases and the filter module are checked
within the stated tolerances.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import TOL, assert_close, io_name, np_of, strided_copy, stride_layouts, to_torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _perm(H, D, Da):
    """legacy column index of each head-interleaved column"""
    idx = []
    for h in range(H):
        idx += [h * D + d for d in range(D)]
        idx += [H * D + h * Da + j for j in range(Da)]
    return np.array(idx)


def to_interleaved(c, H, D, Da):
    return np.ascontiguousarray(c[..., _perm(H, D, Da)])


def to_legacy(c, H, D, Da):
    out = np.empty_like(c)
    out[..., _perm(H, D, Da)] = c
    return out


def legacy_int_combined(B, T, NH, NKVH, Da, r):
    H, D = NH + 2 * NKVH, Da * r
    b, t, h, d = np.meshgrid(np.arange(B), np.arange(T), np.arange(H), np.arange(D), indexing="ij")
    vals = ((11 * b + 7 * t + 5 * h + d) % 7 - 3).reshape(B, T, H * D)
    b, t, h, j = np.meshgrid(np.arange(B), np.arange(T), np.arange(H), np.arange(Da), indexing="ij")
    lg = ((b + t + h + j) % 2).reshape(B, T, H * Da)
    return np.concatenate([vals, lg], axis=-1).astype(np.float32)


def int_inits(B, H, D):
    b, h, d = np.meshgrid(np.arange(B), np.arange(H), np.arange(D), indexing="ij")
    return ((13 * b + 3 * h + d) % 7 - 3).astype(np.float32)


def _expected(c, ini, NH, NKVH, Da, r, sig, io, gy):
    H, D = NH + 2 * NKVH, Da * r
    ci = to_interleaved(c, H, D, Da)
    zb = np.zeros((H, Da), np.float32)
    outs = O.scan_forward(ci, ini, zb, NH, NKVH, Da, r, sig, io)
    gc, gi, _ = O.scan_backward(ci, ini, zb, *outs, gy[:, :NH], gy[:, NH:NH + NKVH],
                                gy[:, NH + NKVH:], NH, NKVH, Da, r, sig, io)
    return outs, to_legacy(gc, H, D, Da), gi


def _run(comb, ini, NH, NKVH, Da, r, sig, grads):
    import nanochat_amd.ops  # noqa: F401
    op = torch.ops.nanochat_cuda.ltv_fused_concat_register_cast_blelloch_scan_cuda_op
    comb = comb.detach().requires_grad_(True)
    ini = ini.detach().requires_grad_(True)
    outs = op(comb, ini, NH, NKVH, Da, r, 32, 1, sig)
    torch.autograd.backward(outs, grads)
    return outs, comb.grad, ini.grad


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=io_name)
@pytest.mark.parametrize("T", [1, 2, 3, 31, 32, 33, 63, 64, 65, 127, 128, 129])
def test_legacy_exact_all_strides(dtype, T):
    B, NH, NKVH, Da, r = 4, 8, 8, 1, 1  # the reference's settings (total_d = 1)
    H, D = NH + 2 * NKVH, Da * r
    c = legacy_int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, H, D)
    rng = np.random.default_rng(T)
    gy = rng.integers(-2, 3, size=(B, H, T, D)).astype(np.float32)
    (eq, ek, ev), egc, egi = _expected(c, ini, NH, NKVH, Da, r, False, io_name(dtype), gy)
    grads = [to_torch(gy[:, :NH], dtype, DEV), to_torch(gy[:, NH:NH + NKVH], dtype, DEV),
             to_torch(gy[:, NH + NKVH:], dtype, DEV)]
    for stride in stride_layouts(c.shape):
        (q, k, v), gc, gi = _run(strided_copy(c, stride, dtype, DEV), to_torch(ini, dtype, DEV),
                                 NH, NKVH, Da, r, False, grads)
        case = f"T={T} stride={stride}"
        assert_close(np_of(q), eq, 0, "q " + case)
        assert_close(np_of(k), ek, 0, "k " + case)
        assert_close(np_of(v), ev, 0, "v " + case)
        assert_close(np_of(gc), egc, 0, "grad_combined " + case)
        assert_close(np_of(gi), egi, 0, "grad_inits " + case)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=io_name)
@pytest.mark.parametrize("D,r", [(128, 128), (128, 16), (128, 2), (128, 1), (12, 3)])
@pytest.mark.parametrize("sig", [False, True])
def test_legacy_wide_heads(dtype, D, r, sig):
    B, NH, NKVH, T = 2, 2, 1, 97
    Da, H = D // r, NH + 2 * NKVH
    io = io_name(dtype)
    rng = np.random.default_rng(D + r + sig)
    if sig:
        c = O.round_io(rng.standard_normal((B, T, H * (D + Da))).astype(np.float32), io)
        ini = O.round_io(rng.standard_normal((B, H, D)).astype(np.float32), io)
        gy = O.round_io(rng.standard_normal((B, H, T, D)).astype(np.float32), io)
        tol = TOL[dtype]
    else:
        c = legacy_int_combined(B, T, NH, NKVH, Da, r)
        ini = int_inits(B, H, D)
        gy = rng.integers(-2, 3, size=(B, H, T, D)).astype(np.float32)
        tol = 0
    (eq, ek, ev), egc, egi = _expected(c, ini, NH, NKVH, Da, r, sig, io, gy)
    grads = [to_torch(gy[:, :NH], dtype, DEV), to_torch(gy[:, NH:NH + NKVH], dtype, DEV),
             to_torch(gy[:, NH + NKVH:], dtype, DEV)]
    (q, k, v), gc, gi = _run(to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV), NH, NKVH, Da, r,
                             sig, grads)
    case = f"D={D} r={r} sig={sig}"
    assert_close(np_of(q), eq, tol, "q " + case)
    assert_close(np_of(k), ek, tol, "k " + case)
    assert_close(np_of(v), ev, tol, "v " + case)
    assert_close(np_of(gc), egc, tol, "grad_combined " + case)
    assert_close(np_of(gi), egi, tol, "grad_inits " + case)


def test_legacy_backward_kernel_fills_grad_logits():
    """The mutating backward kernel also leaves the fp32 logit gradients in
    grad_logits for r > 1, as the reference's kernel does."""
    import nanochat_amd.ops  # noqa: F401
    B, T, NH, NKVH, D, r = 2, 40, 2, 1, 64, 16
    Da, H = D // r, NH + 2 * NKVH
    rng = np.random.default_rng(0)
    c = rng.standard_normal((B, T, H * (D + Da))).astype(np.float32)
    ini = rng.standard_normal((B, H, D)).astype(np.float32)
    cd, ind = to_torch(c, torch.float32, DEV), to_torch(ini, torch.float32, DEV)
    ops = torch.ops.nanochat_cuda
    hq, hk, hv = ops.ltv_fused_concat_register_cast_blelloch_scan_cuda_op(cd, ind, NH, NKVH, Da, r,
                                                                          32, 1, True)
    gys = [torch.randn_like(t) for t in (hq, hk, hv)]
    gc = torch.empty_like(cd)
    gi = torch.empty_like(ind)
    gl = torch.zeros(B, T, H, Da, device=DEV)
    ops.ltv_fused_concat_register_cast_blelloch_scan_cuda_backward_kernel(
        cd, ind, hq, hk, hv, *gys, gc, gi, gl, NH, NKVH, Da, r, 32, 1, True)
    torch.testing.assert_close(gl.view(B, T, H * Da), gc[:, :, H * D:])
    assert float(gl.abs().max()) > 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=io_name)
def test_legacy_filter_module(dtype):
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    from nanochat_amd.ltv_cuda_fused_concat_register_cast_blelloch_scan_qkv_filter import (
        LtvCudaFusedConcatRegisterCastBlellochScanQkvFilter as Filter,
    )
    NH, NKVH, D, r = 2, 1, 128, 32
    Da, H = D // r, NH + 2 * NKVH
    torch.manual_seed(0)
    f = Filter(NH, NKVH, D, r)
    f.init_weights(alpha_mlp_bias_init=0.0, weight_s=(3.0 / (NH * D)) ** 0.5, bias_s=0.5,
                   init_s=0.5)
    f = f.to(DEV)
    B, T, C = 2, 150, NH * D
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, C, generator=g)
    gq = torch.randn(B, T, NH, D, generator=g)
    gk = torch.randn(B, T, NKVH, D, generator=g)
    gv = torch.randn(B, T, NKVH, D, generator=g)
    xd = x.to(DEV).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=dtype == torch.bfloat16):
        q, k, v = f(xd, LtvInitValues())
    assert q.shape == (B, T, NH, D) and q.dtype == dtype
    torch.autograd.backward([q, k, v], [t.to(DEV).to(dtype) for t in (gq, gk, gv)])

    # oracle: the same projection rows permuted to the head-interleaved order,
    # the bias as the scan's logit bias; fp64 for the fp32 run
    io = "f64" if dtype == torch.float32 else "bf16"
    perm = _perm(H, D, Da)
    w = f.c.weight.detach().double().cpu().numpy()[perm]
    bias = f.logit_bias.detach().double().cpu().numpy().reshape(H, Da)
    ini = np.broadcast_to(f.init_param.detach().double().cpu().numpy(), (B, H, D))
    if dtype == torch.bfloat16:  # autocast: bf16 operands, bf16 combined (+ bias rounded in)
        w, x_np, ini = O.bf16_round(w.astype(np.float32)), O.bf16_round(x.numpy()), O.bf16_round(
            np.ascontiguousarray(ini, np.float32))
        comb = O.bf16_round(O.linear_transpose_forward(x_np, w, "bf16").transpose(0, 2, 1))
        comb4 = comb.reshape(B, T, H, D + Da)
        comb4[..., D:] = O.bf16_round(comb4[..., D:] + bias.astype(np.float32))
        eq, ek, ev = O.scan_forward(comb, ini, np.zeros((H, Da), np.float32), NH, NKVH, Da, r,
                                    True, "bf16")
        tol = TOL[dtype]
    else:
        comb = O.linear_transpose_forward(x.double().numpy(), w, "f64").transpose(0, 2, 1)
        eq, ek, ev = O.scan_forward(np.ascontiguousarray(comb), ini, bias, NH, NKVH, Da, r, True,
                                    "f64")
        gys = [np.ascontiguousarray(t.double().numpy().transpose(0, 2, 1, 3)) for t in (gq, gk, gv)]
        gc, gi, gb = O.scan_backward(np.ascontiguousarray(comb), ini, bias, eq, ek, ev, *gys, NH,
                                     NKVH, Da, r, True, "f64")
        gx, gw = O.linear_transpose_backward(x.double().numpy(), w, gc.transpose(0, 2, 1), "f64")
        tol = TOL[dtype]
        assert_close(np_of(xd.grad), gx, tol, "grad_x")
        egw = np.empty_like(gw)
        egw[perm] = gw
        assert_close(np_of(f.c.weight.grad), egw, tol, "grad_weight")
        assert_close(np_of(f.logit_bias.grad), gb.reshape(-1), tol, "grad_logit_bias")
        assert_close(np_of(f.init_param.grad), gi.sum(axis=0), tol, "grad_init_param")
    t = lambda a: np.asarray(a).transpose(0, 2, 1, 3)  # noqa: E731
    assert_close(np_of(q), t(eq), tol, "q")
    assert_close(np_of(k), t(ek), tol, "k")
    assert_close(np_of(v), t(ev), tol, "v")
