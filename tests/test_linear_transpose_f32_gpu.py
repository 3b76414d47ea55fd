"""GPU parity of the strided fp32-MFMA GEMM behind the reference-layout op
``fused_linear_transpose`` (reference ``nanochat/ops/fused_linear_transpose.py``
and ``cpp_ewma/src/fused_linear_transpose_{forward,backward}.cu``, which run
fp32 through strided-batched library GEMMs).

Every result is checked against a float64 product of the same operands under
the worst-case bound of an fp32 sum of n products,
|got - want| <= (n + 4) 2^-24 (|A| |B|)  (+ 2^-8 |want| for bf16 outputs),
with n the reduction length (plus the split count for split partials): an
operand layout, stage form or index mistake breaks it by orders of magnitude.
The cases reach each staging form of both operands (k-contiguous quads,
row-contiguous quads, single elements for misaligned or odd strides), ragged
tiles in every dimension, split and unsplit weight gradients, both grad_out
layouts, and empty reductions.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
U32 = 2.0 ** -24


def _ops():
    import nanochat_amd.ops  # noqa: F401
    return torch.ops


def _lib():
    from nanochat_amd import _native as N
    return N, N.lib()


def _check(got, a, b, n, label, bf16_out=False):
    """got ~ a @ b (float64 on the GPU) within the fp32 summation bound."""
    a, b = a.double().contiguous(), b.double().contiguous()
    want = torch.matmul(a, b)
    bound = (n + 4) * U32 * torch.matmul(a.abs(), b.abs())
    if bf16_out:
        bound = bound + 2.0 ** -8 * want.abs()
    err = (got.double() - want).abs()
    bad = err > bound + 1e-30
    assert not bool(bad.any()), (
        f"{label}: {int(bad.sum())}/{bad.numel()} outside the bound; "
        f"max err {float(err.max()):.3e}, max bound {float(bound.max()):.3e}")
    rel = float(err.norm() / max(float(want.norm()), 1e-30))
    assert rel < (3e-3 if bf16_out else 1e-5), (label, rel)


def _operands(B, T, K, F, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, T, K, generator=g) / max(K, 1) ** 0.5).to(dtype).to(DEV)
    w = (torch.randn(F, K, generator=g) / max(K, 1) ** 0.5).to(dtype).to(DEV)
    go = torch.randn(B, F, T, generator=g).to(dtype).to(DEV)
    return x, w, go


SHAPES = [
    (1, 1, 1, 1),          # one element everywhere
    (2, 37, 50, 29),       # ragged T, K % 4 = 2 (single-element staging), F < one tile
    (3, 130, 96, 257),     # one row past a tile in T and F, quads everywhere
    (1, 300, 33, 131),     # odd K: quads of x and W straddle rows
    (4, 1024, 768, 2322),  # d12: the reference filter's projection at configs[2], B = 4
]


@pytest.mark.parametrize("B,T,K,F", SHAPES)
def test_f32_forward(B, T, K, F):
    ops = _ops()
    x, w, _ = _operands(B, T, K, F, torch.float32, B * 1000 + T + K + F)
    out = ops.nanochat_cuda.fused_linear_transpose_cuda_op(x, w)
    assert out.shape == (B, F, T) and out.dtype == torch.float32
    _check(out, w.unsqueeze(0).expand(B, F, K), x.transpose(1, 2), K, "out")


@pytest.mark.parametrize("btf", [False, True], ids=["bft", "btf"])
@pytest.mark.parametrize("B,T,K,F", SHAPES)
def test_f32_backward(B, T, K, F, btf):
    """Through the op (workspace-sized split of the weight gradient) and the
    entry without a workspace (one pass per tile): both within the bound, the
    op's result twice bitwise equal."""
    N, lib = _lib()
    ops = _ops()
    x, w, go = _operands(B, T, K, F, torch.float32, B * 7 + T * 3 + K + F)
    if btf:
        go = go.transpose(1, 2).contiguous().transpose(1, 2)  # (B, T, F) storage
    runs = []
    for _ in range(2):
        gx, gw = torch.empty_like(x), torch.empty_like(w)
        ops.nanochat_cuda.fused_linear_transpose_backward_kernel(x, w, go, gx, gw)
        runs.append((gx, gw))
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1])
    nx, nw = torch.empty_like(x), torch.empty_like(w)
    N.check(lib.ltv_linear_transpose_backward(
        N.DTYPE_F32, x.data_ptr(), w.data_ptr(), go.data_ptr(), int(btf), nx.data_ptr(),
        nw.data_ptr(), B, T, K, F, N.stream_of(x)), "ltv_linear_transpose_backward")
    torch.cuda.synchronize()
    ws = lib.ltv_linear_transpose_backward_workspace_size(N.DTYPE_F32, B, T, K, F, int(btf))
    splits = ws // (F * K * 4) if ws else 1
    gx, gw = runs[0]
    go_tf = go.transpose(1, 2)                     # (B, T, F) view
    go_f_bt = go.permute(1, 0, 2).reshape(F, B * T)
    x_bt_k = x.reshape(B * T, K)
    _check(gx, go_tf, w.unsqueeze(0).expand(B, F, K), F, "grad_x")
    _check(nx, go_tf, w.unsqueeze(0).expand(B, F, K), F, "grad_x (no workspace)")
    _check(gw, go_f_bt, x_bt_k, B * T + splits, f"grad_weight ({splits} splits)")
    _check(nw, go_f_bt, x_bt_k, B * T, "grad_weight (no workspace)")


def test_f32_weight_gradient_splits_at_d12():
    """The d12 shape's weight gradient is split (the op's workspace is sized
    for it): several partials, each in a fixed-order sum."""
    N, lib = _lib()
    ws = lib.ltv_linear_transpose_backward_workspace_size(N.DTYPE_F32, 32, 1024, 768, 2322, 0)
    assert ws > 0 and ws % (2322 * 768 * 4) == 0 and ws // (2322 * 768 * 4) >= 2


@pytest.mark.parametrize("B,T,K,F", [(2, 40, 24, 56), (2, 256, 64, 100), (3, 33, 17, 9)])
def test_bf16_btf_backward(B, T, K, F):
    """bf16 with a (B, T, F) grad_out, which the direct-to-LDS bf16 kernels do
    not take: the fp32-MFMA kernel, products exact, sums fp32, outputs rounded."""
    ops = _ops()
    x, w, go = _operands(B, T, K, F, torch.bfloat16, B + T + K + F)
    go = go.transpose(1, 2).contiguous().transpose(1, 2)
    gx, gw = torch.empty_like(x), torch.empty_like(w)
    ops.nanochat_cuda.fused_linear_transpose_backward_kernel(x, w, go, gx, gw)
    torch.cuda.synchronize()
    _check(gx, go.transpose(1, 2), w.unsqueeze(0).expand(B, F, K), F, "grad_x", bf16_out=True)
    _check(gw, go.permute(1, 0, 2).reshape(F, B * T), x.reshape(B * T, K), B * T + 8,
           "grad_weight", bf16_out=True)


def test_f32_misaligned_operands_use_single_element_staging():
    """Operands one element past a 16-byte boundary cannot be staged in quads:
    the forward and both gradients still match."""
    N, lib = _lib()
    B, T, K, F = 2, 96, 64, 72
    x0, w0, go0 = _operands(B, T, K, F, torch.float32, 11)
    xb = torch.empty(B * T * K + 1, device=DEV)
    wb = torch.empty(F * K + 1, device=DEV)
    gb = torch.empty(B * F * T + 1, device=DEV)
    x = xb[1:].view(B, T, K)
    w = wb[1:].view(F, K)
    go = gb[1:].view(B, F, T)
    x.copy_(x0)
    w.copy_(w0)
    go.copy_(go0)
    assert x.data_ptr() % 16 and w.data_ptr() % 16 and go.data_ptr() % 16
    out = torch.empty(B, F, T, device=DEV)
    gx, gw = torch.empty_like(x0), torch.empty_like(w0)
    st = N.stream_of(x)
    N.check(lib.ltv_linear_transpose_forward(N.DTYPE_F32, x.data_ptr(), w.data_ptr(),
                                             out.data_ptr(), B, T, K, F, st), "forward")
    N.check(lib.ltv_linear_transpose_backward(N.DTYPE_F32, x.data_ptr(), w.data_ptr(),
                                              go.data_ptr(), 0, gx.data_ptr(), gw.data_ptr(),
                                              B, T, K, F, st), "backward")
    torch.cuda.synchronize()
    _check(out, w.unsqueeze(0).expand(B, F, K), x.transpose(1, 2), K, "out")
    _check(gx, go.transpose(1, 2), w.unsqueeze(0).expand(B, F, K), F, "grad_x")
    _check(gw, go.permute(1, 0, 2).reshape(F, B * T), x.reshape(B * T, K), B * T, "grad_weight")


def test_f32_empty_reductions_give_zeros():
    """K = 0: the output is zeros; F = 0 reduction for grad_x and B T = 0 for
    grad_weight are covered by the op's zero-filled allocations and the
    kernel's empty k-loop storing zeros."""
    N, lib = _lib()
    ops = _ops()
    x = torch.empty(2, 5, 0, device=DEV)
    w = torch.empty(7, 0, device=DEV)
    out = ops.nanochat_cuda.fused_linear_transpose_cuda_op(x, w)
    assert out.shape == (2, 7, 5) and not bool(out.abs().sum())
    # grad_weight over an empty batch: the kernel stores zeros over garbage
    B, T, K, F = 0, 4, 8, 12
    xs = torch.empty(1, T, K, device=DEV)
    ws_ = torch.randn(F, K, device=DEV)
    go = torch.empty(1, F, T, device=DEV)
    gx = torch.empty(1, T, K, device=DEV)
    gw = torch.full((F, K), float("nan"), device=DEV)
    N.check(lib.ltv_linear_transpose_backward(N.DTYPE_F32, xs.data_ptr(), ws_.data_ptr(),
                                              go.data_ptr(), 0, gx.data_ptr(), gw.data_ptr(),
                                              B, T, K, F, N.stream_of(xs)), "backward")
    torch.cuda.synchronize()
    assert np.array_equal(gw.cpu().numpy(), np.zeros((F, K), np.float32))


def test_random_shapes_layouts_and_offsets():
    """24 seeded random cases: B, T, K, F from 1 to a few hundred, fp32 and
    bf16, grad_out (B, F, T) or (B, T, F), tensors 0-3 elements past a
    16-byte boundary (every staging form, tails in every dimension), through
    the forward and both backward entry points (workspace split and none)."""
    N, lib = _lib()
    rng = np.random.default_rng(2024)
    for case in range(24):
        B = int(rng.integers(1, 5))
        T, K, F = (int(v) for v in rng.integers(1, 300, size=3))
        dtype = torch.float32 if case % 3 else torch.bfloat16
        btf = bool(case % 2)
        off = int(rng.integers(0, 4))
        es = 4 if dtype == torch.float32 else 2
        g = torch.Generator().manual_seed(case)

        def place(shape, scale):
            n = int(np.prod(shape))
            buf = torch.empty(n + off, dtype=dtype, device=DEV)
            t = buf[off:].view(*shape)
            t.copy_((torch.randn(*shape, generator=g) * scale).to(dtype))
            return t

        x = place((B, T, K), K ** -0.5)
        w = place((F, K), K ** -0.5)
        go_store = place((B, T, F) if btf else (B, F, T), 1.0)
        go = go_store.transpose(1, 2) if btf else go_store
        out = torch.empty(B, F, T, dtype=dtype, device=DEV)
        gx, gw = torch.empty(B, T, K, dtype=dtype, device=DEV), torch.empty(F, K, dtype=dtype, device=DEV)
        hx, hw = torch.empty_like(gx), torch.empty_like(gw)
        st = N.stream_of(x)
        code = N.dtype_code(dtype)
        label = f"case {case}: B={B} T={T} K={K} F={F} {dtype} btf={btf} off={off * es}B"
        N.check(lib.ltv_linear_transpose_forward(code, x.data_ptr(), w.data_ptr(), out.data_ptr(),
                                                 B, T, K, F, st), label)
        ws_bytes = lib.ltv_linear_transpose_backward_workspace_size(code, B, T, K, F, int(btf))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        N.check(lib.ltv_linear_transpose_backward_ws(
            code, x.data_ptr(), w.data_ptr(), go_store.data_ptr(), int(btf), gx.data_ptr(),
            gw.data_ptr(), ws.data_ptr(), ws_bytes, B, T, K, F, st), label)
        N.check(lib.ltv_linear_transpose_backward(
            code, x.data_ptr(), w.data_ptr(), go_store.data_ptr(), int(btf), hx.data_ptr(),
            hw.data_ptr(), B, T, K, F, st), label)
        torch.cuda.synchronize()
        bf = dtype == torch.bfloat16
        splits = ws_bytes // (F * K * 4) if ws_bytes else 1
        _check(out, w.unsqueeze(0).expand(B, F, K), x.transpose(1, 2), K, f"out, {label}", bf)
        _check(gx, go.transpose(1, 2), w.unsqueeze(0).expand(B, F, K), F, f"grad_x, {label}", bf)
        _check(hx, go.transpose(1, 2), w.unsqueeze(0).expand(B, F, K), F, f"grad_x nows, {label}", bf)
        gof = go.permute(1, 0, 2).reshape(F, B * T)
        _check(gw, gof, x.reshape(B * T, K), B * T + splits, f"grad_weight, {label}", bf)
        _check(hw, gof, x.reshape(B * T, K), B * T, f"grad_weight nows, {label}", bf)
