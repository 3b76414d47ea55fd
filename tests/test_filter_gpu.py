"""GPU parity of the drop-in filter module against the oracle.

one attention layer's LTV QKV filter, B=2, T=256,
C=768 (6 q heads + 6 kv heads of 128, r=128), seed 0, forward and backward.
* fp32 input -> the reference dataflow (fused_linear_transpose into (B, F, T),
  scan through the transposed view), tolerance 1e-4;
* bf16 input -> the MFMA fast path, tolerance 2e-2;
* continuing from cached last rows reproduces the full sequence.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import TOL, assert_close, assert_norm_rel, io_name, np_of

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _make_filter(NH=6, NKVH=6, D=128, r=128, seed=0):
    from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
        LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter,
    )
    torch.manual_seed(seed)
    f = Filter(NH, NKVH, D, r)
    C = NH * D
    # W ~ N(0, 1/C) for value and gate rows; small bias; init ~ U(-0.5, 0.5)
    with torch.no_grad():
        f.c.weight.normal_(0.0, C ** -0.5)
        f.logit_bias.uniform_(-0.5, 0.5)
        f.init_param.uniform_(-0.5, 0.5)
    return f.to(DEV)


def _oracle(f, x_np, dq, dk, dv, io):
    NH, NKVH, Da, r = f.n_head, f.n_kv_head, f.num_alpha_groups, f.r
    B = x_np.shape[0]
    w = f.c.weight.detach().float().cpu().numpy()
    if io == "bf16":
        w = O.bf16_round(w)  # the fast path multiplies with a bf16 copy of the master weight
    ini = np.broadcast_to(f.init_param.detach().float().cpu().numpy(), (B,) + tuple(f.init_param.shape))
    ini = O.round_io(np.ascontiguousarray(ini), io)
    bias = f.logit_bias.detach().float().cpu().numpy()
    q, k, v, comb, saved = O.filter_forward(x_np, w, ini, bias, NH, NKVH, Da, r, io)
    gx, gw, gi, gb = O.filter_backward(x_np, w, ini, bias, comb, saved, dq, dk, dv, NH, NKVH, Da,
                                       r, io)
    return (q, k, v), gx, gw, gi.sum(axis=0), gb


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_filter_config1(dtype):
    io = "bf16" if dtype == torch.bfloat16 else "f32"
    f = _make_filter()
    B, T, C = 2, 256, 768
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, T, C, generator=g).to(dtype)
    H = f.total_active_heads
    dq = torch.randn(B, T, f.n_head, 128, generator=g).to(dtype)
    dk = torch.randn(B, T, f.n_kv_head, 128, generator=g).to(dtype)
    dv = torch.randn(B, T, f.n_kv_head, 128, generator=g).to(dtype)

    xd = x.to(DEV).requires_grad_(True)
    q, k, v = f(xd, __import__("nanochat_amd.ltv.ltv_filter", fromlist=["x"]).LtvInitValues())
    assert q.shape == (B, T, f.n_head, 128) and q.dtype == dtype
    torch.autograd.backward([q, k, v], [dq.to(DEV), dk.to(DEV), dv.to(DEV)])

    (eq, ek, ev), egx, egw, egi, egb = _oracle(
        f, x.float().numpy(), dq.float().numpy(), dk.float().numpy(), dv.float().numpy(), io)
    tol = TOL[dtype]
    assert_close(np_of(q), eq, tol, "q")
    assert_close(np_of(k), ek, tol, "k")
    assert_close(np_of(v), ev, tol, "v")
    assert_close(np_of(xd.grad), egx, tol, "grad_x")
    assert_close(np_of(f.c.weight.grad), egw, tol, "grad_weight")
    assert_close(np_of(f.init_param.grad), egi, tol, "grad_init_param")
    assert_close(np_of(f.logit_bias.grad), egb, tol, "grad_logit_bias")
    assert H == 18


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_filter_state_continuity(dtype):
    """Running T tokens at once equals running them in two calls where the second
    starts from the first call's last q/k/v rows (what the KV cache feeds back)."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    f = _make_filter(NH=2, NKVH=1, D=128, r=128, seed=1)
    B, T, C = 2, 200, 256
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, C, generator=g).to(dtype).to(DEV)
    with torch.no_grad():
        full = f(x, LtvInitValues())
        a = f(x[:, :77], LtvInitValues())
        prev = LtvInitValues(q=a[0][:, -1], k=a[1][:, -1], v=a[2][:, -1])
        b = f(x[:, 77:], prev)
    tol = TOL[dtype]
    for i in range(3):
        got = torch.cat([a[i], b[i]], dim=1)
        assert_close(np_of(got), np_of(full[i]), tol, f"output {i}")


def _random_cases(n=16, seed=7):
    """Seeded filter shapes: heads, head widths (12 to 128: C off the fused
    path's multiple of 8 included), any gate group size r | D (one gate per
    head to one per channel; groups of a non-power-of-two number of lanes
    included), batch and sequence lengths off the kernels' tile sizes (T = 1
    included), both I/O dtypes."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        NH = int(rng.integers(1, 5))
        NKVH = int(rng.integers(1, NH + 1))
        D = int(rng.choice([12, 24, 32, 48, 64, 96, 128]))
        r = int(rng.choice([d for d in range(1, D + 1) if D % d == 0]))
        B = int(rng.integers(1, 4))
        T = 1 if i == 0 else int(rng.integers(2, 301))
        dtype = torch.bfloat16 if i % 2 else torch.float32
        cases.append(pytest.param(NH, NKVH, D, r, B, T, dtype,
                                  id=f"{i}-{io_name(dtype)}-h{NH}.{NKVH}-D{D}-r{r}-B{B}-T{T}"))
    return cases


@pytest.mark.parametrize("NH, NKVH, D, r, B, T, dtype", _random_cases())
def test_filter_random_shapes(NH, NKVH, D, r, B, T, dtype):
    """Forward and every gradient of the module at seeded random shapes against
    the oracle (fp32: the reference dataflow; bf16: the MFMA fast path)."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    io = io_name(dtype)
    f = _make_filter(NH=NH, NKVH=NKVH, D=D, r=r, seed=T)
    C = NH * D
    g = torch.Generator().manual_seed(B * 1000 + T)
    x = torch.randn(B, T, C, generator=g).to(dtype)
    dq = torch.randn(B, T, NH, D, generator=g).to(dtype)
    dk = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    dv = torch.randn(B, T, NKVH, D, generator=g).to(dtype)

    xd = x.to(DEV).requires_grad_(True)
    q, k, v = f(xd, LtvInitValues())
    torch.autograd.backward([q, k, v], [dq.to(DEV), dk.to(DEV), dv.to(DEV)])

    (eq, ek, ev), egx, egw, egi, egb = _oracle(
        f, x.float().numpy(), dq.float().numpy(), dk.float().numpy(), dv.float().numpy(), io)
    tol = TOL[dtype]
    for name, got, want in (("q", q, eq), ("k", k, ek), ("v", v, ev), ("grad_x", xd.grad, egx),
                            ("grad_weight", f.c.weight.grad, egw),
                            ("grad_init_param", f.init_param.grad, egi),
                            ("grad_logit_bias", f.logit_bias.grad, egb)):
        assert_close(np_of(got), want, tol, name)
        assert_norm_rel(np_of(got), want, tol, name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("NH,NKVH,D,r", [(1, 1, 12, 12), (3, 2, 4, 4), (3, 1, 12, 3), (2, 1, 6, 2)])
def test_filter_shapes_outside_the_fused_path(dtype, NH, NKVH, D, r):
    """C not a multiple of 8 or D not of 4: bf16 runs the reference dataflow
    (the projection into (B, F, T) with the weight rounded to bf16, then the
    scan op) instead of the fused path; forward and every gradient against the
    oracle."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    io = io_name(dtype)
    f = _make_filter(NH=NH, NKVH=NKVH, D=D, r=r, seed=D + r)
    B, T, C = 2, 75, NH * D
    g = torch.Generator().manual_seed(C)
    x = torch.randn(B, T, C, generator=g).to(dtype)
    dq = torch.randn(B, T, NH, D, generator=g).to(dtype)
    dk = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    dv = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    xd = x.to(DEV).requires_grad_(True)
    q, k, v = f(xd, LtvInitValues())
    assert q.dtype == dtype
    torch.autograd.backward([q, k, v], [dq.to(DEV), dk.to(DEV), dv.to(DEV)])
    (eq, ek, ev), egx, egw, egi, egb = _oracle(
        f, x.float().numpy(), dq.float().numpy(), dk.float().numpy(), dv.float().numpy(), io)
    tol = TOL[dtype]
    for name, got, want in (("q", q, eq), ("k", k, ek), ("v", v, ev), ("grad_x", xd.grad, egx),
                            ("grad_weight", f.c.weight.grad, egw),
                            ("grad_init_param", f.init_param.grad, egi),
                            ("grad_logit_bias", f.logit_bias.grad, egb)):
        assert_close(np_of(got), want, tol, name)
        assert_norm_rel(np_of(got), want, tol, name)
