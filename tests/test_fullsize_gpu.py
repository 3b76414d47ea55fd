"""Parity of the d12 training shape at full size.

B = 32, T = 1024, C = 768, 6 + 2 x 6 heads of 128, r = 128 (F = 2322), bf16,
forward and backward through the drop-in filter module -- the shape bench.py
times.  At this size the persistent projection GEMMs run several work items per
workgroup (1,280 forward and 384 dX items over 256 CUs), dW runs 8 splits of the
token reduction, and the scan grids cover 576 (b, head) sequences; the config-1
tests reach none of that.

Checks:
* sampled batch rows b in {0, 13, 31}: q, k, v, grad_x and grad_inits against
  the oracle run end to end from x and the bf16-rounded master weight;
* every row: the projection outputs (values, logits) against a float64 product
  of the same bf16 operands, bounded by one bf16 rounding plus the fp32
  accumulation error; the scan outputs and every scan gradient against the
  oracle's scan run on the kernel's own projection outputs; grad_x and
  grad_weight against float64 products of the kernel's own grad_combined;
* the module's autograd gives bit-identical results to the library calls it is
  made of, and two backward passes are bitwise identical.

Inputs follow configs[2]: x ~ N(0, 1); W ~ N(0, 1/768) (value and gate rows);
init_param ~ N(0, 1/768); upstream gradients ~ N(0, 1); logit_bias = 0 (gates
near 1/2), and a long-memory case with logit_bias = -3 (decay about 0.95).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import TOL, assert_close, assert_norm_rel, np_of

pytestmark = pytest.mark.gpu
DEV = "cuda"

B, T, C = 32, 1024, 768
NH = NKVH = 6
D, R = 128, 128
DA = D // R
H = NH + 2 * NKVH
F = H * (D + DA)
ROWS = (0, 13, 31)
TOL_BF16 = TOL[torch.bfloat16]


def _packed_rows():
    """Packed-operand row -> parameter row: values of every head first
    (h D + d -> h (D + Da) + d), then the gate rows (H D + h Da + j ->
    h (D + Da) + D + j)."""
    h, d = np.meshgrid(np.arange(H), np.arange(D), indexing="ij")
    vals = (h * (D + DA) + d).reshape(-1)
    h, j = np.meshgrid(np.arange(H), np.arange(DA), indexing="ij")
    gates = (h * (D + DA) + D + j).reshape(-1)
    return np.concatenate([vals, gates])


def _interleave(values_bhtd: np.ndarray, logits_btl: np.ndarray) -> np.ndarray:
    """(B, H, T, D) values and (B, T, >= H Da) logits -> combined (B, T, F)."""
    b, _, t, _ = values_bhtd.shape
    comb = np.empty((b, t, H, D + DA), np.float32)
    comb[..., :D] = values_bhtd.transpose(0, 2, 1, 3)
    comb[..., D:] = logits_btl[:, :, :H * DA].reshape(b, t, H, DA)
    return comb.reshape(b, t, F)


def _check_gemm(got: torch.Tensor, a64: torch.Tensor, b64: torch.Tensor, k: int, out_bf16: bool,
                label: str):
    """Every element of an fp32-accumulated product of bf16 operands lies within
    the worst-case bound of the float64 product: fp32 accumulation over k terms,
    1.1 k 2^-24 sum|a||b|, plus for a bf16 output one rounding, 2^-8 |e|."""
    want = a64 @ b64
    bound = 1.1 * k * 2.0 ** -24 * (a64.abs() @ b64.abs())
    if out_bf16:
        bound = bound + 2.0 ** -8 * (want.abs() + bound)
    err = (got.double() - want).abs()
    n_bad = int((err > bound).sum())
    assert n_bad == 0, (f"{label}: {n_bad} elements outside the fp32-accumulation"
                        f"{' + bf16 rounding' if out_bf16 else ''} bound; worst excess "
                        f"{float((err - bound).max()):.3e}")


def _make_filter(bias: float):
    from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
        LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter,
    )
    torch.manual_seed(0)
    f = Filter(NH, NKVH, D, R)
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        f.c.weight.copy_(torch.randn(F, C, generator=g) * C ** -0.5)
        f.logit_bias.fill_(bias)
        f.init_param.copy_(torch.randn(H, D, generator=g) * C ** -0.5)
    return f.to(DEV)


@pytest.mark.parametrize("bias", [0.0, -3.0], ids=["bias0", "long_memory"])
def test_d12_full_size(bias):
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    from nanochat_amd.ops import ltv_hm_fast as hm
    print(f"[fullsize] B={B} T={T} C={C} H={H} r={R} bias={bias}", flush=True)

    f = _make_filter(bias)
    g = torch.Generator().manual_seed(1)
    x_cpu = torch.randn(B, T, C, generator=g).to(torch.bfloat16)
    dq_cpu = torch.randn(B, T, NH, D, generator=g).to(torch.bfloat16)
    dk_cpu = torch.randn(B, T, NKVH, D, generator=g).to(torch.bfloat16)
    dv_cpu = torch.randn(B, T, NKVH, D, generator=g).to(torch.bfloat16)
    x = x_cpu.to(DEV)
    dq, dk, dv = dq_cpu.to(DEV), dk_cpu.to(DEV), dv_cpu.to(DEV)

    def run():
        f.zero_grad(set_to_none=True)
        xd = x.clone().requires_grad_(True)
        q, k, v = f(xd, LtvInitValues())
        torch.autograd.backward([q, k, v], [dq, dk, dv])
        torch.cuda.synchronize()
        return (q.detach(), k.detach(), v.detach(), xd.grad, f.c.weight.grad.clone(),
                f.init_param.grad.clone(), f.logit_bias.grad.clone())

    out1 = run()
    out2 = run()
    names = ("q", "k", "v", "grad_x", "grad_weight", "grad_init_param", "grad_logit_bias")
    for name, a, b_ in zip(names, out1, out2):
        assert torch.equal(a, b_), f"{name}: two runs differ"
    q, k, v, gx, gw, gip, gb = out1

    # the library calls the module is made of, with their intermediates
    inits = f.init_param.detach().unsqueeze(0).expand(B, -1, -1).to(torch.bfloat16).contiguous()
    bias_t = f.logit_bias.detach().float().contiguous()
    with torch.no_grad():
        hq, hk, hv, values, logits, wpack = torch.ops.nanochat_amd.qkv_filter(
            x, f.c.weight.detach(), inits, bias_t, NH, NKVH, DA, R)
    assert torch.equal(hq.transpose(1, 2), q) and torch.equal(hk.transpose(1, 2), k)
    assert torch.equal(hv.transpose(1, 2), v)
    gc = torch.empty((B, T, hm.packed_width(H, D, DA)), dtype=torch.bfloat16, device=DEV)
    gi_k, gb_k = hm.scan_backward(values, logits, inits, bias_t, hq, hk, hv,
                                  dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2),
                                  NH, NKVH, DA, R, True, gc)
    gx_k, gw_k = hm.project_backward(x, wpack, gc, H, D, DA)
    torch.cuda.synchronize()
    assert torch.equal(gx_k, gx), "module grad_x differs from the library calls"
    assert torch.equal(gw_k, gw), "module grad_weight differs from the library calls"
    assert torch.equal(gb_k.view_as(gb), gb), "module grad_logit_bias differs"
    assert_close(np_of(gi_k.float().sum(0)), np_of(gip), 1e-6, "grad_init_param (batch sum)")

    # --- projection: every token against a float64 product of the bf16 operands
    perm = torch.from_numpy(_packed_rows()).to(DEV)
    w_bf = f.c.weight.detach().to(torch.bfloat16)
    assert torch.equal(wpack[:F], w_bf[perm]), "packed weight is not the bf16 weight reordered"
    x64 = x.reshape(B * T, C).double()
    wt64 = w_bf[perm].double().t().contiguous()  # (C, F), packed column order
    comb_k = torch.cat([values.permute(0, 2, 1, 3).reshape(B * T, H * D),
                        logits.reshape(B * T, -1)[:, :H * DA]], dim=1)
    _check_gemm(comb_k, x64, wt64, C, True, "projection (values | logits)")

    # --- scan over every (b, head): oracle on the kernel's own projection outputs
    vals_np = np_of(values)
    lg_np = np_of(logits)
    comb = _interleave(vals_np, lg_np)
    ini_np = np_of(inits)
    bias_np = np_of(bias_t)
    eq, ek, ev = O.scan_forward(comb, ini_np, bias_np, NH, NKVH, DA, R, True, "bf16")
    for name, got, want in (("q", hq, eq), ("k", hk, ek), ("v", hv, ev)):
        assert_close(np_of(got), want, TOL_BF16, f"scan {name} (all rows)")
        assert_norm_rel(np_of(got), want, TOL_BF16, f"scan {name} (all rows)")
    e_gc, e_gi, e_gb = O.scan_backward(
        comb, ini_np, bias_np, np_of(hq), np_of(hk), np_of(hv),
        np_of(dq.transpose(1, 2)), np_of(dk.transpose(1, 2)), np_of(dv.transpose(1, 2)),
        NH, NKVH, DA, R, True, "bf16")
    del comb
    gc_np = np_of(gc)
    e_gc = e_gc.reshape(B, T, H, D + DA)
    got_du = gc_np[..., :H * D].reshape(B, T, H, D)
    got_dl = gc_np[..., H * D:H * D + H * DA].reshape(B, T, H, DA)
    assert_close(got_du, e_gc[..., :D], TOL_BF16, "scan grad values (all rows)")
    assert_norm_rel(got_du, e_gc[..., :D], TOL_BF16, "scan grad values (all rows)")
    assert_close(got_dl, e_gc[..., D:], TOL_BF16, "scan grad logits (all rows)")
    assert_norm_rel(got_dl, e_gc[..., D:], TOL_BF16, "scan grad logits (all rows)")
    assert_close(np_of(gi_k), e_gi, TOL_BF16, "scan grad inits (all rows)")
    assert_close(np_of(gb_k), e_gb, TOL_BF16, "scan grad logit_bias (all rows)")
    assert_norm_rel(np_of(gb_k), e_gb, TOL_BF16, "scan grad logit_bias (all rows)")
    del e_gc, got_du, got_dl

    # --- projection backward: float64 products of the kernel's own grad_combined
    gc64 = gc[..., :F].reshape(B * T, F).double()
    _check_gemm(gx.reshape(B * T, C), gc64, wpack[:F].double(), F, True, "grad_x (all rows)")
    gw_packed = gw[perm]  # parameter rows in packed order
    # dW reduces B*T tokens in 4096-token splits summed in fixed order: the
    # fp32 accumulation bound is that of 4096 + 8 terms, not of B*T
    _check_gemm(gw_packed, gc64.t().contiguous(), x64, 4096 + 8, False, "grad_weight")
    del gc64, x64

    # --- sampled rows end to end: the oracle from x and the bf16 master weight
    rows = list(ROWS)
    xr = x_cpu[rows].float().numpy()
    w_np = O.bf16_round(f.c.weight.detach().float().cpu().numpy())
    ini_r = ini_np[rows]
    (oq, ok, ov, ocomb, saved) = O.filter_forward(xr, w_np, ini_r, bias_np, NH, NKVH, DA, R,
                                                  "bf16")
    ogx, _, ogi, _ = O.filter_backward(xr, w_np, ini_r, bias_np, ocomb, saved,
                                       dq_cpu[rows].float().numpy(),
                                       dk_cpu[rows].float().numpy(),
                                       dv_cpu[rows].float().numpy(), NH, NKVH, DA, R, "bf16")
    for name, got, want in (("q", q, oq), ("k", k, ok), ("v", v, ov)):
        assert_close(np_of(got[rows]), want, TOL_BF16, f"{name} rows {ROWS}")
        assert_norm_rel(np_of(got[rows]), want, TOL_BF16, f"{name} rows {ROWS}")
    assert_close(np_of(gx[rows]), ogx, TOL_BF16, f"grad_x rows {ROWS}")
    assert_norm_rel(np_of(gx[rows]), ogx, TOL_BF16, f"grad_x rows {ROWS}")
    assert_close(np_of(gi_k[rows]), ogi, TOL_BF16, f"grad_inits rows {ROWS}")
    print(f"[fullsize] bias={bias} ok", flush=True)
