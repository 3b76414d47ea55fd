"""GPU parity of the projection backward's single launch for both GEMMs
(``ltv_qkv_project_backward`` / ``_zero_padded``: ``gemm_dma_bwd_fused_kernel``
where grad_x's 256 x 256 tiles take between one and two rounds of the device's
compute units).  grad_x must be bitwise that of the separate grad_x call (the
same kernel body and work items); grad_weight sums the same products over
other split boundaries, so it is checked against the separate grad_weight
call to fp32 summation accuracy and against a float64 product of the same
bf16 operands.  Token counts where the fused launch applies with different
plans (d12's 384 grad_x tiles, 480, 192) and where it does not (768: whole
rounds).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ltv_test_utils import assert_close, np_of

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _separate(N, lib, x, wpack, gc, H, D, Da):
    """grad_x and grad_weight through the two separate calls."""
    B, T, C = x.shape
    M = B * T
    st = N.stream_of(x)
    gx = torch.empty((B, T, C), dtype=torch.bfloat16, device=DEV)
    gw = torch.empty((H * (D + Da), C), dtype=torch.float32, device=DEV)
    nb = lib.ltv_qkv_project_backward_workspace_size(M, C, H, D, Da)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=DEV)
    N.check(lib.ltv_qkv_project_backward_input_zero_padded(
        x.data_ptr(), wpack.data_ptr(), gc.data_ptr(), gx.data_ptr(), M, C, H, D, Da, st), "dx")
    N.check(lib.ltv_qkv_project_backward_weight(
        x.data_ptr(), gc.data_ptr(), gw.data_ptr(), ws.data_ptr(), nb, M, C, H, D, Da, st), "dw")
    return gx, gw


@pytest.mark.parametrize("B,T,C", [(32, 1024, 768), (40, 1024, 768), (16, 1024, 768),
                                   (64, 1024, 768), (1, 33000, 768), (3, 11000, 640)],
                         ids=lambda v: str(v))
def test_combined_backward_matches_separate_calls(B, T, C):
    """(32, 1024): d12's 384 grad_x tiles; (40, 1024): 480 tiles, other piece
    lengths; (16, 1024): 192 tiles, a quarter of the CUs with no grad_x tile;
    (64, 1024): 768 tiles, whole rounds, the two GEMMs one after the other;
    (1, 33000): ragged last token tile and reduction (516 k-steps);
    (3, 11000, 640): partial channel tiles."""
    from nanochat_amd import _native as N
    from nanochat_amd.ops import ltv_hm_fast as F_
    lib = N.lib()
    NH, NKVH, D, Da = 6, 6, 128, 1
    H = NH + 2 * NKVH
    F = H * (D + Da)
    Fp = F_.packed_width(H, D, Da)
    g = torch.Generator(device=DEV).manual_seed(B)
    x = torch.randn(B, T, C, generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn(F, C, generator=g, device=DEV) / C ** 0.5
    wpack = F_.pack_weight(w, H, D, Da)
    gc = torch.randn(B, T, Fp, generator=g, device=DEV).to(torch.bfloat16)
    gc[..., F:] = 0  # the padding columns the scan backward zeroes
    gx_s, gw_s = _separate(N, lib, x, wpack, gc, H, D, Da)
    gx_f, gw_f = F_.project_backward(x, wpack, gc, H, D, Da, pad_zeroed=True)
    torch.cuda.synchronize()
    assert torch.equal(gx_f, gx_s), "grad_x differs from the separate call"
    # the same fp32 products summed over other split boundaries
    scale = gw_s.abs().max().item()
    err = (gw_f - gw_s).abs().max().item()
    assert err <= 1e-5 * scale, (err, scale)
    # and the not-zero-padded entry (zeroes the padding itself) on NaN padding
    gc2 = gc.clone()
    gc2[..., F:] = float("nan")
    gx_n, gw_n = F_.project_backward(x, wpack, gc2, H, D, Da)
    assert torch.equal(gx_n, gx_f) and torch.equal(gw_n, gw_f)
    # against a float64 product of the same bf16 operands, on sampled rows
    rows = torch.arange(0, F, 37, device=DEV)
    cols_i = torch.cat([gc[..., : H * D].view(B, T, H, D), gc[..., H * D: F].view(B, T, H, Da)],
                       dim=-1).reshape(B * T, F)[:, rows].double().cpu()
    want = cols_i.T @ x.reshape(B * T, C).double().cpu()
    assert_close(np_of(gw_f[rows]), want.numpy(), 2e-2, "grad_weight rows")


def test_combined_backward_is_deterministic():
    from nanochat_amd.ops import ltv_hm_fast as F_
    B, T, C, H, D, Da = 32, 1024, 768, 18, 128, 1
    F = H * (D + Da)
    Fp = F_.packed_width(H, D, Da)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(B, T, C, generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn(F, C, generator=g, device=DEV) / C ** 0.5
    wpack = F_.pack_weight(w, H, D, Da)
    gc = torch.randn(B, T, Fp, generator=g, device=DEV).to(torch.bfloat16)
    a = F_.project_backward(x, wpack, gc, H, D, Da)
    b = F_.project_backward(x, wpack, gc, H, D, Da)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
