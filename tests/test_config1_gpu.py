"""configs[1] at the bench's own shape: the standalone per-element-decay scan
(r = 1, Da = D = 128) over bf16 head-major values (32, 18, 1024, 128), logits
-z with z ~ N(2, 1), through ``ltv_hm_fast.scan_forward`` -- the call
``bench.py --workload scan_fwd`` times.  The reference checks the exact call it
times the same way: its benchmark mode runs T = 1024, D = 128 and asserts
against the Python reference
(``tests/test_ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py:40-45, 104-109``).

At this shape the library launches 1,152 workgroups (two 64-channel slabs per
(b, head)), which selects the forward's (CL, L, NW) = (8, 2, 4) launch shape
with streaming stores; smaller grids (every other r = 1 test) take 4 steps per
lane.  The backward at the same shape runs the tile kernel with per-channel
gates (no lane-group dlogit sum).

Checked: sampled batch rows (all 18 heads) against the CPU oracle within the
bf16 tolerance, two runs bitwise equal, and grad_logit_bias (a sum over every
row) against the fp64 sum of the kernel's own dlogit outputs within their bf16
rounding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import TOL, assert_close, assert_norm_rel, np_of

pytestmark = pytest.mark.gpu

DEV = "cuda"
B, NH, NKVH, T, D = 32, 6, 6, 1024, 128
H = NH + 2 * NKVH
DA, R = D, 1
FWD_ROWS = (0, 17, 31)
BWD_ROWS = (0, 31)
BF = torch.bfloat16


@pytest.fixture(scope="module")
def case():
    g = torch.Generator().manual_seed(0)
    u = torch.randn(B, H, T, D, generator=g).to(BF)
    lg = (-(2.0 + torch.randn(B, H, T, D, generator=g))).to(BF)
    ini = torch.randn(B, H, D, generator=g).to(BF)
    gys = [torch.randn(B, nh, T, D, generator=g).to(BF) for nh in (NH, NKVH, NKVH)]
    return u, lg, ini, gys


def _comb(u, lg, rows):
    """Rows of the oracle's combined (R, T, H (D + Da)) layout."""
    uu = u[list(rows)].float().numpy().transpose(0, 2, 1, 3)
    ll = lg[list(rows)].float().numpy().transpose(0, 2, 1, 3)
    return np.concatenate([uu, ll], axis=-1).reshape(len(rows), T, -1)


def test_config1_forward_at_bench_shape(case):
    from nanochat_amd import _native as N
    from nanochat_amd.ops import ltv_hm_fast as hm
    u, lg, ini, _ = case
    ud, ld, idv = u.to(DEV), lg.to(DEV), ini.to(DEV)
    bias = torch.zeros(H, DA, dtype=torch.float32, device=DEV)
    # the tile kernel, not the chained one, runs at this shape
    assert N.lib().ltv_hm_scan_forward_chain_workspace_size(N.DTYPE_BF16, B, T, NH, NKVH, DA,
                                                            R) == 0
    first = hm.scan_forward(ud, ld, idv, bias, NH, NKVH, DA, R, True)
    second = hm.scan_forward(ud, ld, idv, bias, NH, NKVH, DA, R, True)
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert torch.equal(a, b), "two runs differ"
    rows = list(FWD_ROWS)
    want = O.scan_forward(_comb(u, lg, rows), ini[rows].float().numpy(),
                          np.zeros((H, DA), np.float32), NH, NKVH, DA, R, True, "bf16")
    for name, got, w in zip("qkv", first, want):
        assert_close(np_of(got[rows]), w, TOL[BF], f"configs[1] forward {name}")
        assert_norm_rel(np_of(got[rows]), w, TOL[BF], f"configs[1] forward {name}")


def test_config1_backward_at_bench_shape(case):
    from nanochat_amd.ops import ltv_hm_fast as hm
    u, lg, ini, gys = case
    ud, idv = u.to(DEV), ini.to(DEV)
    # the backward takes token-major logits (B, T, H Da): column h Da + j
    lg3 = lg.permute(0, 2, 1, 3).reshape(B, T, H * DA).contiguous()
    ld3 = lg3.to(DEV)
    bias = torch.zeros(H, DA, dtype=torch.float32, device=DEV)
    hq, hk, hv = hm.scan_forward(ud, ld3, idv, bias, NH, NKVH, DA, R, True)
    gd = [g.to(DEV) for g in gys]
    Fp = hm.packed_width(H, D, DA)
    F = H * (D + DA)

    def run():
        gc = torch.zeros(B, T, Fp, dtype=BF, device=DEV)
        gi, gb = hm.scan_backward(ud, ld3, idv, bias, hq, hk, hv, *gd, NH, NKVH, DA, R, True, gc)
        return gc, gi, gb

    gc, gi, gb = run()
    gc2, gi2, gb2 = run()
    torch.cuda.synchronize()
    assert torch.equal(gc[..., :F], gc2[..., :F]) and torch.equal(gi, gi2) and torch.equal(gb, gb2)

    rows = list(BWD_ROWS)
    saved = [np_of(h[rows]) for h in (hq, hk, hv)]
    gy = [g[rows].float().numpy() for g in gys]
    egc, egi, _ = O.scan_backward(_comb(u, lg, rows), ini[rows].float().numpy(),
                                  np.zeros((H, DA), np.float32), *saved, *gy, NH, NKVH, DA, R,
                                  True, "bf16")
    # grad_combined: values of head h at columns h D + d, logits at H D + h Da + j
    got = np_of(gc[rows])
    e = egc.reshape(len(rows), T, H, D + DA)
    assert_close(got[..., :H * D], e[..., :D].reshape(len(rows), T, H * D), TOL[BF],
                 "configs[1] backward d(values)")
    assert_close(got[..., H * D:F], e[..., D:].reshape(len(rows), T, H * DA), TOL[BF],
                 "configs[1] backward d(logits)")
    assert_close(np_of(gi[rows]), egi, TOL[BF], "configs[1] backward d(inits)")

    # grad_logit_bias sums the unrounded fp32 dlogits over every (b, t); the
    # kernel's bf16 dlogit outputs are those values rounded (relative error
    # <= 2^-9 each), so their fp64 sum bounds it
    dl = gc[..., H * D:F].double().reshape(B * T, H, DA)
    s = dl.sum(dim=0)
    bound = dl.abs().sum(dim=0) * 2.0 ** -8 + 1e-6
    err = (gb.double() - s).abs()
    assert bool((err <= bound).all()), (
        f"grad_logit_bias off its dlogit sum: max err {float(err.max()):.3e}, "
        f"bound at that element {float(bound.flatten()[int(err.argmax())]):.3e}")
