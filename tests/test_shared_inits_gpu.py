"""GPU parity of the scan's inits forms that the filter module uses for its
(H, D) ``init_param`` (``ltv_hm_look_back_scan_{forward,backward}_split_ws``
with ``inits_dtype`` and a batch-stride-0 ``grad_inits``):

* fp32 inits with bf16 values are rounded to bf16 as they are read -- the
  outputs are bitwise those of the same call on the bf16-cast inits (the
  reference casts ``init_param.expand(B, H, D)`` to bf16 before its kernel);
* a grad_inits view with batch stride 0 receives the sum over the batch of
  each sequence's gradient rounded to the values' dtype, in fp32 in batch
  order -- bitwise a float32 loop over b of the per-sequence bf16 gradients
  (which is the cast's and the broadcast's backward), stored in the inits'
  dtype;
* the filter module's forward and backward with the parameter passed as it is
  equal those of the cast-and-broadcast path (outputs and x / weight / bias
  gradients bitwise, init_param's gradient to fp32 summation order);
* the same batch sum on look-back windows the short-window kernels take.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import ltv_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _F():
    from nanochat_amd.ops import ltv_hm_fast as F
    return F


def _case(B, T, NH, NKVH, Da, r, seed, init_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    H, D = NH + 2 * NKVH, Da * r
    values = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(DEV)
    logits = (-(2.0 + torch.randn(B, T, H * Da, generator=g))).to(torch.bfloat16).to(DEV)
    param = torch.randn(H, D, generator=g).to(init_dtype).to(DEV)
    bias = (0.1 * torch.randn(H, Da, generator=g)).to(DEV)
    gys = [torch.randn(B, nh, T, D, generator=g).to(torch.bfloat16).to(DEV)
           for nh in (NH, NKVH, NKVH)]
    return values, logits, param, bias, gys


# (B, T, NH, NKVH, Da, r): the d12 gate shape through the tile kernels, the
# chained backward, the chained forward (8 chunks of 512 steps), gate groups of
# 16 channels, per-channel gates
SHAPES = [(32, 256, 6, 6, 1, 128), (2, 700, 2, 1, 1, 128), (1, 3600, 1, 1, 1, 128),
          (3, 300, 1, 1, 8, 16), (2, 129, 1, 1, 64, 1), (1, 200, 2, 1, 1, 128)]


@pytest.mark.parametrize("B,T,NH,NKVH,Da,r", SHAPES)
@pytest.mark.parametrize("init_dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_shared_inits_forward_and_batch_sum(B, T, NH, NKVH, Da, r, init_dtype):
    F = _F()
    H, D = NH + 2 * NKVH, Da * r
    Fp = F.packed_width(H, D, Da)
    values, logits, param, bias, gys = _case(B, T, NH, NKVH, Da, r, seed=B * T + r,
                                             init_dtype=init_dtype)
    expanded = param.to(torch.bfloat16).unsqueeze(0).expand(B, H, D).contiguous()
    # forward: (H, D) inits in their own dtype == the bf16-cast (B, H, D) inits
    shared = F.scan_forward(values, logits, param, bias, NH, NKVH, Da, r, True)
    ref = F.scan_forward(values, logits, expanded, bias, NH, NKVH, Da, r, True)
    for a, b in zip(shared, ref):
        assert torch.equal(a, b)
    hq, hk, hv = ref
    # backward: the batch sum, next to the per-sequence bf16 gradients
    gc_s = torch.zeros(B, T, Fp, dtype=torch.bfloat16, device=DEV)
    gi_s, gb_s = F.scan_backward(values, logits, param, bias, hq, hk, hv, *gys, NH, NKVH, Da, r,
                                 True, gc_s)
    gc_r = torch.zeros_like(gc_s)
    gi_r, gb_r = F.scan_backward(values, logits, expanded, bias, hq, hk, hv, *gys, NH, NKVH, Da,
                                 r, True, gc_r)
    assert gi_s.shape == (H, D) and gi_s.dtype == init_dtype
    assert torch.equal(gc_s, gc_r) and torch.equal(gb_s, gb_r)
    per_seq = gi_r.float().cpu().numpy()  # (B, H, D), bf16 values widened
    want = np.zeros((H, D), np.float32)
    for b in range(B):
        want = (want + per_seq[b]).astype(np.float32)
    want_t = torch.from_numpy(want).to(init_dtype)
    assert torch.equal(gi_s.cpu(), want_t), float((gi_s.float().cpu() - want_t.float()).abs().max())
    # and within the fp32 summation order of torch's own reduction (plus, for
    # bf16 inits, the rounding of the sum to bf16: one step, 2^-8 relative)
    rtol = 1e-5 if init_dtype == torch.float32 else 2.0 ** -8
    torch.testing.assert_close(gi_s.float(), gi_r.float().sum(0), rtol=rtol, atol=1e-5)


def test_per_sequence_fp32_inits():
    """(B, H, D) fp32 inits (one set per sequence): read rounded to bf16, and
    grad_inits in fp32 = the bf16 gradients widened."""
    F = _F()
    B, T, NH, NKVH, Da, r = 3, 500, 2, 1, 1, 128
    H, D = NH + 2 * NKVH, Da * r
    values, logits, _, bias, gys = _case(B, T, NH, NKVH, Da, r, seed=9)
    inits32 = torch.randn(B, H, D, device=DEV)
    inits16 = inits32.to(torch.bfloat16)
    a = F.scan_forward(values, logits, inits32, bias, NH, NKVH, Da, r, True)
    b = F.scan_forward(values, logits, inits16, bias, NH, NKVH, Da, r, True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    Fp = F.packed_width(H, D, Da)
    gc1 = torch.zeros(B, T, Fp, dtype=torch.bfloat16, device=DEV)
    gc2 = torch.zeros_like(gc1)
    gi32, _ = F.scan_backward(values, logits, inits32, bias, *b, *gys, NH, NKVH, Da, r, True, gc1)
    gi16, _ = F.scan_backward(values, logits, inits16, bias, *b, *gys, NH, NKVH, Da, r, True, gc2)
    assert gi32.dtype == torch.float32
    assert torch.equal(gi32, gi16.float()) and torch.equal(gc1, gc2)


def test_shared_inits_oracle_rows():
    """The batch-summed fp32 inits gradient against the oracle's per-sequence
    gradients (computed from the bf16-rounded parameter) summed in float64."""
    F = _F()
    B, T, NH, NKVH, Da, r = 4, 64, 1, 1, 1, 128
    H, D = NH + 2 * NKVH, Da * r
    values, logits, param, bias, gys = _case(B, T, NH, NKVH, Da, r, seed=4)
    q, k, v = F.scan_forward(values, logits, param, bias, NH, NKVH, Da, r, True)
    Fp = F.packed_width(H, D, Da)
    gc = torch.zeros(B, T, Fp, dtype=torch.bfloat16, device=DEV)
    gi, _ = F.scan_backward(values, logits, param, bias, q, k, v, *gys, NH, NKVH, Da, r, True, gc)
    comb = torch.cat([values.permute(0, 2, 1, 3),
                      logits.view(B, T, H, Da)], dim=3).reshape(B, T, H * (D + Da))
    ini = param.to(torch.bfloat16).float().unsqueeze(0).expand(B, H, D).cpu().numpy()
    gy = torch.cat(gys, dim=1).float().cpu().numpy()
    _, egi, _ = O.scan_backward(comb.float().cpu().numpy(), ini, bias.cpu().numpy(),
                                q.float().cpu().numpy(), k.float().cpu().numpy(),
                                v.float().cpu().numpy(), gy[:, :NH], gy[:, NH:NH + NKVH],
                                gy[:, NH + NKVH:], NH, NKVH, Da, r, True, "bf16")
    want = egi.astype(np.float64).sum(0)
    got = gi.double().cpu().numpy()
    scale = max(1.0, float(np.abs(want).max()))
    assert np.abs(got - want).max() <= 2e-2 * scale


# (B, T, NH, NKVH, Da, r, (P, Q, K)): look-back windows the short-window kernels
# take -- one window per lane, several per lane (the d12 spec), 16-channel gate
# groups, per-channel gates
LB_SHAPES = [(2, 64, 1, 1, 1, 128, (16, 16, 4)), (5, 300, 2, 1, 1, 128, (16, 16, 9)),
             (3, 300, 1, 1, 8, 16, (32, 8, 9)), (2, 129, 1, 1, 64, 1, (16, 16, 9))]


@pytest.fixture
def windows_per_lane():
    from nanochat_amd import _native as N
    lib = N.lib()

    def set_(n):
        N.check(lib.ltv_lb_set_windows_per_lane(n), "ltv_lb_set_windows_per_lane")

    try:
        yield set_
    finally:
        set_(0)


@pytest.mark.parametrize("wpl", [0, 3], ids=["auto", "wpl3"])
@pytest.mark.parametrize("B,T,NH,NKVH,Da,r,pqk", LB_SHAPES, ids=str)
@pytest.mark.parametrize("init_dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_shared_inits_look_back_batch_sum(B, T, NH, NKVH, Da, r, pqk, init_dtype, wpl,
                                          windows_per_lane):
    """Look-back windows with (H, D) inits: outputs bitwise those of the
    bf16-cast (B, H, D) inits, grad_combined and grad_logit_bias bitwise, and
    grad_inits bitwise the float32 batch-order sum of the per-sequence bf16
    gradients (the per-window shares summed per sequence, then over the batch
    by the reduction launch); with the automatic windows per lane and with
    three (the several-window kernel where the spec allows it)."""
    windows_per_lane(wpl)
    F = _F()
    H, D = NH + 2 * NKVH, Da * r
    Fp = F.packed_width(H, D, Da)
    values, logits, param, bias, gys = _case(B, T, NH, NKVH, Da, r, seed=B + T + r,
                                             init_dtype=init_dtype)
    expanded = param.to(torch.bfloat16).unsqueeze(0).expand(B, H, D).contiguous()
    shared = F.scan_forward(values, logits, param, bias, NH, NKVH, Da, r, True, *pqk)
    ref = F.scan_forward(values, logits, expanded, bias, NH, NKVH, Da, r, True, *pqk)
    for a, b in zip(shared, ref):
        assert torch.equal(a, b)
    gc_s = torch.zeros(B, T, Fp, dtype=torch.bfloat16, device=DEV)
    gi_s, gb_s = F.scan_backward(values, logits, param, bias, *ref, *gys, NH, NKVH, Da, r, True,
                                 gc_s, *pqk)
    gc_r = torch.zeros_like(gc_s)
    gi_r, gb_r = F.scan_backward(values, logits, expanded, bias, *ref, *gys, NH, NKVH, Da, r,
                                 True, gc_r, *pqk)
    assert gi_s.shape == (H, D) and gi_s.dtype == init_dtype
    assert torch.equal(gc_s, gc_r) and torch.equal(gb_s, gb_r)
    per_seq = gi_r.float().cpu().numpy()
    want = np.zeros((H, D), np.float32)
    for b in range(B):
        want = (want + per_seq[b]).astype(np.float32)
    assert torch.equal(gi_s.cpu(), torch.from_numpy(want).to(init_dtype))


def test_unsupported_forms_are_refused():
    """A batch-summed grad_inits needs the full recurrence with gate groups
    the tile kernels reduce, or look-back windows the short-window kernels
    take; the values' dtype must be bf16 for fp32 inits.  Each is an error
    before any launch."""
    F = _F()
    B, T, NH, NKVH, Da, r = 2, 64, 1, 1, 1, 128
    H, D = NH + 2 * NKVH, Da * r
    values, logits, param, bias, gys = _case(B, T, NH, NKVH, Da, r, seed=1)
    with pytest.raises(RuntimeError, match="full recurrence"):  # not a short-window spec
        F.scan_forward(values, logits, param, bias, NH, NKVH, Da, r, True, P=16, Q=100, K=4)
    with pytest.raises(RuntimeError, match="float32 with bfloat16"):
        F.scan_forward(values.float(), logits.float(), param.to(torch.bfloat16), bias, NH, NKVH,
                       Da, r, True)
    # r = 3 (D = 24): gate groups outside the tile kernels' reductions
    B, T, NH, NKVH, Da, r = 2, 32, 1, 1, 8, 3
    H, D = NH + 2 * NKVH, Da * r
    values, logits, param, bias, gys = _case(B, T, NH, NKVH, Da, r, seed=2)
    q, k, v = F.scan_forward(values, logits, param, bias, NH, NKVH, Da, r, True)
    gc = torch.zeros(B, T, F.packed_width(H, D, Da), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="batch"):
        F.scan_backward(values, logits, param, bias, q, k, v, *gys, NH, NKVH, Da, r, True, gc)


def test_empty_time_zeroes_shared_grad():
    F = _F()
    B, T, NH, NKVH, Da, r = 2, 0, 1, 1, 1, 128
    H, D = NH + 2 * NKVH, Da * r
    values = torch.zeros(B, H, 0, D, dtype=torch.bfloat16, device=DEV)
    logits = torch.zeros(B, 0, H * Da, dtype=torch.bfloat16, device=DEV)
    param = torch.randn(H, D, device=DEV)
    bias = torch.zeros(H, Da, device=DEV)
    q, k, v = F.scan_forward(values, logits, param, bias, NH, NKVH, Da, r, True)
    gys = [torch.zeros_like(t) for t in (q, k, v)]
    gc = torch.zeros(B, 0, F.packed_width(H, D, Da), dtype=torch.bfloat16, device=DEV)
    gi, gb = F.scan_backward(values, logits, param, bias, q, k, v, *gys, NH, NKVH, Da, r, True, gc)
    assert gi.shape == (H, D) and int(torch.count_nonzero(gi)) == 0
    assert int(torch.count_nonzero(gb)) == 0


@pytest.mark.parametrize("B,T,Da,r", [(4, 256, 1, 128), (2, 700, 1, 128), (3, 128, 8, 16)])
def test_filter_shared_inits_match_cast_and_broadcast(B, T, Da, r):
    """The module's step with init_param passed as it is against the same step
    through the cast-and-broadcast autograd function."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
        LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter)
    NH, NKVH, D, C = 2, 1, Da * r, 256
    torch.manual_seed(B + T)
    f = Filter(NH, NKVH, D, r).to(DEV)
    with torch.no_grad():
        f.c.weight.normal_(0.0, C ** -0.5)
        f.init_param.normal_()
        f.logit_bias.normal_(0.0, 0.1)
    x = torch.randn(B, T, C, device=DEV).to(torch.bfloat16)
    grads = [torch.randn(B, T, nh, D, device=DEV).to(torch.bfloat16) for nh in (NH, NKVH, NKVH)]

    def step(shared):
        f.zero_grad(set_to_none=True)
        f._shared_inits_in_kernel = (lambda: shared)
        xs = x.clone().requires_grad_(True)
        q, k, v = f(xs, LtvInitValues())
        torch.autograd.backward([q, k, v], grads)
        del f._shared_inits_in_kernel
        return ((q, k, v), xs.grad, f.c.weight.grad.clone(), f.logit_bias.grad.clone(),
                f.init_param.grad.clone())

    new, old = step(True), step(False)
    for a, b in zip(new[0], old[0]):
        assert torch.equal(a, b)
    for name, a, b in (("x", new[1], old[1]), ("weight", new[2], old[2]),
                       ("logit_bias", new[3], old[3])):
        assert torch.equal(a, b), name
    assert new[4].dtype == torch.float32
    torch.testing.assert_close(new[4], old[4], rtol=1e-5, atol=1e-6)


def test_zero_pad_and_zero_padded_grad_x():
    """scan_backward(zero_pad=True) sets grad_combined's columns F ..
    round_up(F, 8) - 1 to zero and leaves every other column it does not own
    untouched; grad_x through ltv_qkv_project_backward_input_zero_padded on it
    equals the zeroing entry point's bitwise."""
    F_ = _F()
    B, T, NH, NKVH, Da, r, C = 2, 300, 6, 6, 1, 128, 256
    H, D = NH + 2 * NKVH, Da * r
    Fv, Fp = H * (D + Da), F_.packed_width(H, D, Da)
    pad_end = (Fv + 7) // 8 * 8
    assert pad_end > Fv
    values, logits, param, bias, gys = _case(B, T, NH, NKVH, Da, r, seed=21)
    q, k, v = F_.scan_forward(values, logits, param, bias, NH, NKVH, Da, r, True)
    gc = torch.full((B, T, Fp), float("nan"), dtype=torch.bfloat16, device=DEV)
    F_.scan_backward(values, logits, param, bias, q, k, v, *gys, NH, NKVH, Da, r, True, gc,
                     zero_pad=True)
    assert int(torch.count_nonzero(gc[..., Fv:pad_end])) == 0
    assert bool(torch.isnan(gc[..., pad_end:].float()).all())
    assert not bool(torch.isnan(gc[..., :Fv].float()).any())
    ref = torch.full_like(gc, float("nan"))
    F_.scan_backward(values, logits, param, bias, q, k, v, *gys, NH, NKVH, Da, r, True, ref)
    assert torch.equal(gc[..., :Fv], ref[..., :Fv])
    assert bool(torch.isnan(ref[..., Fv:pad_end].float()).all())  # not asked: untouched
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, T, C, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(Fv, C, generator=g) * C ** -0.5).to(DEV)
    wpack = F_.pack_weight(w, H, D, Da)
    gx_p, gw_p = F_.project_backward(x, wpack, gc, H, D, Da, pad_zeroed=True)
    gx_z, gw_z = F_.project_backward(x, wpack, ref, H, D, Da)
    assert torch.equal(gx_p, gx_z) and torch.equal(gw_p, gw_z)
