"""The allocation-free scan backward (ltv_hm_scan_backward_noalloc) against
ltv_hm_scan_backward with a caller workspace, through the C ABI.

Both run the same kernels, so every output must be bitwise equal.  Two calls
in a row on each case, the second with a smaller input, check that what the
first call left in the shared device scratch does not leak into the second.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import assert_close, np_of, to_torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(B, T, NH, NKVH, Da, r, dtype, seed):
    """Seeded inputs, forward outputs (from the forward kernel) and upstream
    gradients for one backward call."""
    import nanochat_amd.ops  # noqa: F401
    H, D = NH + 2 * NKVH, Da * r
    g = torch.Generator().manual_seed(seed)
    c = torch.randn(B, T, H * (D + Da), generator=g)
    # gate logits: decay sigmoid(z), z ~ N(2, 1)  (logit = -z)
    c.view(B, T, H, D + Da)[..., D:] = -(2.0 + torch.randn(B, T, H, Da, generator=g))
    ini = 0.5 * torch.randn(B, H, D, generator=g)
    bias = 0.1 * torch.randn(H, Da, generator=g)
    gy = torch.randn(B, H, T, D, generator=g)
    c, ini, gy = (t.to(dtype).to(DEV) for t in (c, ini, gy))
    bias = bias.to(DEV)
    op = torch.ops.nanochat_cuda.ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op
    with torch.no_grad():
        hq, hk, hv = op(c, ini, bias, NH, NKVH, Da, r, 8, 8, 4, 32, 2, 8, True)
    grads = (gy[:, :NH].contiguous(), gy[:, NH:NH + NKVH].contiguous(),
             gy[:, NH + NKVH:].contiguous())
    return c, ini, bias, (hq, hk, hv), grads


def _call(noalloc, c, ini, bias, hs, grads, NH, NKVH, Da, r, fill):
    """One backward through the C ABI; the outputs start as `fill` so that an
    element the call does not write shows."""
    from nanochat_amd import _native as N
    lib = N.lib()
    B, T = c.shape[:2]
    gc = torch.full_like(c, fill)
    gi = torch.full_like(ini, fill)
    gb = torch.full((bias.shape[0], bias.shape[1]), fill, device=DEV, dtype=torch.float32)
    s4 = lambda t: N.strides(t, 4)  # noqa: E731
    args = [N.dtype_code(c.dtype), c.data_ptr(), N.strides(c, 3), ini.data_ptr(),
            N.strides(ini, 3), bias.data_ptr(),
            hs[0].data_ptr(), s4(hs[0]), hs[1].data_ptr(), s4(hs[1]), hs[2].data_ptr(), s4(hs[2]),
            grads[0].data_ptr(), s4(grads[0]), grads[1].data_ptr(), s4(grads[1]),
            grads[2].data_ptr(), s4(grads[2]),
            gc.data_ptr(), N.strides(gc, 3), gi.data_ptr(), N.strides(gi, 3), gb.data_ptr()]
    tail = [B, T, NH, NKVH, Da, r, 1, N.stream_of(c)]
    if noalloc:
        rc = lib.ltv_hm_scan_backward_noalloc(*args, *tail)
        N.check(rc, "ltv_hm_scan_backward_noalloc")
    else:
        ws_bytes = lib.ltv_hm_scan_backward_workspace_size(N.dtype_code(c.dtype), B, T, NH, NKVH,
                                                           Da, r)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        rc = lib.ltv_hm_scan_backward(*args, ws.data_ptr(), ws_bytes, *tail)
        N.check(rc, "ltv_hm_scan_backward")
    torch.cuda.synchronize()
    return gc, gi, gb


# (first call, second call): each pair shrinks; the long-T pairs use the
# time-chunked backward (chunk maps and carries in the scratch)
CASES = [
    ((8, 1024, 6, 6, 1, 128), (2, 256, 6, 6, 1, 128)),       # d12 heads, one chunk per (b, h)
    ((1, 4096, 1, 1, 1, 128), (1, 1000, 1, 1, 1, 128)),       # 3 sequences: chunked, then fewer chunks
    ((2, 700, 2, 1, 2, 64), (1, 33, 2, 1, 2, 64)),            # two gate groups per head
    ((1, 300, 1, 1, 128, 1), (1, 40, 1, 1, 128, 1)),          # per-channel gates (r = 1)
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("first,second", CASES, ids=[f"case{i}" for i in range(len(CASES))])
def test_noalloc_backward_matches_workspace_backward(dtype, first, second):
    for k, shape in enumerate((first, second)):
        B, T, NH, NKVH, Da, r = shape
        print(f"noalloc case {shape} {dtype} call {k}", flush=True)
        c, ini, bias, hs, grads = _inputs(B, T, NH, NKVH, Da, r, dtype, seed=11 + k)
        want = _call(False, c, ini, bias, hs, grads, NH, NKVH, Da, r, float("nan"))
        got = _call(True, c, ini, bias, hs, grads, NH, NKVH, Da, r, float("nan"))
        for name, a, b in zip(("grad_combined", "grad_inits", "grad_logit_bias"), got, want):
            assert not torch.isnan(b).any(), f"{name}: the workspace entry point left elements unwritten"
            assert torch.equal(a, b), f"{name} differs on call {k} of {shape}"


def test_noalloc_backward_matches_oracle_after_a_larger_call():
    """The second, smaller call also against the oracle (bf16 tolerance), so
    the comparison above is anchored to the reference semantics."""
    NH, NKVH, Da, r = 2, 1, 1, 128
    dtype = torch.bfloat16
    c, ini, bias, hs, grads = _inputs(4, 2048, NH, NKVH, Da, r, dtype, seed=3)
    _call(True, c, ini, bias, hs, grads, NH, NKVH, Da, r, 0.0)
    c, ini, bias, hs, grads = _inputs(2, 100, NH, NKVH, Da, r, dtype, seed=4)
    gc, gi, gb = _call(True, c, ini, bias, hs, grads, NH, NKVH, Da, r, float("nan"))
    cn, inin, biasn = np_of(c), np_of(ini), np_of(bias)
    hsn = [np_of(h) for h in hs]
    gyn = [np_of(g) for g in grads]
    egc, egi, egb = O.scan_backward(cn, inin, biasn, *hsn, *gyn, NH, NKVH, Da, r, True, "bf16")
    assert_close(np_of(gc), egc, 2e-2, "grad_combined")
    assert_close(np_of(gi), egi, 2e-2, "grad_inits")
    assert_close(np_of(gb), egb, 2e-2, "grad_logit_bias")


def test_noalloc_rejects_shapes_beyond_its_scratch():
    """A backward whose workspace exceeds the built-in scratch is refused with
    a clear error before any launch (here: odd gate groups take the
    per-channel fallback, whose workspace is B*H*T*D floats)."""
    from nanochat_amd import _native as N
    lib = N.lib()
    cap = lib.ltv_hm_scan_backward_noalloc_max_workspace()
    assert cap == 32 << 20
    B, T, NH, NKVH, Da, r = 4, 8192, 6, 6, 24, 3   # 3 channels per gate: per-channel path
    need = lib.ltv_hm_scan_backward_workspace_size(N.DTYPE_BF16, B, T, NH, NKVH, Da, r)
    assert need > cap
    z3 = (ctypes.c_int64 * 3)(0, 0, 0)
    z4 = (ctypes.c_int64 * 4)(0, 0, 0, 0)
    rc = lib.ltv_hm_scan_backward_noalloc(N.DTYPE_BF16, None, z3, None, z3, None, None, z4, None,
                                          z4, None, z4, None, z4, None, z4, None, z4, None, z3,
                                          None, z3, None, B, T, NH, NKVH, Da, r, 1, None)
    assert rc == 4 and "allocation-free" in N.last_error()
