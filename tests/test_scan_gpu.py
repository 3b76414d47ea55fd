"""GPU parity of the head-major LTV scan op (reference-layout entry points)
against the CPU oracle.

Mirrors tests/test_ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan.py
of the reference (forward :28-116, backward :119-261): the reference's integer
generators without the sigmoid over every stride layout of ``combined`` and
T in {1, 2, 3, 31, 32, 33} must match exactly, in bf16 and fp32; sigmoid cases
(golden vectors from the reference, random inputs, long T) must match within
the stated tolerance.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import (TOL, assert_close, int_combined, int_inits, int_logit_bias,
                            io_name, np_of, strided_copy, stride_layouts, to_torch)

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float32]


def _op():
    import nanochat_amd.ops  # noqa: F401
    return torch.ops.nanochat_cuda.ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op


def _run(combined, inits, bias, NH, NKVH, Da, r, sig, grads=None):
    """Forward (and backward with the given upstream grads) through the op."""
    op = _op()
    if grads is None:
        with torch.no_grad():
            return op(combined, inits, bias, NH, NKVH, Da, r, 8, 8, 4, 32, 2, 8, sig)
    combined = combined.detach().requires_grad_(True)
    inits = inits.detach().requires_grad_(True)
    bias = bias.detach().requires_grad_(True)
    outs = op(combined, inits, bias, NH, NKVH, Da, r, 8, 8, 4, 32, 2, 8, sig)
    torch.autograd.backward(outs, grads)
    return outs, combined.grad, inits.grad, bias.grad


def _expected(c, ini, bias, NH, NKVH, Da, r, sig, io, gy=None):
    outs = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, sig, io)
    if gy is None:
        return outs
    H = NH + 2 * NKVH
    g = O.scan_backward(c, ini, bias, *outs, gy[:, :NH], gy[:, NH:NH + NKVH], gy[:, NH + NKVH:H],
                        NH, NKVH, Da, r, sig, io)
    return outs, g


# ---------------------------------------------------------------------------
# exact integer cases over every stride layout (reference harness)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("T", [1, 2, 3, 31, 32, 33])
def test_forward_exact_all_strides(dtype, T):
    B, NH, NKVH, total_d = 4, 8, 8, 2
    for r in [rr for rr in range(1, total_d + 1) if total_d % rr == 0]:
        Da = total_d // r
        c = int_combined(B, T, NH, NKVH, Da, r)
        ini = int_inits(B, NH, NKVH, Da, r)
        bias = int_logit_bias(NH, NKVH, Da, False)
        eq, ek, ev = _expected(c, ini, bias, NH, NKVH, Da, r, False, io_name(dtype))
        ini_d = to_torch(ini, dtype, DEV)
        bias_d = to_torch(bias, torch.float32, DEV)
        for stride in stride_layouts(c.shape):
            comb = strided_copy(c, stride, dtype, DEV)
            q, k, v = _run(comb, ini_d, bias_d, NH, NKVH, Da, r, False)
            case = f"T={T} r={r} stride={stride}"
            assert_close(np_of(q), eq, 0, "q " + case)
            assert_close(np_of(k), ek, 0, "k " + case)
            assert_close(np_of(v), ev, 0, "v " + case)


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("T", [1, 2, 3, 31, 32, 33])
def test_backward_exact_all_strides(dtype, T):
    B, NH, NKVH, total_d = 4, 8, 8, 2
    H = NH + 2 * NKVH
    for r in [rr for rr in range(1, total_d + 1) if total_d % rr == 0]:
        Da = total_d // r
        D = Da * r
        c = int_combined(B, T, NH, NKVH, Da, r)
        ini = int_inits(B, NH, NKVH, Da, r)
        bias = int_logit_bias(NH, NKVH, Da, False)
        gy = np.ones((B, H, T, D), np.float32)  # the reference backs ones through
        (_, (egc, egi, egb)) = _expected(c, ini, bias, NH, NKVH, Da, r, False,
                                         io_name(dtype), gy)
        grads = [to_torch(gy[:, :NH], dtype, DEV), to_torch(gy[:, NH:NH + NKVH], dtype, DEV),
                 to_torch(gy[:, NH + NKVH:], dtype, DEV)]
        for stride in stride_layouts(c.shape):
            comb = strided_copy(c, stride, dtype, DEV)
            _, gc, gi, gb = _run(comb, to_torch(ini, dtype, DEV),
                                 to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, False,
                                 grads)
            case = f"T={T} r={r} stride={stride}"
            assert_close(np_of(gc), egc, 0, "grad_combined " + case)
            assert_close(np_of(gi), egi, 0, "grad_inits " + case)
            assert_close(np_of(gb), egb, 0, "grad_logit_bias " + case)


# head_dim 128 (every divisor r), plus head dims whose gate groups need the
# per-channel fallback; contiguous (B, T, F) and the projection's (B, F, T) view
WIDE_CASES = [(128, r) for r in (1, 2, 4, 8, 16, 32, 64, 128)] + [(12, 3), (12, 12), (24, 24),
                                                                  (40, 5)]
# gate groups of a non-power-of-two number of channel lanes (r / V = 3, 5, 6, 10, 12 with 8 bf16
# or 4 fp32 channels per lane), which straddle the wavefront's 16-lane rows
WIDE_CASES += [(48, 24), (40, 40), (120, 24), (96, 12), (96, 48)]


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("D,r", WIDE_CASES)
@pytest.mark.parametrize("T", [1, 33, 300])
def test_exact_wide_heads(dtype, D, r, T):
    B, NH, NKVH = 2, 2, 1
    Da = D // r
    H = NH + 2 * NKVH
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, False)
    rng = np.random.default_rng(D * 1000 + r + T)
    gy = rng.integers(-2, 3, size=(B, H, T, D)).astype(np.float32)
    (eq, ek, ev), (egc, egi, egb) = _expected(c, ini, bias, NH, NKVH, Da, r, False,
                                              io_name(dtype), gy)
    grads = [to_torch(gy[:, :NH], dtype, DEV), to_torch(gy[:, NH:NH + NKVH], dtype, DEV),
             to_torch(gy[:, NH + NKVH:], dtype, DEV)]
    F = c.shape[2]
    for layout in ("btf", "bft"):
        if layout == "btf":
            comb = to_torch(c, dtype, DEV)
        else:  # (B, F, T) contiguous seen as (B, T, F): the reference's projection output
            comb = to_torch(np.ascontiguousarray(c.transpose(0, 2, 1)), dtype, DEV).transpose(1, 2)
        (q, k, v), gc, gi, gb = _run(comb, to_torch(ini, dtype, DEV),
                                     to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, False,
                                     grads)
        case = f"D={D} r={r} T={T} {layout}"
        assert_close(np_of(q), eq, 0, "q " + case)
        assert_close(np_of(k), ek, 0, "k " + case)
        assert_close(np_of(v), ev, 0, "v " + case)
        assert_close(np_of(gc), egc, 0, "grad_combined " + case)
        assert_close(np_of(gi), egi, 0, "grad_inits " + case)
        # dbias sums B*T integer terms that can exceed 2**24: fp32 order matters
        assert_close(np_of(gb), egb, 1e-6, "grad_logit_bias " + case)
        assert F == gc.shape[2]


# ---------------------------------------------------------------------------
# sigmoid: golden vectors from the reference, random inputs, long sequences
# ---------------------------------------------------------------------------
GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "scan_*.npz")))


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_golden_vectors(path):
    z = np.load(path)
    B, T, NH, NKVH, Da, r, isbf = (int(v) for v in z["meta"])
    dtype = torch.bfloat16 if isbf else torch.float32
    cv = O.bf16_from_bits if isbf else (lambda a: np.asarray(a, np.float32))
    grads = [to_torch(cv(z[k]), dtype, DEV) for k in ("grad_q", "grad_k", "grad_v")]
    (q, k, v), gc, gi, gb = _run(to_torch(cv(z["combined"]), dtype, DEV),
                                 to_torch(cv(z["inits"]), dtype, DEV),
                                 to_torch(z["logit_bias"], torch.float32, DEV), NH, NKVH, Da, r,
                                 True, grads)
    tol = TOL[dtype]
    assert_close(np_of(q), cv(z["out_q"]), tol, "q")
    assert_close(np_of(k), cv(z["out_k"]), tol, "k")
    assert_close(np_of(v), cv(z["out_v"]), tol, "v")
    assert_close(np_of(gc), cv(z["grad_combined"]), tol, "grad_combined")
    assert_close(np_of(gi), cv(z["grad_inits"]), tol, "grad_inits")
    assert_close(np_of(gb), z["grad_logit_bias"], tol, "grad_logit_bias")


def _random_case(B, T, NH, NKVH, Da, r, seed, z_mean=2.0, z_std=1.0, io="f32"):
    rng = np.random.default_rng(seed)
    H, D = NH + 2 * NKVH, Da * r
    c = rng.standard_normal((B, T, H, D + Da)).astype(np.float32)
    # decay a = 1 - alpha = sigmoid(z), z ~ N(z_mean, z_std)  =>  logit = -z
    c[..., D:] = -(z_mean + z_std * rng.standard_normal((B, T, H, Da)))
    c = O.round_io(c.reshape(B, T, -1), io)
    ini = O.round_io(rng.standard_normal((B, H, D)).astype(np.float32), io)
    bias = (0.1 * rng.standard_normal((H, Da))).astype(np.float32)
    gy = O.round_io(rng.standard_normal((B, H, T, D)).astype(np.float32), io)
    return c, ini, bias, gy


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("B,T,NH,NKVH,Da,r", [
    (2, 1000, 1, 1, 1, 128),   # head-shared gate (d12's r)
    (2, 1000, 1, 1, 128, 1),   # per-channel decay
    (1, 5000, 1, 1, 2, 64),    # many tiles: carries across the workgroup's T loop
    (3, 77, 2, 1, 4, 8),
])
def test_sigmoid_random(dtype, B, T, NH, NKVH, Da, r):
    io = io_name(dtype)
    H = NH + 2 * NKVH
    c, ini, bias, gy = _random_case(B, T, NH, NKVH, Da, r, seed=T + r, io=io)
    (eq, ek, ev), (egc, egi, egb) = _expected(c, ini, bias, NH, NKVH, Da, r, True, io, gy)
    grads = [to_torch(gy[:, :NH], dtype, DEV), to_torch(gy[:, NH:NH + NKVH], dtype, DEV),
             to_torch(gy[:, NH + NKVH:H], dtype, DEV)]
    (q, k, v), gc, gi, gb = _run(to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                                 to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, True,
                                 grads)
    tol = TOL[dtype]
    assert_close(np_of(q), eq, tol, "q")
    assert_close(np_of(k), ek, tol, "k")
    assert_close(np_of(v), ev, tol, "v")
    assert_close(np_of(gc), egc, tol, "grad_combined")
    assert_close(np_of(gi), egi, tol, "grad_inits")
    assert_close(np_of(gb), egb, tol, "grad_logit_bias")


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
def test_long_sequence_long_memory(dtype):
    """Config 5's regime: T = 8192 with gate logits -z, z ~ N(3, 1.5) (decay
    a = 1 - alpha around 0.95, so states carry over hundreds of steps).  Few
    (b, h) sequences, so the op's backward runs chained (one tile-long chunk
    per workgroup, the carries handed between them); its tile kernels with the
    chunk-map carries are compared with it in test_scan_chain_gpu.py."""
    io = io_name(dtype)
    B, T, NH, NKVH, Da, r = 1, 8192, 1, 1, 1, 128
    H = NH + 2 * NKVH
    c, ini, bias, gy = _random_case(B, T, NH, NKVH, Da, r, seed=8192, z_mean=3.0, z_std=1.5,
                                    io=io)
    bias[:] = 0.0
    (eq, ek, ev), (egc, egi, egb) = _expected(c, ini, bias, NH, NKVH, Da, r, True, io, gy)
    grads = [to_torch(gy[:, :NH], dtype, DEV), to_torch(gy[:, NH:NH + NKVH], dtype, DEV),
             to_torch(gy[:, NH + NKVH:H], dtype, DEV)]
    (q, k, v), gc, gi, gb = _run(to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                                 to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, True,
                                 grads)
    tol = TOL[dtype]
    assert_close(np_of(q), eq, tol, "q")
    assert_close(np_of(v), ev, tol, "v")
    assert_close(np_of(gc), egc, tol, "grad_combined")
    assert_close(np_of(gi), egi, tol, "grad_inits")
    assert_close(np_of(gb), egb, tol, "grad_logit_bias")


def test_backward_is_deterministic():
    B, T, NH, NKVH, Da, r = 2, 700, 2, 1, 1, 128
    c, ini, bias, gy = _random_case(B, T, NH, NKVH, Da, r, seed=5, io="bf16")
    dtype = torch.bfloat16
    H = NH + 2 * NKVH
    grads = [to_torch(gy[:, :NH], dtype, DEV), to_torch(gy[:, NH:NH + NKVH], dtype, DEV),
             to_torch(gy[:, NH + NKVH:H], dtype, DEV)]
    runs = [_run(to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                 to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, True, grads)
            for _ in range(2)]
    for a, b in zip(runs[0][1:], runs[1][1:]):
        assert torch.equal(a, b)


def test_rejects_unsupported_tuning_values():
    op = _op()
    c = torch.zeros(1, 2, 3 * (2 + 1), device=DEV)
    ini = torch.zeros(1, 3, 2, device=DEV)
    bias = torch.zeros(3, 1, device=DEV)
    with pytest.raises(RuntimeError, match="Unsupported scan_threads"):
        op(c, ini, bias, 1, 1, 1, 2, 7, 8, 4, 32, 2, 8, True)
    with pytest.raises(RuntimeError, match="Unsupported r_items"):
        op(c, ini, bias, 1, 1, 1, 2, 8, 8, 3, 32, 2, 8, True)


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
def test_backward_empty_time_zeroes_grads(dtype):
    """T == 0: no step reads the inits or the bias, so both gradients are zero
    (as the oracle and the reference's autograd give); the kernel must write
    them, whatever the caller's buffers held, also through strided views."""
    import nanochat_amd.ops  # noqa: F401
    kern = torch.ops.nanochat_cuda.ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward_kernel
    B, NH, NKVH, Da, r = 3, 2, 1, 2, 4
    H, D = NH + 2 * NKVH, Da * r
    c = torch.zeros(B, 0, H * (D + Da), device=DEV, dtype=dtype)
    ini = torch.randn(B, H, D, device=DEV).to(dtype)
    bias = torch.randn(H, Da, device=DEV)
    hq = torch.zeros(B, NH, 0, D, device=DEV, dtype=dtype)
    hk = torch.zeros(B, NKVH, 0, D, device=DEV, dtype=dtype)
    hv = torch.zeros(B, NKVH, 0, D, device=DEV, dtype=dtype)
    gc = torch.zeros_like(c)
    # grad_inits as a (B, H, D) view with a gap between heads
    gi_store = torch.full((B, H, D + 3), float("nan"), device=DEV, dtype=dtype)
    gi = gi_store[:, :, :D]
    gb = torch.full((H, Da), float("nan"), device=DEV)
    kern(c, ini, bias, hq, hk, hv, hq, hk, hv, gc, gi, gb, NH, NKVH, Da, r, 32, 2, 8, True)
    torch.cuda.synchronize()
    assert torch.equal(gi.float().cpu(), torch.zeros(B, H, D))
    assert torch.equal(gb.cpu(), torch.zeros(H, Da))
    # the gap columns are not part of the view and stay untouched
    assert torch.isnan(gi_store[:, :, D:].float()).all()
    # the oracle agrees: empty T gives zero gradients
    eg = O.scan_backward(np.zeros((B, 0, H * (D + Da)), np.float32), np.ones((B, H, D), np.float32),
                         np.zeros((H, Da), np.float32),
                         np.zeros((B, NH, 0, D), np.float32), np.zeros((B, NKVH, 0, D), np.float32),
                         np.zeros((B, NKVH, 0, D), np.float32),
                         np.zeros((B, NH, 0, D), np.float32), np.zeros((B, NKVH, 0, D), np.float32),
                         np.zeros((B, NKVH, 0, D), np.float32), NH, NKVH, Da, r, True, "f32")
    assert not np.any(eg[1]) and not np.any(eg[2])


# ---------------------------------------------------------------------------
# long sequences at small batch (configs[4] prefill)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("D,r", [(128, 128), (128, 1), (64, 16)])
def test_forward_long_exact(dtype, D, r):
    """The reference's integer generators (gates 0 / 1, sigmoid off) at T =
    2000 with one sequence slab: hundreds of tiles walked by one workgroup
    (the few-workgroup launch shape), every output exact."""
    B, T, NH, NKVH = 1, 2000, 1, 0
    Da = D // r
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, False)
    eq, ek, ev = _expected(c, ini, bias, NH, NKVH, Da, r, False, io_name(dtype))
    q, k, v = _run(to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                   to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, False)
    assert_close(np_of(q), eq, 0, f"q D={D} r={r}")


def test_forward_config5_prefill():
    """configs[4]'s prefill shape (B = 8, T = 8192, 18 heads of 128, r = 128,
    bf16, decay sigmoid(z), z ~ N(3, 1.5)) through the fast path's scan: two
    batch rows (all heads) against the oracle within the bf16 tolerance, and
    two runs bitwise equal."""
    from nanochat_amd.ops import ltv_hm_fast as F_
    B, T, NH, NKVH, D = 8, 8192, 6, 6, 128
    H = NH + 2 * NKVH
    g = torch.Generator().manual_seed(5)
    values = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    logits = (-(3.0 + 1.5 * torch.randn(B, T, H, generator=g))).to(torch.bfloat16)
    inits = (0.5 * torch.randn(B, H, D, generator=g)).to(torch.bfloat16)
    bias = torch.zeros(H, 1)
    vd, ld, idv, bd = values.to(DEV), logits.to(DEV), inits.to(DEV), bias.to(DEV)
    outs = F_.scan_forward(vd, ld, idv, bd, NH, NKVH, 1, D, True)
    outs2 = F_.scan_forward(vd, ld, idv, bd, NH, NKVH, 1, D, True)
    for a, b in zip(outs, outs2):
        assert torch.equal(a, b)
    got = torch.cat(outs, dim=1)  # (B, H, T, D)
    for b in (0, 7):
        # the oracle's (B, T, F) layout: per head [values D | logit]
        comb = torch.cat([values[b].permute(1, 0, 2), logits[b].unsqueeze(-1)], dim=-1)
        comb = comb.reshape(1, T, H * (D + 1)).float().numpy()
        eq, ek, ev = O.scan_forward(comb, inits[b:b + 1].float().numpy(), bias.numpy(), NH, NKVH,
                                    1, D, True, "bf16")
        want = np.concatenate([eq, ek, ev], axis=1)[0]
        assert_close(np_of(got[b]), want, 2e-2, f"config5 prefill b={b}")
