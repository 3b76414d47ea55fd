"""GPU parity of the look-back scan (chunk restarts with a K - 1 step warm-up)
against the CPU oracle, through the reference-layout ops, the fused filter path
and the KV-cache module layer.

Mirrors the reference's
tests/test_ltv_cuda_look_back_fused_concat_head_major_register_cast_{blelloch,sequential}_scan.py
(forward/backward over SUPPORTED_PQK_CONFIGS, T in {1, 2, 3, 31, 32, 33},
every stride layout, integer generators without the sigmoid: exact) and adds
what those never reach -- several chunk windows (T > P), warm-ups longer than
Q, an empty first chunk -- plus sigmoid cases against the oracle and the
reference's golden vectors, and a d12-size run checked window by window
against the full-recurrence kernels.
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
UNB = O.UNBOUNDED_P
# the reference's SUPPORTED_PQK_CONFIGS (tests/ltv_scan_test_utils.py:11-19)
REF_PQK = [(UNB, 1, 1), (1024, 1024, 1), (64, 60, 5), (128, 112, 17), (160, 108, 53),
           (192, 104, 89), (224, 100, 125)]
# several windows at small T: warm-up < Q, warm-up > Q, empty first chunk, d12 layer spec
MULTI_PQK = [(8, 6, 4), (5, 2, 6), (0, 3, 2), (16, 16, 9), (4, 4, 1)]


def _ops():
    import nanochat_amd.ops  # noqa: F401
    return (torch.ops.nanochat_cuda.ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_cuda_op,
            torch.ops.nanochat_cuda.ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_cuda_op)


def _run(variant, combined, inits, bias, NH, NKVH, Da, r, pqk, sig, grads=None):
    blelloch, sequential = _ops()

    def call(c, i, b):
        if variant == "blelloch":
            return blelloch(c, i, b, NH, NKVH, Da, r, *pqk, 8, 8, 4, 32, 2, 8, sig)
        return sequential(c, i, b, NH, NKVH, Da, r, *pqk, 8, 4, 2, 8, sig)

    if grads is None:
        with torch.no_grad():
            return call(combined, inits, bias)
    combined = combined.detach().requires_grad_(True)
    inits = inits.detach().requires_grad_(True)
    bias = bias.detach().requires_grad_(True)
    outs = call(combined, inits, bias)
    torch.autograd.backward(outs, grads)
    return outs, combined.grad, inits.grad, bias.grad


def _expected(c, ini, bias, NH, NKVH, Da, r, pqk, sig, io, gy):
    outs = O.look_back_forward(c, ini, bias, NH, NKVH, Da, r, *pqk, sig, io)
    H = NH + 2 * NKVH
    g = O.look_back_backward(c, ini, bias, gy[:, :NH], gy[:, NH:NH + NKVH], gy[:, NH + NKVH:H],
                             NH, NKVH, Da, r, *pqk, sig, io)
    return outs, g


def _grads(gy, NH, NKVH, dtype):
    return [to_torch(gy[:, :NH], dtype, DEV), to_torch(gy[:, NH:NH + NKVH], dtype, DEV),
            to_torch(gy[:, NH + NKVH:], dtype, DEV)]


def _check(got, want, tol, case):
    (q, k, v), gc, gi, gb = got
    (eq, ek, ev), (egc, egi, egb) = want
    assert_close(np_of(q), eq, tol, "q " + case)
    assert_close(np_of(k), ek, tol, "k " + case)
    assert_close(np_of(v), ev, tol, "v " + case)
    assert_close(np_of(gc), egc, tol, "grad_combined " + case)
    assert_close(np_of(gi), egi, tol, "grad_inits " + case)
    assert_close(np_of(gb), egb, max(tol, 1e-6), "grad_logit_bias " + case)


# ---------------------------------------------------------------------------
# exact integer cases (sigmoid off): the reference harness and several windows
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("pqk", REF_PQK + MULTI_PQK, ids=str)
@pytest.mark.parametrize("T", [1, 2, 3, 31, 32, 33])
def test_exact_all_strides(dtype, pqk, T):
    B, NH, NKVH, total_d = 4, 8, 8, 2
    H = NH + 2 * NKVH
    for r in (1, 2):
        Da = total_d // r
        c = int_combined(B, T, NH, NKVH, Da, r)
        ini = int_inits(B, NH, NKVH, Da, r)
        bias = int_logit_bias(NH, NKVH, Da, False)
        rng = np.random.default_rng(T * 13 + r)
        gy = rng.integers(-2, 3, size=(B, H, T, total_d)).astype(np.float32)
        want = _expected(c, ini, bias, NH, NKVH, Da, r, pqk, False, io_name(dtype), gy)
        layouts = stride_layouts(c.shape)
        for i, stride in enumerate(layouts):
            variant = "blelloch" if i % 2 == 0 else "sequential"
            comb = strided_copy(c, stride, dtype, DEV)
            got = _run(variant, comb, to_torch(ini, dtype, DEV),
                       to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, pqk, False,
                       _grads(gy, NH, NKVH, dtype))
            _check(got, want, 0, f"{variant} T={T} r={r} pqk={pqk} stride={stride}")


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("D,r", [(128, 128), (128, 16), (128, 8), (128, 1), (64, 4), (32, 32),
                                 (48, 24), (40, 40), (120, 24)])
@pytest.mark.parametrize("pqk", [(64, 60, 5), (224, 100, 125), (16, 16, 9), (0, 48, 80)],
                         ids=str)
def test_exact_wide_heads_many_windows(dtype, D, r, pqk):
    B, NH, NKVH, T = 2, 2, 1, 300
    Da = D // r
    H = NH + 2 * NKVH
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, False)
    rng = np.random.default_rng(D + r)
    gy = rng.integers(-2, 3, size=(B, H, T, D)).astype(np.float32)
    want = _expected(c, ini, bias, NH, NKVH, Da, r, pqk, False, io_name(dtype), gy)
    for layout in ("btf", "bft"):
        if layout == "btf":
            comb = to_torch(c, dtype, DEV)
        else:  # the projection's (B, F, T) buffer seen as (B, T, F)
            comb = to_torch(np.ascontiguousarray(c.transpose(0, 2, 1)), dtype, DEV).transpose(1, 2)
        got = _run("blelloch", comb, to_torch(ini, dtype, DEV),
                   to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, pqk, False,
                   _grads(gy, NH, NKVH, dtype))
        _check(got, want, 0, f"D={D} r={r} pqk={pqk} {layout}")


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("D,r", [(12, 3), (24, 6), (40, 5), (96, 4), (36, 12)])
@pytest.mark.parametrize("pqk", [(8, 6, 4), (0, 5, 9), (64, 60, 5)], ids=str)
def test_exact_gate_groups_outside_the_tile_patterns(dtype, D, r, pqk):
    """Several windows with gate groups neither filling whole lanes nor fitting
    in one (r = 3, 5, 6, 12 against 8 bf16 / 4 fp32 channels per lane) or more
    than 16 per head (D = 96, r = 4): the per-channel look-back backward
    (warm-ups in fp32 sums across windows), exact on the integer inputs, with
    the full-recurrence kernels for one window."""
    B, T, NH, NKVH = 2, 70, 1, 1
    Da = D // r
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, False)
    rng = np.random.default_rng(D + r)
    gy = rng.integers(-2, 3, size=(B, NH + 2 * NKVH, T, D)).astype(np.float32)
    for spec in (pqk, (T, 6, 4)):
        got = _run("blelloch", to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                   to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, spec, False,
                   _grads(gy, NH, NKVH, dtype))
        want = _expected(c, ini, bias, NH, NKVH, Da, r, spec, False, io_name(dtype), gy)
        _check(got, want, 0, f"D={D} r={r} pqk={spec}")


# ---------------------------------------------------------------------------
# sigmoid on: golden vectors of the reference and random inputs
# ---------------------------------------------------------------------------
GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "look_back_*.npz")))


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_golden_vectors(path):
    z = np.load(path)
    B, T, NH, NKVH, Da, r, isbf, P, Q, K = (int(v) for v in z["meta"])
    dtype = torch.bfloat16 if isbf else torch.float32
    cv = O.bf16_from_bits if isbf else (lambda a: np.asarray(a, np.float32))
    grads = [to_torch(cv(z[k]), dtype, DEV) for k in ("grad_q", "grad_k", "grad_v")]
    got = _run("blelloch", to_torch(cv(z["combined"]), dtype, DEV),
               to_torch(cv(z["inits"]), dtype, DEV),
               to_torch(np.asarray(z["logit_bias"], np.float32), torch.float32, DEV),
               NH, NKVH, Da, r, (P, Q, K), True, grads)
    want = ((cv(z["out_q"]), cv(z["out_k"]), cv(z["out_v"])),
            (cv(z["grad_combined"]), cv(z["grad_inits"]),
             np.asarray(z["grad_logit_bias"], np.float32)))
    _check(got, want, TOL[dtype], os.path.basename(path))


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("D,r", [(128, 128), (128, 16), (128, 1)])
@pytest.mark.parametrize("pqk", [(16, 16, 9), (64, 60, 5), (5, 2, 6), (128, 112, 17)], ids=str)
def test_sigmoid_random(dtype, D, r, pqk):
    B, NH, NKVH, T = 2, 2, 1, 257
    Da = D // r
    H = NH + 2 * NKVH
    rng = np.random.default_rng(D * 7 + r + pqk[0])
    io = io_name(dtype)
    c = O.round_io(rng.standard_normal((B, T, H * (D + Da))).astype(np.float32), io)
    ini = O.round_io(rng.standard_normal((B, H, D)).astype(np.float32), io)
    bias = (rng.standard_normal((H, Da)) * 0.5).astype(np.float32)
    gy = O.round_io(rng.standard_normal((B, H, T, D)).astype(np.float32), io)
    want = _expected(c, ini, bias, NH, NKVH, Da, r, pqk, True, io, gy)
    got = _run("sequential", to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
               to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, pqk, True,
               _grads(gy, NH, NKVH, dtype))
    _check(got, want, TOL[dtype], f"D={D} r={r} pqk={pqk}")


# ---------------------------------------------------------------------------
# d12 size, the layer spec (16, 16, 9): window by window against the
# full-recurrence kernels (each window is a full scan of its slice from the inits)
# ---------------------------------------------------------------------------
def test_d12_windows_match_full_recurrence_per_window():
    import nanochat_amd.ops  # noqa: F401
    full = torch.ops.nanochat_cuda.ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op
    B, T, NH, NKVH, D, r = 32, 1024, 6, 6, 128, 128
    P, Q, K = 16, 16, 9
    Da, H = D // r, NH + 2 * NKVH
    g = torch.Generator(device="cpu").manual_seed(0)
    bf = torch.bfloat16
    c = torch.randn(B, T, H * (D + Da), generator=g).to(bf).to(DEV)
    ini = torch.randn(B, H, D, generator=g).to(bf).to(DEV)
    bias = (torch.randn(H, Da, generator=g) * 0.5).to(DEV)
    gy = [torch.randn(B, nh, T, D, generator=g).to(bf).to(DEV) for nh in (NH, NKVH, NKVH)]
    (q, k, v), gc, gi, gb = _run("blelloch", c, ini, bias, NH, NKVH, Da, r, (P, Q, K), True, gy)
    out = torch.cat([q, k, v], dim=1).float()
    gy_all = torch.cat(gy, dim=1)
    e_out = torch.empty_like(out)
    e_gc = torch.zeros(c.shape, dtype=torch.float32, device=DEV)
    e_gi = torch.zeros(ini.shape, dtype=torch.float32, device=DEV)
    e_gb = torch.zeros(bias.shape, dtype=torch.float32, device=DEV)
    for lo, st, hi in O.look_back_windows(T, P, Q, K):
        cw = c[:, lo:hi].detach().clone().requires_grad_(True)
        iw = ini.detach().clone().requires_grad_(True)
        bw = bias.detach().clone().requires_grad_(True)
        wq, wk, wv = full(cw, iw, bw, NH, NKVH, Da, r, 8, 8, 4, 32, 2, 8, True)
        wo = torch.cat([wq, wk, wv], dim=1)
        e_out[:, :, st:hi] = wo[:, :, st - lo:].float()
        gw = torch.zeros_like(wo)
        gw[:, :, st - lo:] = gy_all[:, :, st:hi]
        torch.autograd.backward([wo], [gw])
        e_gc[:, lo:hi] += cw.grad.float()
        e_gi += iw.grad.float()
        e_gb += bw.grad
    tol = TOL[bf]
    assert_close(np_of(out), np_of(e_out), tol, "outputs")
    assert_close(np_of(gc), np_of(e_gc), tol, "grad_combined")
    assert_close(np_of(gi), np_of(e_gi), tol, "grad_inits")
    assert_close(np_of(gb), np_of(e_gb), 1e-3, "grad_logit_bias")


@pytest.mark.parametrize("pqk", [(128, 112, 17), (224, 100, 125)], ids=str)
def test_look_back_tile_backward_is_deterministic_per_channel_gates(pqk):
    """The look-back backward on the tile kernels with per-channel gates (r = 1,
    D = 128, bf16: 16 channel lanes, 4 steps per lane, 2 wavefronts; windows
    longer than the short-window kernels take): two runs bitwise equal, and
    within tolerance of the oracle.  This is the instantiation whose parity
    buffers once gave run-dependent gradients in a build with a wave-uniform
    wavefront index."""
    B, NH, NKVH, T, D, r = 2, 2, 1, 700, 128, 1
    Da = D // r
    H = NH + 2 * NKVH
    dtype = torch.bfloat16
    rng = np.random.default_rng(700 + pqk[0])
    c = O.round_io(rng.standard_normal((B, T, H * (D + Da))).astype(np.float32), "bf16")
    ini = O.round_io(rng.standard_normal((B, H, D)).astype(np.float32), "bf16")
    bias = (rng.standard_normal((H, Da)) * 0.5).astype(np.float32)
    gy = O.round_io(rng.standard_normal((B, H, T, D)).astype(np.float32), "bf16")
    runs = [_run("blelloch", to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                 to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, pqk, True,
                 _grads(gy, NH, NKVH, dtype)) for _ in range(3)]
    for other in runs[1:]:
        for a, b in zip(runs[0][1:], other[1:]):
            assert torch.equal(a, b)
    want = _expected(c, ini, bias, NH, NKVH, Da, r, pqk, True, "bf16", gy)
    _check(runs[0], want, TOL[dtype], f"pqk={pqk}")
