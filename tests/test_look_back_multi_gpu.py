"""GPU parity of the short-window look-back backward with several windows per
lane (``ltv_lb_set_windows_per_lane``): a lane walks consecutive windows last
to first and hands each window's chain value and warm-up states to the window
before it instead of recomputing them from memory.

Checked bitwise against one window per lane (the same operations in the same
order) for every gate mode the kernel is built for, window counts that are and
are not multiples of the windows per lane, and layer specs it does not take
(which must fall back unchanged); exactly against the oracle on the integer
generators; and the automatic choice at the d12 shape
(``test_look_back_gpu.py::test_d12_windows_match_full_recurrence_per_window``
runs that one against the full-recurrence kernels).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import int_combined, int_inits, int_logit_bias, io_name, np_of, to_torch
from test_look_back_gpu import _check, _expected, _grads, _run

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture
def wpl():
    """Sets the windows per lane for the launches that follow; back to
    automatic afterwards."""
    from nanochat_amd import _native as N
    lib = N.lib()

    def set_(n):
        N.check(lib.ltv_lb_set_windows_per_lane(n), "ltv_lb_set_windows_per_lane")

    try:
        yield set_
    finally:
        set_(0)


def _random_case(B, T, NH, NKVH, D, r, dtype, seed):
    Da = D // r
    H = NH + 2 * NKVH
    rng = np.random.default_rng(seed)
    io = io_name(dtype)
    c = O.round_io(rng.standard_normal((B, T, H * (D + Da))).astype(np.float32), io)
    ini = O.round_io(rng.standard_normal((B, H, D)).astype(np.float32), io)
    bias = (rng.standard_normal((H, Da)) * 0.5).astype(np.float32)
    gy = O.round_io(rng.standard_normal((B, H, T, D)).astype(np.float32), io)
    return c, ini, bias, gy


def _go(c, ini, bias, gy, NH, NKVH, Da, r, pqk, sig, dtype):
    return _run("blelloch", to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, pqk, sig,
                _grads(gy, NH, NKVH, dtype))


def _assert_bitwise(a, b, case):
    (qa, ka, va), gca, gia, gba = a
    (qb, kb, vb), gcb, gib, gbb = b
    for name, x, y in (("q", qa, qb), ("k", ka, kb), ("v", va, vb), ("grad_combined", gca, gcb),
                       ("grad_inits", gia, gib), ("grad_logit_bias", gba, gbb)):
        assert torch.equal(x, y), f"{name} differs: {case}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=io_name)
@pytest.mark.parametrize("D,r", [(128, 128), (128, 16), (128, 1), (64, 64)])
@pytest.mark.parametrize("pqk", [(16, 16, 9), (64, 60, 5), (20, 12, 9), (5, 2, 6)], ids=str)
def test_windows_per_lane_bitwise_equals_one(wpl, dtype, D, r, pqk):
    """T = 300: 19 windows at (16, 16, 9), 5 at (64, 60, 5), 25 at (20, 12, 9);
    (5, 2, 6) has warm-ups longer than Q and keeps one window per lane.  Every
    windows-per-lane value gives bitwise the one-window results."""
    B, NH, NKVH, T = 2, 2, 1, 300
    Da = D // r
    c, ini, bias, gy = _random_case(B, T, NH, NKVH, D, r, dtype, seed=D * 3 + r + pqk[0])
    wpl(1)
    ref = _go(c, ini, bias, gy, NH, NKVH, Da, r, pqk, True, dtype)
    for n in (2, 3, 5, 64):
        wpl(n)
        got = _go(c, ini, bias, gy, NH, NKVH, Da, r, pqk, True, dtype)
        _assert_bitwise(got, ref, f"wpl={n} D={D} r={r} pqk={pqk}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=io_name)
@pytest.mark.parametrize("pqk", [(16, 16, 9), (8, 6, 4), (4, 4, 1), (0, 3, 2)], ids=str)
@pytest.mark.parametrize("T", [31, 33, 100])
def test_windows_per_lane_exact_integer(wpl, dtype, pqk, T):
    """The integer generators without the sigmoid: exact against the oracle
    with three windows per lane (a last group of fewer windows at most T)."""
    B, NH, NKVH, total_d = 4, 8, 8, 16
    H = NH + 2 * NKVH
    for r in (8, 16):
        Da = total_d // r
        c = int_combined(B, T, NH, NKVH, Da, r)
        ini = int_inits(B, NH, NKVH, Da, r)
        bias = int_logit_bias(NH, NKVH, Da, False)
        gy = np.random.default_rng(T + r).integers(-2, 3, size=(B, H, T, total_d)).astype(
            np.float32)
        want = _expected(c, ini, bias, NH, NKVH, Da, r, pqk, False, io_name(dtype), gy)
        wpl(3)
        got = _go(c, ini, bias, gy, NH, NKVH, Da, r, pqk, False, dtype)
        _check(got, want, 0, f"wpl=3 T={T} r={r} pqk={pqk}")


def test_windows_per_lane_d12_layer_spec_bitwise():
    """The d12 layer spec at B = 8, T = 1024 (64 windows per sequence): the
    automatic choice, 4 and 7 windows per lane all equal one per lane."""
    from nanochat_amd import _native as N
    lib = N.lib()
    B, T, NH, NKVH, D, r = 8, 1024, 6, 6, 128, 128
    Da = 1
    c, ini, bias, gy = _random_case(B, T, NH, NKVH, D, r, torch.bfloat16, seed=12)
    try:
        N.check(lib.ltv_lb_set_windows_per_lane(1), "wpl")
        ref = _go(c, ini, bias, gy, NH, NKVH, Da, r, (16, 16, 9), True, torch.bfloat16)
        for n in (0, 4, 7):
            N.check(lib.ltv_lb_set_windows_per_lane(n), "wpl")
            got = _go(c, ini, bias, gy, NH, NKVH, Da, r, (16, 16, 9), True, torch.bfloat16)
            _assert_bitwise(got, ref, f"wpl={n}")
    finally:
        lib.ltv_lb_set_windows_per_lane(0)
