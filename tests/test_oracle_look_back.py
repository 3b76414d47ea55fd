"""Pins the look-back part of the CPU oracle (``look_back_forward/backward``).

The look-back scan (``ltv_reference_ops.py:37-124`` with general P, Q, K) runs
each chunk window from the inits over a K - 1 step warm-up.  Checks, each able
to catch a plausible mistake in the window arithmetic or the gradient sums:

* golden vectors written by the reference's own look-back function
  (``tests/golden/make_golden.py``): several windows, warm-ups longer than Q,
  an empty first chunk (P = 0), fp32 and bf16 with the sigmoid on;
* P >= T reduces both to the full-recurrence scan (already pinned);
* with the reference generators and no sigmoid the gates are 0/1, and every
  window is a sample-and-hold whose forward and backward have the closed forms
  of test_oracle.py; the windows are embedded and summed here by index
  arithmetic;
* float64 central finite differences over overlapping windows, with a planted
  mistake (dropping the warm-up contributions, as the reference's CUDA
  backward does for multi-chunk inputs) that the check must catch.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest

import ltv_oracle as O
from ltv_test_utils import int_combined, int_inits, int_logit_bias
from test_oracle import _hold_backward, _hold_forward

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "look_back_*.npz")))


def _load(path):
    z = np.load(path)  # allow_pickle stays False
    B, T, NH, NKVH, Da, r, isbf, P, Q, K = (int(v) for v in z["meta"])
    cv = O.bf16_from_bits if isbf else (lambda a: np.asarray(a, np.float32))
    return dict(B=B, T=T, NH=NH, NKVH=NKVH, Da=Da, r=r, P=P, Q=Q, K=K,
                io="bf16" if isbf else "f32", get=lambda k: cv(z[k]),
                bias=np.asarray(z["logit_bias"], np.float32),
                gbias=np.asarray(z["grad_logit_bias"], np.float32))


def _coverage(T, P, Q, K):
    """Number of windows whose range [lo, hi) contains each step."""
    cov = np.zeros(T, np.int64)
    for lo, st, hi in O.look_back_windows(T, P, Q, K):
        cov[lo:hi] += 1
    return cov


def test_look_back_golden_fixtures_present():
    assert len(GOLDEN) >= 5


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_look_back_oracle_matches_reference_golden(path):
    g = _load(path)
    get = g["get"]
    pqk = (g["P"], g["Q"], g["K"])
    args = (g["NH"], g["NKVH"], g["Da"], g["r"], *pqk, True, g["io"])
    assert len(O.look_back_windows(g["T"], *pqk)) >= 3  # several chunk windows
    oq, ok, ov = O.look_back_forward(get("combined"), get("inits"), g["bias"], *args)
    gc, gi, gb = O.look_back_backward(get("combined"), get("inits"), g["bias"], get("grad_q"),
                                      get("grad_k"), get("grad_v"), *args)
    single = _coverage(g["T"], *pqk) == 1  # steps that only one window reads
    if g["io"] == "bf16":
        # same fp32 ops per window: the forward agrees bit for bit
        for a, k in ((oq, "out_q"), (ok, "out_k"), (ov, "out_v")):
            np.testing.assert_array_equal(a, get(k), err_msg=k)
        # a step read by one window has one gradient contribution: bit-exact;
        # where windows overlap the reference adds bf16-rounded contributions
        # while the oracle adds in fp32 and rounds once: the sums differ by
        # a few roundings of the contributions (a bf16 ulp of the largest)
        ref = get("grad_combined")
        np.testing.assert_array_equal(gc[:, single], ref[:, single])
        np.testing.assert_allclose(gc, ref, rtol=0, atol=2 ** -7 * np.abs(ref).max())
        gref = get("grad_inits")
        np.testing.assert_allclose(gi, gref, rtol=0, atol=2 ** -7 * np.abs(gref).max())
    else:
        for a, k in ((oq, "out_q"), (ok, "out_k"), (ov, "out_v"), (gc, "grad_combined"),
                     (gi, "grad_inits")):
            np.testing.assert_allclose(a, get(k), rtol=1e-5, atol=1e-6, err_msg=k)
    np.testing.assert_allclose(gb, g["gbias"], rtol=1e-4, atol=1e-4)


def test_look_back_windows_bounds():
    # first chunk [0, P), then chunks of Q, each warmed up over K - 1 steps
    assert O.look_back_windows(20, 8, 5, 3) == [(0, 0, 8), (6, 8, 13), (11, 13, 18),
                                               (16, 18, 20)]
    assert O.look_back_windows(7, 8, 5, 3) == [(0, 0, 7)]
    assert O.look_back_windows(7, O.UNBOUNDED_P, 1, 1) == [(0, 0, 7)]
    assert O.look_back_windows(5, 0, 2, 4) == [(0, 0, 0), (0, 0, 2), (0, 2, 4), (1, 4, 5)]
    assert O.look_back_windows(0, 3, 2, 2) == [(0, 0, 0)]


@pytest.mark.parametrize("io", ["f32", "bf16"])
def test_look_back_reduces_to_full_scan_when_p_covers_t(io):
    rng = np.random.default_rng(4)
    B, T, NH, NKVH, Da, r = 2, 17, 1, 1, 2, 4
    H, D = NH + 2 * NKVH, Da * r
    c = O.round_io(rng.standard_normal((B, T, H * (D + Da))), io)
    ini = O.round_io(rng.standard_normal((B, H, D)), io)
    bias = (rng.standard_normal((H, Da)) * 0.5).astype(np.float32)
    gy = O.round_io(rng.standard_normal((B, H, T, D)), io)
    gq, gk, gv = gy[:, :NH], gy[:, NH:NH + NKVH], gy[:, NH + NKVH:]
    full = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, True, io)
    fb = O.scan_backward(c, ini, bias, *full, gq, gk, gv, NH, NKVH, Da, r, True, io)
    for P, Q, K in ((O.UNBOUNDED_P, 1, 1), (T, 3, 5), (1024, 1024, 1)):
        lb = O.look_back_forward(c, ini, bias, NH, NKVH, Da, r, P, Q, K, True, io)
        for a, b in zip(lb, full):
            np.testing.assert_array_equal(a, b)
        lbb = O.look_back_backward(c, ini, bias, gq, gk, gv, NH, NKVH, Da, r, P, Q, K, True, io)
        for a, b in zip(lbb, fb):
            np.testing.assert_array_equal(a, b)


def _hold_look_back(c, ini, gy, NH, NKVH, Da, r, P, Q, K):
    """Closed form: each window is a sample-and-hold from the inits; the
    gradients are the windows' closed-form gradients embedded at [lo, hi)."""
    B, T, F = c.shape
    H, D = NH + 2 * NKVH, Da * r
    out = np.zeros((B, H, T, D))
    gc = np.zeros((B, T, F))
    gi = np.zeros((B, H, D))
    gb = np.zeros((H, Da))
    for lo, st, hi in O.look_back_windows(T, P, Q, K):
        if hi <= lo:
            continue
        out[:, :, st:hi] = _hold_forward(c[:, lo:hi], ini, NH, NKVH, Da, r)[:, :, st - lo:]
        g = gy[:, :, lo:hi].copy()
        g[:, :, : st - lo] = 0.0  # no upstream gradient on the warm-up steps
        wgc, wgi, wgb = _hold_backward(c[:, lo:hi], ini, g, NH, NKVH, Da, r)
        gc[:, lo:hi] += wgc
        gi += wgi
        gb += wgb
    return out, gc, gi, gb


@pytest.mark.parametrize("T", [1, 2, 3, 31, 32, 33])
@pytest.mark.parametrize("pqk", [(8, 6, 4), (5, 2, 6), (4, 4, 1), (0, 3, 2)])
@pytest.mark.parametrize("Da,r", [(2, 1), (1, 2)])
def test_look_back_hold_closed_form(T, pqk, Da, r):
    B, NH, NKVH = 3, 2, 1
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, sigmoid=False)
    H = NH + 2 * NKVH
    rng = np.random.default_rng(T * 11 + pqk[0])
    gy = rng.integers(-3, 4, size=(B, H, T, Da * r)).astype(np.float32)
    out, egc, egi, egb = _hold_look_back(c, ini, gy, NH, NKVH, Da, r, *pqk)
    args = (NH, NKVH, Da, r, *pqk, False, "f32")
    oq, ok, ov = O.look_back_forward(c, ini, bias, *args)
    np.testing.assert_array_equal(np.concatenate([oq, ok, ov], axis=1), out)
    gc, gi, gb = O.look_back_backward(c, ini, bias, gy[:, :NH], gy[:, NH:NH + NKVH],
                                      gy[:, NH + NKVH:], *args)
    np.testing.assert_array_equal(gc, egc)
    np.testing.assert_array_equal(gi, egi)
    np.testing.assert_array_equal(gb, egb)


def _fd_case():
    rng = np.random.default_rng(5)
    B, T, NH, NKVH, Da, r = 1, 11, 1, 1, 2, 2
    H, D = NH + 2 * NKVH, Da * r
    c = rng.standard_normal((B, T, H * (D + Da)))
    ini = rng.standard_normal((B, H, D))
    bias = rng.standard_normal((H, Da)) * 0.5
    w = rng.standard_normal((B, H, T, D))  # loss = sum(w * out)
    return c, ini, bias, w, (NH, NKVH, Da, r)


def _fd_mismatches(gc, gi, gb, c, ini, bias, w, shape_args, pqk):
    NH, NKVH, Da, r = shape_args

    def loss(c_, ini_, bias_):
        o = O.look_back_forward(c_, ini_, bias_, NH, NKVH, Da, r, *pqk, True, "f64")
        return float((np.concatenate(o, axis=1) * w).sum())

    eps = 1e-6
    bad = []
    for name, arr, grad, fn in (("combined", c, gc, lambda x: loss(x, ini, bias)),
                                ("inits", ini, gi, lambda x: loss(c, x, bias)),
                                ("bias", bias, gb, lambda x: loss(c, ini, x))):
        for idx in np.ndindex(arr.shape):
            p, m = arr.copy(), arr.copy()
            p[idx] += eps
            m[idx] -= eps
            num = (fn(p) - fn(m)) / (2 * eps)
            if abs(num - grad[idx]) > 1e-6 * (1 + abs(num)):
                bad.append((name, idx, num, grad[idx]))
    return bad


@pytest.mark.parametrize("pqk", [(4, 3, 3), (3, 2, 5), (0, 4, 2)])
def test_look_back_backward_matches_finite_differences(pqk):
    c, ini, bias, w, sa = _fd_case()
    NH, NKVH = sa[0], sa[1]
    gc, gi, gb = O.look_back_backward(c, ini, bias, w[:, :NH], w[:, NH:NH + NKVH],
                                      w[:, NH + NKVH:], *sa, *pqk, True, "f64")
    assert _fd_mismatches(gc, gi, gb, c, ini, bias, w, sa, pqk) == []


def test_finite_differences_catch_dropped_warm_up_gradients(monkeypatch):
    """A backward that ignores the warm-up steps' contributions (every window
    differentiated as if it started at its first own step) must fail."""
    c, ini, bias, w, sa = _fd_case()
    NH, NKVH = sa[0], sa[1]
    pqk = (4, 3, 3)
    real = O.look_back_windows
    monkeypatch.setattr(O, "look_back_windows",
                        lambda T, P, Q, K: [(st, st, hi) for _, st, hi in real(T, P, Q, K)])
    gc, gi, gb = O.look_back_backward(c, ini, bias, w[:, :NH], w[:, NH:NH + NKVH],
                                      w[:, NH + NKVH:], *sa, *pqk, True, "f64")
    monkeypatch.setattr(O, "look_back_windows", real)
    assert _fd_mismatches(gc, gi, gb, c, ini, bias, w, sa, pqk) != []
