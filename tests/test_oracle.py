"""Pins the CPU oracle (oracle/ltv_oracle.py) before anything is compared to it.

Each check is chosen so that a plausible mistake in the oracle (a dropped term,
a wrong sign, an off-by-one in time, a transposed operand) fails it:

* golden vectors written by the reference's own ltv_reference_ops.py
  (tests/golden/make_golden.py) -- bf16 outputs and gradients bit-exact;
* the reference test generators without the sigmoid: gates are 0/1, so the
  scan is a sample-and-hold whose forward and backward have closed forms
  computed here by index arithmetic (a different route than the recurrence);
* constant alpha: geometric-series closed form;
* float64 central finite differences of the forward for every gradient;
* state continuity (splitting T and carrying the last row) and linearity;
* the projection against torch.matmul / autograd in float64.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import int_combined, int_inits, int_logit_bias

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "scan_*.npz")))


def _load_golden(path):
    z = np.load(path)  # allow_pickle stays False
    B, T, NH, NKVH, Da, r, isbf = (int(v) for v in z["meta"])
    cv = O.bf16_from_bits if isbf else (lambda a: np.asarray(a, np.float32))
    get = lambda k: cv(z[k])  # noqa: E731
    return dict(B=B, T=T, NH=NH, NKVH=NKVH, Da=Da, r=r, io="bf16" if isbf else "f32",
                get=get, bias=np.asarray(z["logit_bias"], np.float32),
                gbias=np.asarray(z["grad_logit_bias"], np.float32))


def test_golden_fixtures_present():
    assert len(GOLDEN) >= 6


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_oracle_matches_reference_golden(path):
    g = _load_golden(path)
    get = g["get"]
    args = (g["NH"], g["NKVH"], g["Da"], g["r"], True, g["io"])
    oq, ok, ov = O.scan_forward(get("combined"), get("inits"), g["bias"], *args)
    gc, gi, gb = O.scan_backward(get("combined"), get("inits"), g["bias"], get("out_q"),
                                 get("out_k"), get("out_v"), get("grad_q"), get("grad_k"),
                                 get("grad_v"), *args)
    if g["io"] == "bf16":
        # the fp32 state is identical op for op; rounding to bf16 then agrees bit for bit
        for a, k in ((oq, "out_q"), (ok, "out_k"), (ov, "out_v"), (gc, "grad_combined"),
                     (gi, "grad_inits")):
            np.testing.assert_array_equal(a, get(k), err_msg=k)
    else:
        # fp32: torch's sigmoid and numpy's exp may differ in the last ulp
        for a, k in ((oq, "out_q"), (ok, "out_k"), (ov, "out_v"), (gc, "grad_combined"),
                     (gi, "grad_inits")):
            np.testing.assert_allclose(a, get(k), rtol=1e-5, atol=1e-6, err_msg=k)
    np.testing.assert_allclose(gb, g["gbias"], rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------
# sample-and-hold closed form (gates exactly 0 or 1)
# ---------------------------------------------------------------------------
def _hold_forward(combined, inits, NH, NKVH, Da, r):
    """h_t = u at the last s <= t with alpha_s = 1, else the init."""
    u, lg = O.split_combined(combined, NH, NKVH, Da, r)
    B, T, H, D = u.shape
    alpha = np.repeat(lg, r, axis=-1)  # (B, T, H, D) in {0, 1}
    t_idx = np.arange(T)[None, :, None, None]
    last = np.where(alpha == 1, t_idx, -1)
    last = np.maximum.accumulate(last, axis=1)
    gathered = np.take_along_axis(u, np.maximum(last, 0), axis=1)
    init_b = np.broadcast_to(inits.reshape(B, 1, H, D), u.shape)
    h = np.where(last >= 0, gathered, init_b)
    return h.transpose(0, 2, 1, 3)  # (B, H, T, D)


def _hold_backward(combined, inits, gy, NH, NKVH, Da, r):
    """g_t = sum of gy over [t, next s > t with alpha_s = 1); then the slot grads."""
    u, lg = O.split_combined(combined, NH, NKVH, Da, r)
    B, T, H, D = u.shape
    alpha = np.repeat(lg, r, axis=-1)
    gy_t = gy.transpose(0, 2, 1, 3)  # (B, T, H, D)
    g = np.zeros_like(gy_t)
    csum = np.concatenate([np.zeros((B, 1, H, D)), np.cumsum(gy_t, axis=1)], axis=1)
    nxt = np.full((B, H, D), T)
    for t in range(T - 1, -1, -1):
        g[:, t] = csum[np.arange(B)[:, None, None], nxt, np.arange(H)[None, :, None],
                       np.arange(D)[None, None, :]] - csum[:, t]
        nxt = np.where(alpha[:, t] == 1, t, nxt)
    h = _hold_forward(combined, inits, NH, NKVH, Da, r).transpose(0, 2, 1, 3)
    h_prev = np.concatenate([inits.reshape(B, 1, H, D), h[:, :-1]], axis=1)
    du = alpha * g
    dalpha = (u - h_prev) * g
    dlogit = dalpha.reshape(B, T, H, Da, r).sum(-1)
    dinit = (1 - alpha[:, 0]) * g[:, 0]
    gc = np.concatenate([du, dlogit], axis=-1).reshape(B, T, -1)
    return gc, dinit, dlogit.sum(axis=(0, 1))


@pytest.mark.parametrize("T", [1, 2, 3, 31, 32, 33])
@pytest.mark.parametrize("Da,r", [(2, 1), (1, 2), (2, 4), (1, 8)])
def test_oracle_hold_closed_form(T, Da, r):
    B, NH, NKVH = 4, 8, 8
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, sigmoid=False)
    oq, ok, ov = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, False, "f32")
    h = _hold_forward(c, ini, NH, NKVH, Da, r)
    np.testing.assert_array_equal(np.concatenate([oq, ok, ov], axis=1), h)
    rng = np.random.default_rng(T * 7 + r)
    gy = rng.integers(-3, 4, size=h.shape).astype(np.float32)
    gq, gk, gv = gy[:, :NH], gy[:, NH:2 * NH], gy[:, 2 * NH:]
    gc, gi, gb = O.scan_backward(c, ini, bias, oq, ok, ov, gq, gk, gv, NH, NKVH, Da, r,
                                 False, "f32")
    egc, egi, egb = _hold_backward(c, ini, gy, NH, NKVH, Da, r)
    np.testing.assert_array_equal(gc, egc)
    np.testing.assert_array_equal(gi, egi)
    np.testing.assert_array_equal(gb, egb)


def test_hold_check_catches_a_planted_mistake(monkeypatch):
    """Swapping the roles of alpha and 1 - alpha in the oracle must fail the check."""
    B, T, NH, NKVH, Da, r = 2, 9, 1, 1, 1, 2
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, sigmoid=False)
    real = O._alphas
    monkeypatch.setattr(O, "_alphas", lambda lg, b, s, rr, cd: tuple(
        1 - x for x in real(lg, b, s, rr, cd)))
    oq, ok, ov = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, False, "f32")
    h = _hold_forward(c, ini, NH, NKVH, Da, r)
    assert not np.array_equal(np.concatenate([oq, ok, ov], axis=1), h)


# ---------------------------------------------------------------------------
# constant alpha: geometric closed form (float64)
# ---------------------------------------------------------------------------
def test_oracle_constant_alpha_closed_form():
    rng = np.random.default_rng(0)
    B, T, NH, NKVH, Da, r = 2, 40, 1, 1, 2, 3
    H, D = NH + 2 * NKVH, Da * r
    c = rng.standard_normal((B, T, H * (D + Da)))
    c4 = c.reshape(B, T, H, D + Da)
    z = 0.7
    c4[..., D:] = z  # every logit the same
    bias = np.full((H, Da), -0.3)
    ini = rng.standard_normal((B, H, D))
    oq, ok, ov = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, True, "f64")
    h = np.concatenate([oq, ok, ov], axis=1)  # (B, H, T, D)
    a = 1.0 / (1.0 + np.exp(-(z - 0.3)))
    u = c4[..., :D].transpose(0, 2, 1, 3)
    for t in range(T):
        k = np.arange(t + 1)
        w = a * (1 - a) ** (t - k)
        expect = (1 - a) ** (t + 1) * ini + np.einsum("k,bhkd->bhd", w, u[:, :, : t + 1])
        np.testing.assert_allclose(h[:, :, t], expect, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# finite differences of the float64 oracle
# ---------------------------------------------------------------------------
def test_oracle_backward_matches_finite_differences():
    rng = np.random.default_rng(1)
    B, T, NH, NKVH, Da, r = 2, 7, 1, 1, 2, 2
    H, D = NH + 2 * NKVH, Da * r
    c = rng.standard_normal((B, T, H * (D + Da)))
    ini = rng.standard_normal((B, H, D))
    bias = rng.standard_normal((H, Da)) * 0.5
    w = rng.standard_normal((B, H, T, D))  # loss = sum(w * out)
    args = (NH, NKVH, Da, r, True, "f64")

    def loss(c_, ini_, bias_):
        oq, ok, ov = O.scan_forward(c_, ini_, bias_, *args)
        return float((np.concatenate([oq, ok, ov], axis=1) * w).sum())

    oq, ok, ov = O.scan_forward(c, ini, bias, *args)
    gc, gi, gb = O.scan_backward(c, ini, bias, oq, ok, ov, w[:, :NH], w[:, NH:NH + NKVH],
                                 w[:, NH + NKVH:], *args)
    eps = 1e-6

    def fd(arr, idx, fn):
        p = arr.copy()
        m = arr.copy()
        p[idx] += eps
        m[idx] -= eps
        return (fn(p) - fn(m)) / (2 * eps)

    for idx in np.ndindex(c.shape):
        num = fd(c, idx, lambda x: loss(x, ini, bias))
        assert abs(num - gc[idx]) < 1e-6 * (1 + abs(num)), ("combined", idx, num, gc[idx])
    for idx in np.ndindex(ini.shape):
        num = fd(ini, idx, lambda x: loss(c, x, bias))
        assert abs(num - gi[idx]) < 1e-6 * (1 + abs(num)), ("inits", idx)
    for idx in np.ndindex(bias.shape):
        num = fd(bias, idx, lambda x: loss(c, ini, x))
        assert abs(num - gb[idx]) < 1e-6 * (1 + abs(num)), ("bias", idx)


def test_oracle_state_continuity_and_linearity():
    rng = np.random.default_rng(2)
    B, T, NH, NKVH, Da, r = 2, 30, 2, 1, 1, 4
    H, D = NH + 2 * NKVH, Da * r
    c = rng.standard_normal((B, T, H * (D + Da)))
    ini = rng.standard_normal((B, H, D))
    bias = rng.standard_normal((H, Da))
    args = (NH, NKVH, Da, r, True, "f64")
    full = np.concatenate(O.scan_forward(c, ini, bias, *args), axis=1)
    first = np.concatenate(O.scan_forward(c[:, :13], ini, bias, *args), axis=1)
    second = np.concatenate(O.scan_forward(c[:, 13:], first[:, :, -1], bias, *args), axis=1)
    np.testing.assert_array_equal(np.concatenate([first, second], axis=2), full)
    # linear in (values, inits) at fixed gates
    c2 = rng.standard_normal(c.shape)
    c2.reshape(B, T, H, D + Da)[..., D:] = c.reshape(B, T, H, D + Da)[..., D:]
    ini2 = rng.standard_normal(ini.shape)
    mix = 0.3 * c + 0.7 * c2
    mix.reshape(B, T, H, D + Da)[..., D:] = c.reshape(B, T, H, D + Da)[..., D:]
    lhs = np.concatenate(O.scan_forward(mix, 0.3 * ini + 0.7 * ini2, bias, *args), axis=1)
    rhs = 0.3 * full + 0.7 * np.concatenate(O.scan_forward(c2, ini2, bias, *args), axis=1)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# projection
# ---------------------------------------------------------------------------
def test_oracle_linear_transpose_matches_torch():
    rng = np.random.default_rng(3)
    B, T, K, F = 2, 31, 63, 127
    x = rng.standard_normal((B, T, K))
    w = rng.standard_normal((F, K))
    go = rng.standard_normal((B, F, T))
    out = O.linear_transpose_forward(x, w, "f64")
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    ref = torch.matmul(wt, xt.transpose(-1, -2))
    ref.backward(torch.tensor(go))
    np.testing.assert_allclose(out, ref.detach().numpy(), rtol=1e-12, atol=1e-12)
    gx, gw = O.linear_transpose_backward(x, w, go, "f64")
    np.testing.assert_allclose(gx, xt.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gw, wt.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_bf16_rounding_is_round_to_nearest_even():
    vals = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, -3.0e38, np.inf, 1e-40],
                    np.float32)
    want = torch.tensor(vals).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(vals), want)


def test_oracle_empty_time():
    """T == 0: no step runs, so the outputs are empty and no gradient reaches
    the inits or the bias (the autograd of an empty loop)."""
    B, NH, NKVH, Da, r = 2, 1, 1, 2, 3
    H, D = NH + 2 * NKVH, Da * r
    c = np.zeros((B, 0, H * (D + Da)), np.float32)
    ini = np.ones((B, H, D), np.float32)
    bias = np.ones((H, Da), np.float32)
    hq, hk, hv = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, True, "f32")
    assert hq.shape == (B, NH, 0, D) and hk.shape == (B, NKVH, 0, D) and hv.shape == (B, NKVH, 0, D)
    gc, gi, gb = O.scan_backward(c, ini, bias, hq, hk, hv, hq, hk, hv, NH, NKVH, Da, r, True, "f32")
    assert gc.shape == c.shape
    assert gi.shape == (B, H, D) and not np.any(gi)
    assert gb.shape == (H, Da) and not np.any(gb)
