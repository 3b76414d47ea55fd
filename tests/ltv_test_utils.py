"""Shared helpers for the LTV parity tests.

The integer generators, the stride-layout enumeration and the tolerance rule
follow the reference's own test utilities
(tests/ltv_scan_test_utils.py:59-136 of aioaneid/nanochat-filter): values
((9b + 7t + 3h + d) % 5) - 2, gate logits (b + t + h + j) % 2, inits
((13b + 3h + d) % 7) - 3, logit bias ((h + 2j) % 3) - 1 with the sigmoid and 0
without it.  Without the sigmoid the gates are 0 or 1 and every result is a
small integer, so kernel and oracle must agree exactly.
"""

from __future__ import annotations

import itertools

import numpy as np
import torch

import ltv_oracle as O


def stride_layouts(shape):
    """Every axis order x gap factor in {1, 2} per axis (reference :66-77)."""
    layouts = set()
    ndim = len(shape)
    for order in itertools.permutations(range(ndim)):
        for gaps in itertools.product((1, 2), repeat=ndim):
            stride = [0] * ndim
            running = 1
            for axis, gap in zip(order, gaps):
                stride[axis] = running * gap
                running = stride[axis] * shape[axis]
            layouts.add(tuple(stride))
    return sorted(layouts)


def storage_size(shape, stride):
    return 1 + sum((n - 1) * s for n, s in zip(shape, stride))


def int_combined(B, T, NH, NKVH, Da, r):
    H = NH + 2 * NKVH
    D = Da * r
    b, t, h, e = np.meshgrid(np.arange(B), np.arange(T), np.arange(H), np.arange(D + Da),
                             indexing="ij")
    vals = ((9 * b + 7 * t + 3 * h + e) % 5) - 2
    gates = (b + t + h + (e - D)) % 2
    c = np.where(e < D, vals, gates).astype(np.float32)
    return c.reshape(B, T, H * (D + Da))


def int_inits(B, NH, NKVH, Da, r):
    H = NH + 2 * NKVH
    D = Da * r
    b, h, d = np.meshgrid(np.arange(B), np.arange(H), np.arange(D), indexing="ij")
    return (((13 * b + 3 * h + d) % 7) - 3).astype(np.float32)


def int_logit_bias(NH, NKVH, Da, sigmoid):
    H = NH + 2 * NKVH
    h, j = np.meshgrid(np.arange(H), np.arange(Da), indexing="ij")
    if not sigmoid:
        return np.zeros((H, Da), np.float32)
    return (((h + 2 * j) % 3) - 1).astype(np.float32)


def to_torch(a: np.ndarray, dtype: torch.dtype, device="cpu") -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t.to(dtype).to(device)


def strided_copy(a: np.ndarray, stride, dtype, device) -> torch.Tensor:
    """Device tensor with the values of ``a`` and the given element strides."""
    base = torch.zeros(storage_size(a.shape, stride), dtype=dtype, device=device)
    view = torch.as_strided(base, size=a.shape, stride=stride)
    view.copy_(to_torch(a, dtype, device))
    return view


def np_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def io_name(dtype: torch.dtype) -> str:
    return "bf16" if dtype == torch.bfloat16 else "f32"


# tolerances: fp32 1e-4, bf16 I/O with fp32 state 2e-2
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}

# error statistics of every assert_close call, written out at session end when
# LTV_ERR_REPORT names a file (tests/conftest.py)
ERR_LOG: list = []


def err_stats(actual, expected):
    """max |a - e|; normwise relative error max|a - e| / max|e|; element-wise
    relative error max |a - e| / |e| over the elements with |e| >= 1e-2 max|e|
    (below that floor a relative error measures cancellation in the inputs,
    not the kernel)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    if e.size == 0:
        return {"max_abs": 0.0, "norm_rel": 0.0, "elem_rel": 0.0}
    diff = np.abs(a - e)
    emax = float(np.abs(e).max())
    max_abs = float(diff.max())
    norm_rel = max_abs / emax if emax > 0 else (0.0 if max_abs == 0 else float("inf"))
    big = np.abs(e) >= 1e-2 * emax
    elem_rel = float((diff[big] / np.abs(e[big])).max()) if emax > 0 and big.any() else 0.0
    return {"max_abs": max_abs, "norm_rel": norm_rel, "elem_rel": elem_rel}


def assert_close(actual, expected, tol, label=""):
    """|a - e| <= tol * (|e| + max(1, max|e|)) elementwise; tol = 0 means exact.

    Returns (and logs) the error statistics of ``err_stats``: the normwise and
    element-wise relative errors are reported beside this rule."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, (label, a.shape, e.shape)
    if tol == 0:
        bad = a != e
    else:
        scale = max(1.0, float(np.abs(e).max()) if e.size else 1.0)
        bad = np.abs(a - e) > tol * (np.abs(e) + scale)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        msg = ", ".join(f"{tuple(i)}: got {a[tuple(i)]} want {e[tuple(i)]}" for i in idx)
        raise AssertionError(f"{label}: {int(bad.sum())}/{bad.size} mismatches (tol={tol}): {msg}")
    stats = err_stats(a, e)
    ERR_LOG.append({"label": label, "tol": tol, "size": int(e.size), **stats})
    return stats


def assert_norm_rel(actual, expected, tol, label=""):
    """The north star's "max rel err" read normwise: max|a - e| <= tol * max|e|."""
    stats = err_stats(actual, expected)
    assert stats["norm_rel"] <= tol, f"{label}: normwise relative error {stats['norm_rel']:.3e} > {tol}"
    ERR_LOG.append({"label": label + " (normwise)", "tol": tol,
                    "size": int(np.asarray(expected).size), **stats})
    return stats
