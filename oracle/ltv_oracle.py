"""CPU oracle for the LTV combined-QKV filter path.

TEST INFRASTRUCTURE ONLY.  This module is the checker that the HIP kernels are
compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
as the timed CPU baseline -- never as a product code path.  The product
(``nanochat_amd``) fails loudly when its HIP library is missing; it never falls
back to this module.

What it restates (all citations relative to the reference tree):

* ``scan_forward``  -- the sequential head-major recurrence of
  ``nanochat/ops/ltv_reference_ops.py:37-124`` with P=2**31-1, Q=1, K=1
  (``:162-192``): ``h_t = (1 - a_t) * h_{t-1} + a_t * u_t`` per channel,
  ``a_t = sigmoid(logit_t + bias)`` shared by ``r`` channels, fp32 state,
  outputs rounded to the I/O dtype.
* ``scan_backward`` -- the autograd of that loop through ``QuantizedStateUpdate``
  (``ltv_reference_ops.py:7-34``): the alpha gradient uses the *I/O-rounded*
  previous state, exactly what the CUDA kernel reads back from its saved output
  (``cpp_ewma/src/ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_backward.cu:51-81``).
* ``look_back_forward/backward`` -- the same loop with chunk restarts
  (``ltv_reference_ops.py:37-124`` with general P, Q, K) and the autograd of
  it summed over the overlapping windows.
* ``linear_transpose_forward/backward`` -- ``fused_linear_transpose_reference``
  (``ltv_reference_ops.py:299-308``): ``matmul(x, W^T).transpose(1, 2)``.

Arithmetic contract: numpy float32 element-wise ops, one rounding per op, in the
same operation order as the torch CPU reference; bf16 rounding is
round-to-nearest-even on the fp32 bit pattern.  GEMMs accumulate in float64 and
round once (the device accumulates in fp32; both are within the tolerances the
tests state).

How each function is pinned (tests/test_oracle.py):
  * scan_forward / scan_backward: the reference's exact-integer generators
    (tests/ltv_scan_test_utils.py:84-131, use_sigmoid=False) against the
    sample-and-hold closed form; the constant-alpha geometric closed form;
    float64 finite differences of scan_forward for scan_backward; state
    continuity; and golden vectors written by the reference's own
    ltv_reference_ops.py (tests/golden/).
  * look_back_forward / look_back_backward: P >= T reduces them to the
    scan above; the exact-integer generators against a per-window
    sample-and-hold closed form; each window equals scan_forward of its slice;
    float64 finite differences over overlapping windows (K - 1 > Q included);
    golden vectors of the reference's look-back function (tests/golden/).
  * linear_transpose_*: numpy/torch matmul (a library routine) and finite
    differences.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_round",
    "bf16_bits",
    "bf16_from_bits",
    "round_io",
    "sigmoid_f32",
    "split_combined",
    "scan_forward",
    "scan_backward",
    "UNBOUNDED_P",
    "look_back_windows",
    "look_back_forward",
    "look_back_backward",
    "linear_transpose_forward",
    "linear_transpose_backward",
    "filter_forward",
    "filter_backward",
]


# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------
def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16), round-to-nearest-even, NaN kept quiet."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounding_bias = ((u >> 16) & 1) + 0x7FFF
    r = ((u + rounding_bias) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 value, returned as fp32."""
    return bf16_from_bits(bf16_bits(x))


def round_io(x: np.ndarray, io_dtype: str) -> np.ndarray:
    if io_dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    if io_dtype == "bf16":
        return bf16_round(np.asarray(x, dtype=np.float32))
    if io_dtype == "f64":
        return np.asarray(x, dtype=np.float64)
    raise ValueError(f"unknown io dtype {io_dtype!r}")


def _compute_dtype(io_dtype: str):
    return np.float64 if io_dtype == "f64" else np.float32


def sigmoid_f32(x: np.ndarray) -> np.ndarray:
    """1 / (1 + exp(-x)) in the array's precision.

    Same formula as ``sigmoid_f32`` in
    ``cpp_ewma/src/ltv_fused_concat_head_major_register_cast_scan_cuda_common.cuh:114-117``
    and torch's CPU sigmoid used by ``ltv_reference_ops.py:113``.
    """
    dt = x.dtype
    one = dt.type(1.0)
    with np.errstate(over="ignore"):
        return (one / (one + np.exp(-x))).astype(dt)


# ---------------------------------------------------------------------------
# layout helpers
# ---------------------------------------------------------------------------
def split_combined(combined: np.ndarray, NH: int, NKVH: int, Da: int, r: int):
    """(B, T, F) head-interleaved -> values (B, T, H, D), logits (B, T, H, Da).

    Feature layout ``[h0 values (D) | h0 logits (Da) | h1 values | ...]``
    (``nanochat/ltv_combined_head_major_qkv_filter.py:12, 43-58``).
    """
    B, T, F = combined.shape
    H = NH + 2 * NKVH
    D = Da * r
    assert F == H * (D + Da), (F, H, D, Da)
    per_head = combined.reshape(B, T, H, D + Da)
    return per_head[..., :D], per_head[..., D:]


def _split_heads(h_all: np.ndarray, NH: int, NKVH: int):
    """(B, H, T, D) -> out_q (B, NH, T, D), out_k, out_v (B, NKVH, T, D)."""
    return (
        np.ascontiguousarray(h_all[:, :NH]),
        np.ascontiguousarray(h_all[:, NH : NH + NKVH]),
        np.ascontiguousarray(h_all[:, NH + NKVH :]),
    )


# ---------------------------------------------------------------------------
# scan
# ---------------------------------------------------------------------------
def _alphas(logits, logit_bias, use_sigmoid, r, cd):
    # logits (B, T, H, Da) already I/O-exact; bias (H, Da) fp32.
    # ltv_reference_ops.py:107-114: alpha_raw = logit.to(f32) + bias;
    # alpha = sigmoid(alpha_raw) or alpha_raw; broadcast with repeat_interleave(r).
    raw = logits.astype(cd) + logit_bias.astype(cd)[None, None]
    alpha = sigmoid_f32(raw) if use_sigmoid else raw
    return alpha, np.repeat(alpha, r, axis=-1)


def scan_forward(
    combined: np.ndarray,
    inits: np.ndarray,
    logit_bias: np.ndarray,
    NH: int,
    NKVH: int,
    Da: int,
    r: int,
    use_sigmoid: bool,
    io_dtype: str = "f32",
):
    """Full-recurrence forward scan.

    Follows ``ltv_reference_ops.py:83-124`` (``P=2**31-1, Q=1, K=1`` makes a
    single chunk covering all of T, ``:65-75``).

    combined (B, T, F), inits (B, H, D) and logit_bias (H, Da) hold values that
    are already exact in ``io_dtype`` (bias is fp32).  Returns
    ``(out_q, out_k, out_v)`` with shapes (B, NH|NKVH, T, D), rounded to
    ``io_dtype`` and returned as fp32 (or fp64 for io_dtype="f64").
    """
    cd = _compute_dtype(io_dtype)
    u, logits = split_combined(np.asarray(combined), NH, NKVH, Da, r)
    B, T = u.shape[:2]
    H = NH + 2 * NKVH
    D = Da * r
    u = u.astype(cd)
    _, alpha_bc = _alphas(logits, np.asarray(logit_bias), use_sigmoid, r, cd)
    one = cd(1.0)
    h = np.asarray(inits, dtype=cd).reshape(B, H, D).copy()
    out = np.empty((B, H, T, D), dtype=cd)
    for t in range(T):
        a = alpha_bc[:, t]
        # QuantizedStateUpdate.forward (ltv_reference_ops.py:11):
        #   next_state = (1.0 - alpha) * state + alpha * x_val
        h = ((one - a) * h + a * u[:, t]).astype(cd)
        out[:, :, t] = round_io(h, io_dtype)
    return _split_heads(out, NH, NKVH)


def scan_backward(
    combined: np.ndarray,
    inits: np.ndarray,
    logit_bias: np.ndarray,
    hq: np.ndarray,
    hk: np.ndarray,
    hv: np.ndarray,
    grad_hq: np.ndarray,
    grad_hk: np.ndarray,
    grad_hv: np.ndarray,
    NH: int,
    NKVH: int,
    Da: int,
    r: int,
    use_sigmoid: bool,
    io_dtype: str = "f32",
):
    """Backward of ``scan_forward``.

    Semantics of ``QuantizedStateUpdate.backward`` (``ltv_reference_ops.py:20-34``)
    chained over t, which is also what the CUDA kernel computes
    (``…_cuda_backward.cu:51-81, 271-300, 349-399``):

      g_t        = gy_t + (1 - a_{t+1}) * g_{t+1},     g_T = 0
      d u_t      = a_t * g_t
      d a_t[d]   = (u_t[d] - h_{t-1}[d]) * g_t[d]       h_{t-1}: saved output (I/O-rounded), h_{-1} = inits
      d logit_t  = sum_{d in group} d a_t[d]  (* a_t (1 - a_t) with sigmoid)
      d bias     = sum_{b,t} d logit_t   (fp32, never rounded to the I/O dtype)
      d inits    = (1 - a_0) * g_0

    Returns ``(grad_combined (B, T, F), grad_inits (B, H, D), grad_logit_bias (H, Da))``;
    grad_combined and grad_inits rounded to ``io_dtype``; grad_logit_bias fp32.
    """
    cd = _compute_dtype(io_dtype)
    combined = np.asarray(combined)
    u, logits = split_combined(combined, NH, NKVH, Da, r)
    B, T = u.shape[:2]
    H = NH + 2 * NKVH
    D = Da * r
    u = u.astype(cd)
    alpha, alpha_bc = _alphas(logits, np.asarray(logit_bias), use_sigmoid, r, cd)
    h_saved = np.concatenate([hq, hk, hv], axis=1).astype(cd)  # (B, H, T, D)
    gy = np.concatenate([grad_hq, grad_hk, grad_hv], axis=1).astype(cd)
    init = np.asarray(inits, dtype=cd).reshape(B, H, D)
    one = cd(1.0)

    g = np.zeros((B, H, D), dtype=cd)
    grad_u = np.empty((B, T, H, D), dtype=cd)
    grad_logit = np.empty((B, T, H, Da), dtype=cd)
    for t in range(T - 1, -1, -1):
        if t == T - 1:
            g = gy[:, :, t].copy()
        else:
            # grad_state = grad_next_state * (1.0 - alpha)  (ltv_reference_ops.py:24)
            # accumulated with the output's own gradient.
            g = (gy[:, :, t] + g * (one - alpha_bc[:, t + 1])).astype(cd)
        a = alpha_bc[:, t]
        grad_u[:, t] = g * a  # ltv_reference_ops.py:27
        h_prev = init if t == 0 else h_saved[:, :, t - 1]
        d_alpha = g * (u[:, t] - h_prev)  # ltv_reference_ops.py:32
        d_alpha_sum = d_alpha.reshape(B, H, Da, r).sum(axis=-1, dtype=cd)
        if use_sigmoid:
            at = alpha[:, t]
            d_logit = (d_alpha_sum * ((one - at) * at)).astype(cd)
        else:
            d_logit = d_alpha_sum
        grad_logit[:, t] = d_logit
        if t == 0:
            grad_init = (g * (one - a)).astype(cd)
    if T == 0:
        grad_init = np.zeros((B, H, D), dtype=cd)

    grad_bias = grad_logit.sum(axis=(0, 1), dtype=np.float64).astype(
        np.float64 if io_dtype == "f64" else np.float32
    )
    grad_combined = np.concatenate([grad_u, grad_logit], axis=-1).reshape(B, T, H * (D + Da))
    return (
        round_io(grad_combined, io_dtype),
        round_io(grad_init, io_dtype),
        grad_bias,
    )


# ---------------------------------------------------------------------------
# look-back scan: chunk restarts with a K - 1 step warm-up
# ---------------------------------------------------------------------------
UNBOUNDED_P = 2_147_483_647


def look_back_windows(T: int, P: int, Q: int, K: int):
    """Chunk windows ``(lo, st, hi)`` of the look-back scan.

    ``ltv_reference_ops.py:65-75`` cuts T into ``[0, min(P, T))`` and then
    chunks of Q steps ``[P + (i - 1) Q, min(P + i Q, T))``; each chunk
    ``[st, hi)`` restarts from the inits at ``lo = max(0, st - (K - 1))``
    (``:99-101``) and outputs only its own steps.  The same bounds as the CUDA
    forward (``…look_back…blelloch_scan_cuda_forward.cu:36-37, 104-110``).
    """
    if T > P:
        M = (T - P + Q - 1) // Q
        chunks = [(0, min(P, T))]
        for i in range(1, M + 1):
            s, e = P + (i - 1) * Q, min(P + i * Q, T)
            if s < T:
                chunks.append((s, e))
    else:
        chunks = [(0, T)]
    return [(max(0, s - (K - 1)), s, e) for s, e in chunks]


def look_back_forward(combined, inits, logit_bias, NH, NKVH, Da, r, P, Q, K,
                      use_sigmoid, io_dtype="f32"):
    """Forward of ``ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_minimal``
    (``ltv_reference_ops.py:37-124``): every window of ``look_back_windows``
    runs the recurrence from the inits over ``[lo, hi)`` in fp32 and writes
    the I/O-rounded states of ``[st, hi)``.  Returns (out_q, out_k, out_v)."""
    cd = _compute_dtype(io_dtype)
    u, logits = split_combined(np.asarray(combined), NH, NKVH, Da, r)
    B, T = u.shape[:2]
    H = NH + 2 * NKVH
    D = Da * r
    u = u.astype(cd)
    _, alpha_bc = _alphas(logits, np.asarray(logit_bias), use_sigmoid, r, cd)
    one = cd(1.0)
    init = np.asarray(inits, dtype=cd).reshape(B, H, D)
    out = np.zeros((B, H, T, D), dtype=cd)
    for lo, st, hi in look_back_windows(T, P, Q, K):
        h = init.copy()
        for t in range(lo, hi):
            a = alpha_bc[:, t]
            h = ((one - a) * h + a * u[:, t]).astype(cd)
            if t >= st:
                out[:, :, t] = round_io(h, io_dtype)
    return _split_heads(out, NH, NKVH)


def look_back_backward(combined, inits, logit_bias, grad_hq, grad_hk, grad_hv, NH, NKVH,
                       Da, r, P, Q, K, use_sigmoid, io_dtype="f32"):
    """Backward of ``look_back_forward``: the autograd of the reference loop
    (``QuantizedStateUpdate.backward``, ``ltv_reference_ops.py:20-34``) summed
    over the windows.  Each window ``(lo, st, hi)`` runs its own reverse chain
    from ``g_hi = 0``, taking upstream gradients only on its own steps
    ``[st, hi)``; its alpha gradient uses its own I/O-rounded states (the
    warm-up states included); every window adds ``(1 - a_lo) g_lo`` to the
    inits gradient.  A step inside later windows' warm-ups therefore collects
    one contribution per covering window.  Contributions are summed in fp32 in
    window order and rounded once.

    Returns ``(grad_combined (B, T, F), grad_inits (B, H, D), grad_logit_bias (H, Da))``.
    """
    cd = _compute_dtype(io_dtype)
    combined = np.asarray(combined)
    u, logits = split_combined(combined, NH, NKVH, Da, r)
    B, T = u.shape[:2]
    H = NH + 2 * NKVH
    D = Da * r
    u = u.astype(cd)
    alpha, alpha_bc = _alphas(logits, np.asarray(logit_bias), use_sigmoid, r, cd)
    gy = np.concatenate([grad_hq, grad_hk, grad_hv], axis=1).astype(cd)
    init = np.asarray(inits, dtype=cd).reshape(B, H, D)
    one = cd(1.0)
    grad_u = np.zeros((B, T, H, D), dtype=cd)
    grad_logit = np.zeros((B, T, H, Da), dtype=cd)
    grad_init = np.zeros((B, H, D), dtype=cd)
    for lo, st, hi in look_back_windows(T, P, Q, K):
        if hi <= lo:
            continue
        # I/O-rounded state entering each step of the window (state_quant)
        hq = np.empty((hi - lo, B, H, D), dtype=cd)
        h = init.copy()
        for t in range(lo, hi):
            hq[t - lo] = round_io(h, io_dtype)
            a = alpha_bc[:, t]
            h = ((one - a) * h + a * u[:, t]).astype(cd)
        g = np.zeros((B, H, D), dtype=cd)
        for t in range(hi - 1, lo - 1, -1):
            gyt = gy[:, :, t] if t >= st else np.zeros((B, H, D), dtype=cd)
            if t == hi - 1:
                g = gyt.copy()
            else:
                g = (gyt + g * (one - alpha_bc[:, t + 1])).astype(cd)
            grad_u[:, t] += g * alpha_bc[:, t]
            d_alpha = g * (u[:, t] - hq[t - lo])
            d_alpha_sum = d_alpha.reshape(B, H, Da, r).sum(axis=-1, dtype=cd)
            if use_sigmoid:
                at = alpha[:, t]
                grad_logit[:, t] += (d_alpha_sum * ((one - at) * at)).astype(cd)
            else:
                grad_logit[:, t] += d_alpha_sum
        grad_init += (g * (one - alpha_bc[:, lo])).astype(cd)
    grad_bias = grad_logit.sum(axis=(0, 1), dtype=np.float64).astype(
        np.float64 if io_dtype == "f64" else np.float32
    )
    grad_combined = np.concatenate([grad_u, grad_logit], axis=-1).reshape(B, T, H * (D + Da))
    return (
        round_io(grad_combined, io_dtype),
        round_io(grad_init, io_dtype),
        grad_bias,
    )


# ---------------------------------------------------------------------------
# projection
# ---------------------------------------------------------------------------
def linear_transpose_forward(x: np.ndarray, weight: np.ndarray, io_dtype: str = "f32"):
    """(B, T, K) x (F, K) -> (B, F, T) = matmul(x, W^T).transpose(1, 2)

    ``ltv_reference_ops.py:299-308``.  Accumulated in float64, rounded once to
    the I/O dtype.
    """
    out = np.matmul(np.asarray(x, np.float64), np.asarray(weight, np.float64).T)
    out = np.ascontiguousarray(out.transpose(0, 2, 1))
    if io_dtype == "f64":
        return out
    return round_io(out.astype(np.float32), io_dtype)


def linear_transpose_backward(x: np.ndarray, weight: np.ndarray, grad_out: np.ndarray,
                              io_dtype: str = "f32"):
    """grad of ``linear_transpose_forward``: grad_out (B, F, T) ->
    grad_x (B, T, K) (I/O dtype) and grad_weight (F, K) (fp32 accumulate)."""
    go = np.asarray(grad_out, np.float64).transpose(0, 2, 1)  # (B, T, F)
    gx = np.matmul(go, np.asarray(weight, np.float64))
    gw = np.einsum("btf,btk->fk", go, np.asarray(x, np.float64))
    if io_dtype == "f64":
        return gx, gw
    return round_io(gx.astype(np.float32), io_dtype), gw.astype(np.float32)


# ---------------------------------------------------------------------------
# whole filter (projection + scan), the module-level semantics of
# nanochat/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter.py:24-73
# ---------------------------------------------------------------------------
def filter_forward(x, weight, inits, logit_bias, NH, NKVH, Da, r, io_dtype="f32",
                   use_sigmoid=True):
    """Returns (q, k, v) as (B, T, H, D) arrays plus the combined (B, T, F)."""
    out_bft = linear_transpose_forward(x, weight, io_dtype)
    combined = np.ascontiguousarray(out_bft.transpose(0, 2, 1))
    hq, hk, hv = scan_forward(combined, inits, logit_bias, NH, NKVH, Da, r,
                              use_sigmoid, io_dtype)
    return (hq.transpose(0, 2, 1, 3), hk.transpose(0, 2, 1, 3),
            hv.transpose(0, 2, 1, 3), combined, (hq, hk, hv))


def filter_backward(x, weight, inits, logit_bias, combined, saved, dq, dk, dv,
                    NH, NKVH, Da, r, io_dtype="f32", use_sigmoid=True):
    """Gradients of ``filter_forward`` for upstream (B, T, H, D) grads.

    Returns grad_x, grad_weight (fp32), grad_inits (B, H, D), grad_logit_bias.
    """
    hq, hk, hv = saved
    gq = np.ascontiguousarray(np.asarray(dq).transpose(0, 2, 1, 3))
    gk = np.ascontiguousarray(np.asarray(dk).transpose(0, 2, 1, 3))
    gv = np.ascontiguousarray(np.asarray(dv).transpose(0, 2, 1, 3))
    gc, ginit, gbias = scan_backward(combined, inits, logit_bias, hq, hk, hv,
                                     gq, gk, gv, NH, NKVH, Da, r, use_sigmoid,
                                     io_dtype)
    gx, gw = linear_transpose_backward(x, weight, gc.transpose(0, 2, 1), io_dtype)
    return gx, gw, ginit, gbias
