"""GPU parity of the chained scans.  Forward (``ltv_hm_scan_forward_ws`` and the
split-layout ``ltv_hm_look_back_scan_forward_split_ws``, called here): one
workgroup per chunk of T, the state at a chunk's end handed to the next
chunk's workgroup through a zero-invariant workspace.  Backward
(``ltv_hm_look_back_scan_backward_split_ws``): one tile-long chunk per
workgroup, last chunk first, the gradient carry handed to the chunk before.

Checked against the CPU oracle (exact on the reference's integer generators,
within the stated tolerance with the sigmoid), against the tile kernel (the
same entry point without a workspace) on the same inputs, for bitwise
run-to-run equality, and for the workspace contract: all zero after every call, the ticket counter
back at 0 and no wait past its bound.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import (TOL, assert_close, int_combined, int_inits, int_logit_bias, io_name,
                            np_of, to_torch)

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float32]


def _lib():
    from nanochat_amd import _native as N
    return N, N.lib()


def _s(t):
    from nanochat_amd import _native as N
    return N.strides(t)


def _outs(B, T, NH, NKVH, D, dtype):
    return [torch.full((B, nh, T, D), float("nan"), dtype=dtype, device=DEV)
            for nh in (NH, NKVH, NKVH)]


def _split(comb, NH, NKVH, Da, r):
    """(B, T, H (D + Da)) -> head-major values (B, H, T, D) and logits
    (B, H, T, Da), contiguous: the layout the fast path hands the scan, with
    16-byte channel vectors (the combined layout's heads start at multiples of
    D + Da columns, which the chained kernel does not take)."""
    B, T, _ = comb.shape
    H, D = NH + 2 * NKVH, Da * r
    x = comb.reshape(B, T, H, D + Da).permute(0, 2, 1, 3)
    return x[..., :D].contiguous(), x[..., D:].contiguous()


UNBOUNDED_P = 2147483647


def _forward(comb, ini, bias, NH, NKVH, Da, r, sig, ws=None):
    """Scan forward of the split layout through the C ABI: the chained kernel
    with a workspace tensor, the tile kernel without one."""
    N, lib = _lib()
    B, T, _ = comb.shape
    D = Da * r
    values, logits = _split(comb, NH, NKVH, Da, r)
    out = _outs(B, T, NH, NKVH, D, comb.dtype)
    head = [N.dtype_code(comb.dtype), values.data_ptr(), _s(values), logits.data_ptr(),
            _s(logits), ini.data_ptr(), _s(ini)]
    rest = [bias.data_ptr(), out[0].data_ptr(), _s(out[0]), out[1].data_ptr(), _s(out[1]),
            out[2].data_ptr(), _s(out[2])]
    tail = [B, T, NH, NKVH, Da, r, UNBOUNDED_P, 1, 1, int(sig), N.stream_of(comb)]
    if ws is None:
        rc = lib.ltv_hm_look_back_scan_forward_split(*head, *rest, *tail)
    else:
        rc = lib.ltv_hm_look_back_scan_forward_split_ws(*head, N.dtype_code(ini.dtype), *rest,
                                                        ws.data_ptr(), ws.numel(), *tail)
    N.check(rc, "scan forward")
    return out


def _ws_bytes(dtype, B, T, NH, NKVH, Da, r):
    N, lib = _lib()
    return lib.ltv_hm_scan_forward_chain_workspace_size(N.dtype_code(dtype), B, T, NH, NKVH, Da, r)


def _zero_ws(nbytes):
    return torch.zeros((nbytes + 255) // 256 * 256, dtype=torch.uint8, device=DEV)


def _random_case(B, T, NH, NKVH, Da, r, seed, io, z_mean=2.0, z_std=1.0):
    rng = np.random.default_rng(seed)
    H, D = NH + 2 * NKVH, Da * r
    c = rng.standard_normal((B, T, H, D + Da)).astype(np.float32)
    c[..., D:] = -(z_mean + z_std * rng.standard_normal((B, T, H, Da)))
    c = O.round_io(c.reshape(B, T, -1), io)
    ini = O.round_io(rng.standard_normal((B, H, D)).astype(np.float32), io)
    bias = (0.1 * rng.standard_normal((H, Da))).astype(np.float32)
    return c, ini, bias


def _assert_same_up_to_association(a, b, dtype, label):
    """Two kernels that evaluate the same fp32 recurrence in different
    association orders: their fp32 states differ by a few fp32 rounding errors
    of the largest state (bound 1e-5 max|b| here), and a bf16 output can then
    round to the neighbouring value (one bf16 step, <= 2^-7 |b|)."""
    if b.numel() == 0:
        return
    a, b = a.float(), b.float()
    scale = float(b.abs().max())
    d = (a - b).abs()
    step = b.abs() * 2.0 ** -7 if dtype == torch.bfloat16 else torch.zeros_like(b)
    bad = d > step + 1e-5 * scale
    assert not bool(bad.any()), (
        f"{label}: {int(bad.sum())} elements differ beyond association; max |a-b| = "
        f"{float(d.max()):.3e}, max|b| = {scale:.3e}")


def _check_ws_clean(ws, label):
    torch.cuda.synchronize()
    nz = int(torch.count_nonzero(ws))
    assert nz == 0, f"{label}: {nz} nonzero workspace bytes after the call (ticket/err/words)"


# The library takes the chained kernel from 8 chunks per sequence on (chunks
# of 512 steps, 256 for r = 1): T spans 8 chunks whose last holds one step,
# exactly 8 chunks, and more with a ragged tail, for the d12 gate shape (one
# gate per head), gate groups of 16 channels, and per-channel gates (r = 1).
CASES = [
    # (B, T, NH, NKVH, Da, r)
    (2, 3585, 2, 1, 1, 128),
    (2, 4096, 1, 1, 1, 128),
    (2, 4700, 2, 1, 1, 128),
    (1, 4133, 1, 1, 8, 16),
    (2, 2000, 1, 1, 64, 1),
    (1, 1793, 1, 0, 128, 1),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("B,T,NH,NKVH,Da,r", CASES)
def test_chain_exact_integer(dtype, B, T, NH, NKVH, Da, r):
    """The reference's integer generators without the sigmoid (gates 0 / 1):
    every output exact, across chunk boundaries."""
    nbytes = _ws_bytes(dtype, B, T, NH, NKVH, Da, r)
    assert nbytes > 0
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, False)
    eq, ek, ev = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, False, io_name(dtype))
    ws = _zero_ws(nbytes)
    q, k, v = _forward(to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                       to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, False, ws)
    case = f"T={T} Da={Da} r={r}"
    assert_close(np_of(q), eq, 0, "q " + case)
    if NKVH:
        assert_close(np_of(k), ek, 0, "k " + case)
        assert_close(np_of(v), ev, 0, "v " + case)
    _check_ws_clean(ws, case)


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("B,T,NH,NKVH,Da,r", CASES)
def test_chain_sigmoid_vs_oracle_and_tile(dtype, B, T, NH, NKVH, Da, r):
    """Sigmoid gates, decay sigmoid(N(2, 1)): within the tolerance of the
    oracle; against the tile kernel (a different association of the same fp32
    recurrence) within one bf16 rounding step or 1e-5 in fp32; three calls on
    one workspace bitwise equal."""
    io = io_name(dtype)
    c, ini, bias = _random_case(B, T, NH, NKVH, Da, r, seed=T * 7 + r, io=io)
    eq, ek, ev = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, True, io)
    cd, idv, bd = to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV), to_torch(bias, torch.float32, DEV)
    ws = _zero_ws(_ws_bytes(dtype, B, T, NH, NKVH, Da, r))
    runs = [_forward(cd, idv, bd, NH, NKVH, Da, r, True, ws) for _ in range(3)]
    for run in runs[1:]:
        for a, b in zip(runs[0], run):
            assert torch.equal(a, b)
    q, k, v = runs[0]
    tol = TOL[dtype]
    case = f"T={T} Da={Da} r={r}"
    assert_close(np_of(q), eq, tol, "q " + case)
    if NKVH:
        assert_close(np_of(k), ek, tol, "k " + case)
        assert_close(np_of(v), ev, tol, "v " + case)
    tile = _forward(cd, idv, bd, NH, NKVH, Da, r, True)
    for a, b in zip(runs[0], tile):
        _assert_same_up_to_association(a, b, dtype, "chained vs tile " + case)
    _check_ws_clean(ws, case)


def test_chain_workspace_reuse_across_shapes():
    """One zeroed buffer serves calls of different shapes in a row (the
    invariant leaves it zeroed), including one with more chunks than the
    buffer's previous user."""
    dtype = torch.bfloat16
    shapes = [(2, 4100, 2, 1, 1, 128), (3, 3700, 1, 1, 1, 128), (1, 5000, 1, 1, 128, 1),
              (2, 4100, 2, 1, 1, 128)]
    need = max(_ws_bytes(dtype, *s) for s in shapes)
    ws = _zero_ws(need)
    for B, T, NH, NKVH, Da, r in shapes:
        c, ini, bias = _random_case(B, T, NH, NKVH, Da, r, seed=B + T, io="bf16")
        eq, _, _ = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, True, "bf16")
        q, _, _ = _forward(to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                           to_torch(bias, torch.float32, DEV), NH, NKVH, Da, r, True, ws)
        assert_close(np_of(q), eq, TOL[dtype], f"reuse T={T}")
        _check_ws_clean(ws, f"reuse T={T}")


def test_chain_workspace_errors():
    """A workspace below the queried size or off 256-byte alignment is
    refused before any launch; no workspace selects the tile kernel."""
    N, lib = _lib()
    B, T, NH, NKVH, Da, r = 1, 4000, 1, 1, 1, 128
    dtype = torch.bfloat16
    nbytes = _ws_bytes(dtype, B, T, NH, NKVH, Da, r)
    assert nbytes > 0
    c, ini, bias = _random_case(B, T, NH, NKVH, Da, r, seed=1, io="bf16")
    cd, idv, bd = to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV), to_torch(bias, torch.float32, DEV)
    small = _zero_ws(nbytes - 512)
    with pytest.raises(RuntimeError, match="workspace too small"):
        _forward(cd, idv, bd, NH, NKVH, Da, r, True, small[: nbytes - 512])
    big = _zero_ws(nbytes + 256)
    with pytest.raises(RuntimeError, match="256-byte aligned"):
        _forward(cd, idv, bd, NH, NKVH, Da, r, True, big[16:])
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(small)) == 0 and int(torch.count_nonzero(big)) == 0


def test_chain_combined_layout():
    """ltv_hm_scan_forward_ws on the reference's combined (B, T, F) layout,
    where every head's values start on a 16-byte boundary (D + Da = 136
    columns): the chained kernel runs (a short workspace is refused) and is
    exact on the integer generators."""
    N, lib = _lib()
    B, T, NH, NKVH, Da, r = 2, 4000, 1, 1, 8, 16
    D = Da * r
    dtype = torch.bfloat16
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, False)
    eq, ek, ev = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, False, "bf16")
    comb, idv = to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV)
    bd = to_torch(bias, torch.float32, DEV)
    nbytes = _ws_bytes(dtype, B, T, NH, NKVH, Da, r)

    def run(ws, nb):
        out = _outs(B, T, NH, NKVH, D, dtype)
        rc = lib.ltv_hm_scan_forward_ws(
            N.dtype_code(dtype), comb.data_ptr(), _s(comb), idv.data_ptr(), _s(idv),
            bd.data_ptr(), out[0].data_ptr(), _s(out[0]), out[1].data_ptr(), _s(out[1]),
            out[2].data_ptr(), _s(out[2]), ws.data_ptr(), nb, B, T, NH, NKVH, Da, r, 0,
            N.stream_of(comb))
        N.check(rc, "ltv_hm_scan_forward_ws")
        return out

    ws = _zero_ws(nbytes)
    with pytest.raises(RuntimeError, match="workspace too small"):
        run(ws, nbytes - 8)
    q, k, v = run(ws, nbytes)
    assert_close(np_of(q), eq, 0, "q combined")
    assert_close(np_of(k), ek, 0, "k combined")
    assert_close(np_of(v), ev, 0, "v combined")
    _check_ws_clean(ws, "combined")


def test_chain_config5_prefill_vs_tile():
    """configs[4]'s prefill (B = 8, T = 8192, 18 heads of 128, r = 128, bf16,
    decay sigmoid(z), z ~ N(3, 1.5)): the chained kernel (16 chunks per
    sequence, 4,608 workgroups) against the oracle on two batch rows and
    against the tile kernel everywhere."""
    N, lib = _lib()
    B, T, NH, NKVH, D = 8, 8192, 6, 6, 128
    H = NH + 2 * NKVH
    g = torch.Generator().manual_seed(11)
    comb = torch.empty(B, T, H, D + 1)
    comb[..., :D] = torch.randn(B, T, H, D, generator=g)
    comb[..., D] = -(3.0 + 1.5 * torch.randn(B, T, H, generator=g))
    comb = comb.reshape(B, T, H * (D + 1)).to(torch.bfloat16)
    inits = (0.5 * torch.randn(B, H, D, generator=g)).to(torch.bfloat16)
    bias = torch.zeros(H, 1)
    cd, idv, bd = comb.to(DEV), inits.to(DEV), bias.to(DEV)
    ws = _zero_ws(_ws_bytes(torch.bfloat16, B, T, NH, NKVH, 1, D))
    chain = _forward(cd, idv, bd, NH, NKVH, 1, D, True, ws)
    tile = _forward(cd, idv, bd, NH, NKVH, 1, D, True)
    for a, b in zip(chain, tile):
        _assert_same_up_to_association(a, b, torch.bfloat16, "config5 prefill chained vs tile")
    got = torch.cat(chain, dim=1)
    for b in (0, 5):
        eq, ek, ev = O.scan_forward(comb[b:b + 1].float().numpy(), inits[b:b + 1].float().numpy(),
                                    bias.numpy(), NH, NKVH, 1, D, True, "bf16")
        want = np.concatenate([eq, ek, ev], axis=1)[0]
        assert_close(np_of(got[b]), want, 2e-2, f"config5 prefill chained b={b}")
    _check_ws_clean(ws, "config5 prefill")


def test_chain_graph_replays_match_eager():
    """The fast path's scan forward (chained, workspace from the graph's pool)
    captured in a HIP graph: every replay equals the eager result, with eager
    work and synchronisation between replays."""
    from nanochat_amd.ops import ltv_hm_fast as F_
    B, T, NH, NKVH, D = 2, 4000, 2, 1, 128
    H = NH + 2 * NKVH
    assert _ws_bytes(torch.bfloat16, B, T, NH, NKVH, 1, D) > 0
    g = torch.Generator().manual_seed(3)
    values = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(DEV)
    logits = (-(2.0 + torch.randn(B, T, H, generator=g))).to(torch.bfloat16).to(DEV)
    inits = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV)
    bias = torch.zeros(H, 1, device=DEV)
    eager = F_.scan_forward(values, logits, inits, bias, NH, NKVH, 1, D, True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        F_.scan_forward(values, logits, inits, bias, NH, NKVH, 1, D, True)  # warm-up
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = F_.scan_forward(values, logits, inits, bias, NH, NKVH, 1, D, True)
    for i in range(3):
        for o in outs:
            o.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b), f"replay {i}"
        # eager work between the replays, on the same buffers' stream
        again = F_.scan_forward(values, logits, inits, bias, NH, NKVH, 1, D, True)
        for a, b in zip(again, eager):
            assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# chained backward (ltv_hm_look_back_scan_backward_split_ws /
# ltv_hm_scan_backward_ws): one tile-long chunk per workgroup, last chunk
# first, the gradient carry handed backwards through the same kind of
# zero-invariant workspace
# ---------------------------------------------------------------------------
def _bwd_ws_bytes(dtype, B, T, NH, NKVH, Da, r):
    N, lib = _lib()
    return lib.ltv_hm_scan_backward_chain_workspace_size(N.dtype_code(dtype), B, T, NH, NKVH,
                                                         Da, r)


def _backward(comb, ini, bias, outs, grads, NH, NKVH, Da, r, sig, ws=None):
    """Scan backward of the split layout through the C ABI: the chained kernel
    with a chain workspace tensor, the tile kernels (with their chunk-map
    passes below 256 sequences) without one.  Returns grad_values
    (B, H, T, D), grad_logits (B, H, T, Da), grad_inits (B, H, D) and
    grad_logit_bias (H, Da)."""
    N, lib = _lib()
    B, T, _ = comb.shape
    H, D = NH + 2 * NKVH, Da * r
    dt = N.dtype_code(comb.dtype)
    values, logits = _split(comb, NH, NKVH, Da, r)
    nan = float("nan")
    gval = torch.full((B, H, T, D), nan, dtype=comb.dtype, device=DEV)
    glog = torch.full((B, H, T, Da), nan, dtype=comb.dtype, device=DEV)
    gini = torch.full((B, H, D), nan, dtype=comb.dtype, device=DEV)
    gbias = torch.full((H, Da), nan, dtype=torch.float32, device=DEV)
    nbytes = lib.ltv_hm_look_back_scan_backward_workspace_size(dt, B, T, NH, NKVH, Da, r,
                                                               UNBOUNDED_P, 1, 1)
    scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
    head = [dt, values.data_ptr(), _s(values), logits.data_ptr(), _s(logits), ini.data_ptr(),
            _s(ini)]
    rest = [bias.data_ptr()]
    for t in list(outs) + list(grads):
        rest += [t.data_ptr(), _s(t)]
    rest += [gval.data_ptr(), _s(gval), glog.data_ptr(), _s(glog)]
    rest2 = [gini.data_ptr(), _s(gini), gbias.data_ptr(), scratch.data_ptr(), nbytes]
    tail = [B, T, NH, NKVH, Da, r, UNBOUNDED_P, 1, 1, int(sig), N.stream_of(comb)]
    if ws is None:
        rc = lib.ltv_hm_look_back_scan_backward_split(*head, *rest, *rest2, *tail)
    else:
        rc = lib.ltv_hm_look_back_scan_backward_split_ws(*head, dt, *rest, 0, *rest2,
                                                         ws.data_ptr(), ws.numel(), *tail)
    N.check(rc, "scan backward")
    return gval, glog, gini, gbias


def _expected_backward(c, ini, bias, outs, gy, NH, NKVH, Da, r, sig, io):
    """The oracle's backward from the given saved outputs, in the split
    layout: (grad_values (B, H, T, D), grad_logits (B, H, T, Da), grad_inits,
    grad_logit_bias)."""
    H, D = NH + 2 * NKVH, Da * r
    B, T = c.shape[:2]
    gc, gi, gb = O.scan_backward(c, ini, bias, *outs, gy[:, :NH], gy[:, NH:NH + NKVH],
                                 gy[:, NH + NKVH:H], NH, NKVH, Da, r, sig, io)
    x = gc.reshape(B, T, H, D + Da).transpose(0, 2, 1, 3)
    return x[..., :D], x[..., D:], gi, gb


def _torch_grads(gy, NH, NKVH, dtype):
    """Upstream gradients (B, H, T, D) as the (B, T, nh, D)-contiguous views a
    caller's transposes hand the scan."""
    H = gy.shape[1]
    out = []
    for lo, hi in ((0, NH), (NH, NH + NKVH), (NH + NKVH, H)):
        g = to_torch(np.ascontiguousarray(gy[:, lo:hi].transpose(0, 2, 1, 3)), dtype, DEV)
        out.append(g.transpose(1, 2))
    return out


# chained-eligible shapes: several chunks (64 steps in bf16, 32 in fp32 at
# 128 channels), ragged tails, one gate per head, gate groups of 16 channels,
# and per-channel gates (r = 1)
BWD_CASES = [
    # (B, T, NH, NKVH, Da, r)
    (2, 65, 2, 1, 1, 128),
    (2, 300, 2, 1, 1, 128),
    (1, 1537, 1, 1, 1, 128),
    (1, 4133, 1, 1, 8, 16),
    (2, 700, 1, 1, 64, 1),
    (1, 129, 1, 0, 128, 1),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("B,T,NH,NKVH,Da,r", BWD_CASES)
def test_chain_backward_exact_integer(dtype, B, T, NH, NKVH, Da, r):
    """The reference's integer generators without the sigmoid, upstream
    gradients of ones (its own backward check): every gradient exact, the
    dbias sums included (integers below 2^24), across chunk hand-offs."""
    nbytes = _bwd_ws_bytes(dtype, B, T, NH, NKVH, Da, r)
    assert nbytes > 0, "the chained backward should apply to this shape"
    io = io_name(dtype)
    H, D = NH + 2 * NKVH, Da * r
    c = int_combined(B, T, NH, NKVH, Da, r)
    ini = int_inits(B, NH, NKVH, Da, r)
    bias = int_logit_bias(NH, NKVH, Da, False)
    outs = O.scan_forward(c, ini, bias, NH, NKVH, Da, r, False, io)
    gy = np.ones((B, H, T, D), np.float32)
    want = _expected_backward(c, ini, bias, outs, gy, NH, NKVH, Da, r, False, io)
    ws = _zero_ws(nbytes)
    got = _backward(to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV),
                    to_torch(bias, torch.float32, DEV), [to_torch(o, dtype, DEV) for o in outs],
                    _torch_grads(gy, NH, NKVH, dtype), NH, NKVH, Da, r, False, ws)
    case = f"T={T} Da={Da} r={r}"
    for name, g, w in zip(("grad_values", "grad_logits", "grad_inits", "grad_logit_bias"),
                          got, want):
        assert_close(np_of(g), w, 0, f"{name} {case}")
    _check_ws_clean(ws, case)


@pytest.mark.parametrize("dtype", DTYPES, ids=io_name)
@pytest.mark.parametrize("B,T,NH,NKVH,Da,r", BWD_CASES)
def test_chain_backward_sigmoid_vs_oracle_and_tile(dtype, B, T, NH, NKVH, Da, r):
    """Sigmoid gates, decay sigmoid(N(2, 1)), random upstream gradients:
    within the tolerance of the oracle; against the tile kernels (chunk-map
    carries at these sequence counts: another association of the same fp32
    recurrence) within one bf16 rounding step or 1e-5 in fp32; three calls on
    one workspace bitwise equal."""
    io = io_name(dtype)
    H, D = NH + 2 * NKVH, Da * r
    c, ini, bias = _random_case(B, T, NH, NKVH, Da, r, seed=T * 5 + r, io=io)
    gy = O.round_io(np.random.default_rng(T).standard_normal((B, H, T, D)).astype(np.float32),
                    io)
    cd, idv, bd = to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV), to_torch(bias, torch.float32, DEV)
    outs = _forward(cd, idv, bd, NH, NKVH, Da, r, True)
    grads = _torch_grads(gy, NH, NKVH, dtype)
    want = _expected_backward(c, ini, bias, [np_of(o) for o in outs], gy, NH, NKVH, Da, r, True,
                              io)
    ws = _zero_ws(_bwd_ws_bytes(dtype, B, T, NH, NKVH, Da, r))
    runs = [_backward(cd, idv, bd, outs, grads, NH, NKVH, Da, r, True, ws) for _ in range(3)]
    for run in runs[1:]:
        for a, b in zip(runs[0], run):
            assert torch.equal(a, b)
    tol = TOL[dtype]
    case = f"T={T} Da={Da} r={r}"
    names = ("grad_values", "grad_logits", "grad_inits", "grad_logit_bias")
    for name, g, w in zip(names, runs[0], want):
        assert_close(np_of(g), w, tol, f"{name} {case}")
    tile = _backward(cd, idv, bd, outs, grads, NH, NKVH, Da, r, True)
    for name, a, b, w in zip(names, runs[0], tile, want):
        assert_close(np_of(b), w, tol, f"tile {name} {case}")
        _assert_same_up_to_association(a, b, dtype if name != "grad_logit_bias" else torch.float32,
                                       f"chained vs tile {name} {case}")
    _check_ws_clean(ws, case)


def test_chain_backward_bitwise_equals_unchunked_tile():
    """fp32 I/O at T = 64 (72 (b, h) sequences of heads of 128, r = 16): the
    chained kernel runs two 32-step chunks, the tile kernel one unchunked pass
    (no chunk-map carries up to 64 steps), both with 4 steps per lane, and the
    chained carries are composed in the tile loop's order -- so grad_values,
    grad_logits and grad_inits are bitwise equal; grad_logit_bias sums
    per-chunk partials instead of per-sequence ones (rel. 1e-5)."""
    B, T, NH, NKVH, Da, r = 4, 64, 6, 6, 8, 16
    dtype = torch.float32
    H, D = NH + 2 * NKVH, Da * r
    assert _bwd_ws_bytes(dtype, B, T, NH, NKVH, Da, r) > 0
    c, ini, bias = _random_case(B, T, NH, NKVH, Da, r, seed=16, io="f32")
    gy = np.random.default_rng(7).standard_normal((B, H, T, D)).astype(np.float32)
    cd, idv, bd = to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV), to_torch(bias, torch.float32, DEV)
    outs = _forward(cd, idv, bd, NH, NKVH, Da, r, True)
    grads = _torch_grads(gy, NH, NKVH, dtype)
    ws = _zero_ws(_bwd_ws_bytes(dtype, B, T, NH, NKVH, Da, r))
    chain = _backward(cd, idv, bd, outs, grads, NH, NKVH, Da, r, True, ws)
    tile = _backward(cd, idv, bd, outs, grads, NH, NKVH, Da, r, True)
    for name, a, b in zip(("grad_values", "grad_logits", "grad_inits"), chain[:3], tile[:3]):
        assert torch.equal(a, b), name
    assert torch.allclose(chain[3], tile[3], rtol=1e-5, atol=1e-5 * float(tile[3].abs().max()))
    _check_ws_clean(ws, "fp32 T = 64")


def test_chain_backward_workspace_errors():
    """A chain workspace below the queried size or off 256-byte alignment is
    refused before any launch and left untouched."""
    B, T, NH, NKVH, Da, r = 1, 2000, 1, 1, 1, 128
    dtype = torch.bfloat16
    H, D = NH + 2 * NKVH, Da * r
    nbytes = _bwd_ws_bytes(dtype, B, T, NH, NKVH, Da, r)
    c, ini, bias = _random_case(B, T, NH, NKVH, Da, r, seed=2, io="bf16")
    cd, idv, bd = to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV), to_torch(bias, torch.float32, DEV)
    outs = _forward(cd, idv, bd, NH, NKVH, Da, r, True)
    grads = _torch_grads(np.ones((B, H, T, D), np.float32), NH, NKVH, dtype)
    small = _zero_ws(nbytes - 512)
    with pytest.raises(RuntimeError, match="workspace too small"):
        _backward(cd, idv, bd, outs, grads, NH, NKVH, Da, r, True, small[: nbytes - 512])
    big = _zero_ws(nbytes + 256)
    with pytest.raises(RuntimeError, match="256-byte aligned"):
        _backward(cd, idv, bd, outs, grads, NH, NKVH, Da, r, True, big[16:])
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(small)) == 0 and int(torch.count_nonzero(big)) == 0


def test_chain_forward_and_backward_share_one_workspace():
    """The fast path's per-stream buffer serves the chained forward and the
    chained backward in turn: a filter step (B = 2, T = 4000, d12 heads)
    through the module's autograd, twice, bitwise equal, the buffer zeroed
    after each."""
    from nanochat_amd import _native as N
    from nanochat_amd.ops import ltv_hm_fast as F_
    B, T, NH, NKVH, D, C = 2, 4000, 2, 1, 128, 256
    H = NH + 2 * NKVH
    assert _ws_bytes(torch.bfloat16, B, T, NH, NKVH, 1, D) > 0
    assert _bwd_ws_bytes(torch.bfloat16, B, T, NH, NKVH, 1, D) > 0
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, T, C, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(H * (D + 1), C, generator=g) * C ** -0.5).to(DEV)
    inits = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV)
    bias = torch.zeros(H, 1, device=DEV)
    dq = torch.randn(B, NH, T, D, generator=g).to(torch.bfloat16).to(DEV)
    dk = torch.randn(B, NKVH, T, D, generator=g).to(torch.bfloat16).to(DEV)
    dv = torch.randn(B, NKVH, T, D, generator=g).to(torch.bfloat16).to(DEV)

    def step():
        xs, ws_, bs = (t.detach().clone().requires_grad_(True) for t in (x, w, bias))
        q, k, v, *_ = F_.qkv_filter(xs, ws_, inits, bs, NH, NKVH, 1, D)
        torch.autograd.backward([q, k, v], [dq, dk, dv])
        return q, xs.grad, ws_.grad, bs.grad

    first, second = step(), step()
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    torch.cuda.synchronize()
    for buf in N._CHAIN_WS.values():
        assert int(torch.count_nonzero(buf)) == 0


def test_chain_backward_graph_replays_match_eager():
    """The fast path's scan backward (chained, chain workspace from the
    graph's pool) captured in a HIP graph: every replay equals the eager
    result, with eager work and synchronisation between replays."""
    from nanochat_amd.ops import ltv_hm_fast as F_
    B, T, NH, NKVH, D = 2, 3000, 2, 1, 128
    H = NH + 2 * NKVH
    g = torch.Generator().manual_seed(5)
    values = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(DEV)
    logits = (-(2.0 + torch.randn(B, T, H, generator=g))).to(torch.bfloat16).to(DEV)
    inits = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV)
    bias = torch.zeros(H, 1, device=DEV)
    gys = [torch.randn(B, nh, T, D, generator=g).to(torch.bfloat16).to(DEV) for nh in (NH, NKVH, NKVH)]
    hq, hk, hv = F_.scan_forward(values, logits, inits, bias, NH, NKVH, 1, D, True)
    Fp = F_.packed_width(H, D, 1)

    def run(gc):
        return F_.scan_backward(values, logits, inits, bias, hq, hk, hv, *gys, NH, NKVH, 1, D,
                                True, gc)

    gc_eager = torch.zeros(B, T, Fp, dtype=torch.bfloat16, device=DEV)
    gi_eager, gb_eager = run(gc_eager)
    gc = torch.zeros_like(gc_eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(gc)  # warm-up
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gi, gb = run(gc)
    F = H * (D + 1)
    for i in range(3):
        gc.zero_()
        gi.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gc[..., :F], gc_eager[..., :F]), f"replay {i}"
        assert torch.equal(gi, gi_eager) and torch.equal(gb, gb_eager), f"replay {i}"
        # eager work between the replays
        gc2 = torch.zeros_like(gc_eager)
        gi2, gb2 = run(gc2)
        assert torch.equal(gc2[..., :F], gc_eager[..., :F]) and torch.equal(gi2, gi_eager)


# ---------------------------------------------------------------------------
# Failure handling.  The host forces the failure: ltv_chain_set_test_controls
# bounds every carry wait at a few polls and makes the chained launches
# publish no carry, so every wait of a chunk after a sequence's first runs out
# and every kernel still exits normally.
# ---------------------------------------------------------------------------
@pytest.fixture
def forced_chain_timeouts():
    """Yields a switch for forced carry-wait timeouts: on = 16 polls per wait
    and no carry published; off = the defaults; an int n = n polls per wait
    with carries published.  Restores the default controls, drains the error
    mailbox and drops the cached chain workspaces afterwards."""
    N, lib = _lib()

    def switch(on):
        spin, nopub = (on, 0) if type(on) is int else ((16, 1) if on else (0, 0))
        N.check(lib.ltv_chain_set_test_controls(spin, nopub), "ltv_chain_set_test_controls")

    try:
        yield switch
    finally:
        switch(False)
        torch.cuda.synchronize()
        lib.ltv_chain_take_error()
        N._CHAIN_WS.clear()


def _fast_inputs(B, T, NH, NKVH, D, seed):
    H = NH + 2 * NKVH
    g = torch.Generator().manual_seed(seed)
    values = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).to(DEV)
    logits = (-(2.0 + torch.randn(B, T, H, generator=g))).to(torch.bfloat16).to(DEV)
    inits = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV)
    bias = torch.zeros(H, 1, device=DEV)
    return values, logits, inits, bias


def test_chain_failure_reported_through_the_abi(forced_chain_timeouts):
    """A chained forward whose waits run out reports code 1 in the
    workspace's error word and in the host mailbox (read once, then clear);
    with the controls back to normal and the workspace re-zeroed (what the
    header asks after an error), the next launch is bitwise the healthy
    result."""
    N, lib = _lib()
    B, T, NH, NKVH, Da, r = 2, 4100, 1, 1, 1, 128
    dtype = torch.bfloat16
    nbytes = _ws_bytes(dtype, B, T, NH, NKVH, Da, r)
    assert nbytes > 0
    c, ini, bias = _random_case(B, T, NH, NKVH, Da, r, seed=11, io="bf16")
    cd, idv, bd = to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV), to_torch(bias, torch.float32, DEV)
    ws = _zero_ws(nbytes)
    assert lib.ltv_chain_take_error() == 0
    good = _forward(cd, idv, bd, NH, NKVH, Da, r, True, ws)
    torch.cuda.synchronize()
    assert lib.ltv_chain_take_error() == 0
    forced_chain_timeouts(True)
    _forward(cd, idv, bd, NH, NKVH, Da, r, True, ws)
    torch.cuda.synchronize()
    assert int(ws.view(torch.int32)[1]) == 1, "error word"
    assert lib.ltv_chain_take_error() == 1
    assert lib.ltv_chain_take_error() == 0, "the mailbox is cleared by a read"
    forced_chain_timeouts(False)
    ws.zero_()
    again = _forward(cd, idv, bd, NH, NKVH, Da, r, True, ws)
    torch.cuda.synchronize()
    assert lib.ltv_chain_take_error() == 0
    for a, b in zip(again, good):
        assert torch.equal(a, b)
    _check_ws_clean(ws, "after recovery")


@pytest.mark.parametrize("sync_check", [True, False], ids=["sync", "deferred"])
def test_chain_forward_failure_raises_and_recovers(forced_chain_timeouts, monkeypatch, sync_check):
    """Through the fast path's op: with LTV_CHAIN_SYNC_CHECK=1 the failing
    call raises; without it the next chained call raises.  Either way the
    cached workspace is dropped and the call after that is bitwise the
    healthy result."""
    from nanochat_amd.ops import ltv_hm_fast as F_
    N, lib = _lib()
    monkeypatch.setenv("LTV_CHAIN_SYNC_CHECK", "1" if sync_check else "0")
    B, T, NH, NKVH, D = 2, 4100, 1, 1, 128
    values, logits, inits, bias = _fast_inputs(B, T, NH, NKVH, D, seed=12)
    assert N.chain_workspace_for(values.dtype, values.device, B, T, NH, NKVH, 1, D).nbytes > 0

    def run():
        return F_.scan_forward(values, logits, inits, bias, NH, NKVH, 1, D, True)

    good = run()
    forced_chain_timeouts(True)
    if sync_check:
        with pytest.raises(RuntimeError, match=r"chained LTV scan failed \(code 1"):
            run()
        forced_chain_timeouts(False)
    else:
        run()  # fails on the device, reported later
        torch.cuda.synchronize()
        forced_chain_timeouts(False)
        with pytest.raises(RuntimeError, match=r"chained LTV scan failed \(code 1"):
            run()
    assert not N._CHAIN_WS, "the chain workspaces are dropped after an error"
    again = run()
    torch.cuda.synchronize()
    for a, b in zip(again, good):
        assert torch.equal(a, b)
    for buf in N._CHAIN_WS.values():
        assert int(torch.count_nonzero(buf)) == 0


def test_chain_backward_failure_raises_and_recovers(forced_chain_timeouts, monkeypatch):
    """The chained backward under forced timeouts: the op raises (sync
    check), and the next backward is bitwise the healthy one."""
    from nanochat_amd.ops import ltv_hm_fast as F_
    N, lib = _lib()
    monkeypatch.setenv("LTV_CHAIN_SYNC_CHECK", "1")
    B, T, NH, NKVH, D = 2, 3000, 2, 1, 128
    H = NH + 2 * NKVH
    values, logits, inits, bias = _fast_inputs(B, T, NH, NKVH, D, seed=13)
    assert N.chain_workspace_for(values.dtype, values.device, B, T, NH, NKVH, 1, D,
                                 backward=True).nbytes > 0
    g = torch.Generator().manual_seed(14)
    gys = [torch.randn(B, nh, T, D, generator=g).to(torch.bfloat16).to(DEV) for nh in (NH, NKVH, NKVH)]
    hq, hk, hv = F_.scan_forward(values, logits, inits, bias, NH, NKVH, 1, D, True)
    Fp = F_.packed_width(H, D, 1)
    F = H * (D + 1)

    def run():
        gc = torch.zeros(B, T, Fp, dtype=torch.bfloat16, device=DEV)
        gi, gb = F_.scan_backward(values, logits, inits, bias, hq, hk, hv, *gys, NH, NKVH, 1, D,
                                  True, gc)
        return gc[..., :F], gi, gb

    good = run()
    forced_chain_timeouts(True)
    with pytest.raises(RuntimeError, match=r"chained LTV scan failed \(code 1"):
        run()
    forced_chain_timeouts(False)
    again = run()
    torch.cuda.synchronize()
    for a, b in zip(again, good):
        assert torch.equal(a, b)
    for buf in N._CHAIN_WS.values():
        assert int(torch.count_nonzero(buf)) == 0


def test_chain_late_carries_leave_no_stale_words(forced_chain_timeouts):
    """Waits bounded at one poll while every chunk still publishes: readers
    that give up before their carry lands mark the word abandoned, and the
    late publisher clears it, so the workspace is all zero after every call
    whether or not a wait ran out; a call whose waits all succeeded is
    bitwise the healthy result, one with a timeout reports code 1."""
    N, lib = _lib()
    B, T, NH, NKVH, Da, r = 1, 8200, 1, 1, 1, 128
    dtype = torch.bfloat16
    nbytes = _ws_bytes(dtype, B, T, NH, NKVH, Da, r)
    assert nbytes > 0
    c, ini, bias = _random_case(B, T, NH, NKVH, Da, r, seed=15, io="bf16")
    cd, idv, bd = to_torch(c, dtype, DEV), to_torch(ini, dtype, DEV), to_torch(bias, torch.float32, DEV)
    ws = _zero_ws(nbytes)
    good = _forward(cd, idv, bd, NH, NKVH, Da, r, True, ws)
    torch.cuda.synchronize()
    assert lib.ltv_chain_take_error() == 0
    forced_chain_timeouts(1)
    codes = []
    for i in range(6):
        out = _forward(cd, idv, bd, NH, NKVH, Da, r, True, ws)
        torch.cuda.synchronize()
        code = lib.ltv_chain_take_error()
        codes.append(code)
        assert code in (0, 1), code
        nz = int(torch.count_nonzero(ws[256:]))
        assert nz == 0, f"call {i}: {nz} nonzero carry-word bytes (code {code})"
        assert int(ws.view(torch.int32)[0]) == 0, f"call {i}: ticket counter"
        if code == 0:
            for a, b in zip(out, good):
                assert torch.equal(a, b)
        ws.zero_()  # the error word (header) after a reported error
    print(f"error codes with 1-poll waits: {codes}")


_CAPTURE_FIRST = r"""
import sys
import torch
from nanochat_amd import _native as N
from nanochat_amd.ops import ltv_hm_fast as F_

B, T, NH, NKVH, D = 2, 4100, 1, 1, 128
H = NH + 2 * NKVH
g = torch.Generator().manual_seed(16)
values = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16).cuda()
logits = (-(2.0 + torch.randn(B, T, H, generator=g))).to(torch.bfloat16).cuda()
inits = torch.randn(B, H, D, generator=g).to(torch.bfloat16).cuda()
bias = torch.zeros(H, 1, device="cuda")
run = lambda: F_.scan_forward(values, logits, inits, bias, NH, NKVH, 1, D, True)
assert N.chain_workspace_for(values.dtype, values.device, B, T, NH, NKVH, 1, D).nbytes > 0
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the process's first chained launch
    outs = run()
print("captured", flush=True)
for o in outs:
    o.fill_(0)
graph.replay()
torch.cuda.synchronize()
eager = run()
torch.cuda.synchronize()
for a, b in zip(outs, eager):
    assert torch.equal(a, b), "replay differs from eager"
assert N.lib().ltv_chain_take_error() == 0
# the eager launch allocated the mailbox: a forced failure now reaches it
N.check(N.lib().ltv_chain_set_test_controls(16, 1), "controls")
try:
    run()
except RuntimeError as e:
    assert "code 1" in str(e), e
else:
    sys.exit("a forced chain failure after capture was not reported")
N.check(N.lib().ltv_chain_set_test_controls(0, 0), "controls")
again = run()
torch.cuda.synchronize()
for a, b in zip(again, eager):
    assert torch.equal(a, b), "recovery differs from eager"
print("capture-first ok", flush=True)
"""


def test_chain_first_launch_under_capture():
    """In a fresh process whose first chained launch is made under HIP graph
    capture (no eager warm-up): the capture succeeds (the library does not
    allocate its error mailbox then), a replay equals the eager result, and
    the first eager launch afterwards sets the mailbox up, so a forced
    failure is reported through it."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, LTV_CHAIN_SYNC_CHECK="1",
               PYTHONPATH=os.pathsep.join([os.path.join(root, "nanochat-filter_amd"), root,
                                           os.environ.get("PYTHONPATH", "")]))
    p = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST], env=env, capture_output=True,
                       text=True, timeout=100)
    assert p.returncode == 0, f"rc={p.returncode}\n{p.stdout}\n{p.stderr[-3000:]}"
    assert "capture-first ok" in p.stdout
