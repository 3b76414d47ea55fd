"""GPU parity of the look-back filter modules (projection + chunked scan) and
of the KV-cache path, against the oracle.

* bf16 through this package's ops takes the fused path (MFMA projection into
  the head-major layout, look-back scan, fused backward): q, k, v and every
  gradient against the oracle composition, tolerance 2e-2;
* fp32 runs the reference dataflow (fused_linear_transpose, then the op on the
  transposed view): tolerance 1e-4;
* through ``LtvLookBackQkvComputerModule`` and a ``KVCache`` (the reference's
  ``advance_kv_cache`` protocol, ``ltv_look_back_qkv_computer_module.py:15-165``)
  feeding tokens whole, in groups, one at a time (the fused decode kernel) or
  through a prefilled copy gives the rows of the chunked scan without a cache.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import TOL, assert_close, assert_norm_rel, np_of

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _make(variant, NH, NKVH, D, r, pqk, seed=0):
    from nanochat_amd.gpt_config import ChunksAndHistory
    from nanochat_amd.ops.ltv_cuda_ops import (
        fused_linear_transpose,
        ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan as blelloch_op,
        ltv_cuda_look_back_fused_concat_head_major_register_cast_sequential_scan as seq_op,
    )
    from nanochat_amd.ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
        LtvLookBackFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Blelloch,
    )
    from nanochat_amd.ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_qkv_filter import (
        LtvLookBackFusedConcatHeadMajorRegisterCastSequentialScanQkvFilter as Sequential,
    )
    torch.manual_seed(seed)
    spec = ChunksAndHistory(*pqk)
    if variant == "blelloch":
        f = Blelloch(NH, NKVH, D, r, spec, transpose_op=fused_linear_transpose,
                     look_back_op=blelloch_op)
    else:
        f = Sequential(NH, NKVH, D, r, spec, sequential_look_back_op=seq_op)
    C = NH * D
    with torch.no_grad():
        f.c.weight.normal_(0.0, C ** -0.5)
        f.logit_bias.uniform_(-0.5, 0.5)
        f.init_param.uniform_(-0.5, 0.5)
    return f.to(DEV)


def _oracle(f, x_np, gq, gk, gv, pqk, io):
    """Projection (reference fused_linear_transpose) then the look-back scan,
    forward and backward; q/k/v and their grads as (B, T, H, D)."""
    NH, NKVH, Da, r = f.n_head, f.n_kv_head, f.num_alpha_groups, f.r
    B = x_np.shape[0]
    w = f.c.weight.detach().float().cpu().numpy()
    if io == "bf16":
        w = O.bf16_round(w)
    ini = np.broadcast_to(f.init_param.detach().float().cpu().numpy(),
                          (B,) + tuple(f.init_param.shape))
    ini = O.round_io(np.ascontiguousarray(ini), io)
    bias = f.logit_bias.detach().float().cpu().numpy()
    comb = np.ascontiguousarray(O.linear_transpose_forward(x_np, w, io).transpose(0, 2, 1))
    outs = O.look_back_forward(comb, ini, bias, NH, NKVH, Da, r, *pqk, True, io)
    t = lambda a: np.ascontiguousarray(np.asarray(a).transpose(0, 2, 1, 3))  # noqa: E731
    gc, gi, gb = O.look_back_backward(comb, ini, bias, t(gq), t(gk), t(gv), NH, NKVH, Da, r,
                                      *pqk, True, io)
    gx, gw = O.linear_transpose_backward(x_np, w, gc.transpose(0, 2, 1), io)
    return tuple(t(o) for o in outs), gx, gw, gi.sum(axis=0), gb


@pytest.mark.parametrize("variant", ["blelloch", "sequential"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("pqk", [(16, 16, 9), (64, 60, 5), (5, 2, 6)], ids=str)
def test_look_back_filter_matches_oracle(variant, dtype, pqk):
    io = "bf16" if dtype == torch.bfloat16 else "f32"
    NH, NKVH, D, r = 2, 1, 128, 128
    f = _make(variant, NH, NKVH, D, r, pqk)
    B, T, C = 2, 133, NH * D
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, C, generator=g).to(dtype)
    gq = torch.randn(B, T, NH, D, generator=g).to(dtype)
    gk = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    gv = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    xd = x.to(DEV).requires_grad_(True)
    inits = f.init_param.unsqueeze(0).expand(B, -1, -1)
    q, k, v = f(xd, inits, full_recurrence=False)
    assert q.shape == (B, T, NH, D) and q.dtype == dtype
    torch.autograd.backward([q, k, v], [gq.to(DEV), gk.to(DEV), gv.to(DEV)])
    (eq, ek, ev), egx, egw, egi, egb = _oracle(f, x.float().numpy(), gq.float().numpy(),
                                              gk.float().numpy(), gv.float().numpy(), pqk, io)
    tol = TOL[dtype]
    case = f"{variant} {io} pqk={pqk}"
    assert_close(np_of(q), eq, tol, "q " + case)
    assert_close(np_of(k), ek, tol, "k " + case)
    assert_close(np_of(v), ev, tol, "v " + case)
    assert_close(np_of(xd.grad), egx, tol, "grad_x " + case)
    assert_close(np_of(f.c.weight.grad), egw, tol, "grad_weight " + case)
    assert_close(np_of(f.init_param.grad), egi, tol, "grad_init_param " + case)
    assert_close(np_of(f.logit_bias.grad), egb, tol, "grad_logit_bias " + case)


def _cache(B, NH, NKVH, D, spec, total):
    from nanochat_amd.kv_cache import KVCache
    return KVCache(batch_size=B, num_q_heads=NH, num_kv_heads=NKVH, seq_len=total + 10,
                   head_dim=D, num_layers=1, layer_specs=[spec])


@pytest.mark.parametrize("variant", ["blelloch", "sequential"])
@pytest.mark.parametrize("pqk", [(16, 16, 9), (5, 2, 6), (0, 4, 3)], ids=str)
def test_kv_cache_groupings_match_chunked_scan(variant, pqk):
    from nanochat_amd.gpt_config import ChunksAndHistory
    from nanochat_amd.ltv_look_back_qkv_computer_module import LtvLookBackQkvComputerModule
    NH, NKVH, D, r = 2, 1, 128, 128
    f = _make(variant, NH, NKVH, D, r, pqk, seed=3)
    m = LtvLookBackQkvComputerModule(0, f)
    spec = ChunksAndHistory(*pqk)
    B = 8
    counts = [7, 1, 1, 16, 3, 1, 1, 1, 9, 2]
    total = sum(counts)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(B, total, NH * D, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        chunked = m(x, None)
        whole = m(x, _cache(B, NH, NKVH, D, spec, total))
        cache = _cache(B, NH, NKVH, D, spec, total)
        prev = _cache(B, NH, NKVH, D, spec, total)
        steps, steps3 = [], []
        start = 0
        for n in counts:
            xs = x[:, start:start + n]
            start += n
            steps.append(m(xs, cache))
            steps3.append(m(xs, prev))
            fresh = _cache(B, NH, NKVH, D, spec, total)
            fresh.prefill(prev)
            prev = fresh
    tol = TOL[torch.bfloat16]
    for i, name in enumerate("qkv"):
        ref = np_of(chunked[i])
        assert_close(np_of(whole[i]), ref, tol, f"{name} whole")
        assert_close(np_of(torch.cat([s[i] for s in steps], dim=1)), ref, tol, f"{name} steps")
        assert_close(np_of(torch.cat([s[i] for s in steps3], dim=1)), ref, tol,
                     f"{name} prefilled steps")


@pytest.mark.parametrize("pqk", [(16, 16, 9), (64, 60, 5), (32, 8, 9)], ids=str)
def test_fp32_inits_bitwise_equal_bf16_cast(pqk, monkeypatch):
    """The bf16 look-back filter hands the fp32 inits (the expanded parameter)
    to the kernels, which round them to bf16 as they read them and return the
    widened bf16 gradient: outputs and every gradient bitwise those of casting
    the inits to bf16 first (the reference's ``.to(dtype)``), with and without
    the fp32 hand-over."""
    from nanochat_amd.ops import ltv_hm_fast as F_
    NH, NKVH, D, r = 2, 1, 128, 128
    B, T = 4, 200
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, T, NH * D, generator=g).to(torch.bfloat16).to(DEV)
    gy = [torch.randn(B, T, n, D, generator=g).to(torch.bfloat16).to(DEV) for n in (NH, NKVH, NKVH)]

    def run():
        f = _make("blelloch", NH, NKVH, D, r, pqk, seed=5)
        xd = x.clone().requires_grad_(True)
        inits = f.init_param.unsqueeze(0).expand(B, -1, -1)
        q, k, v = f(xd, inits, full_recurrence=False)
        torch.autograd.backward([q, k, v], gy)
        return [q, k, v, xd.grad, f.c.weight.grad, f.init_param.grad, f.logit_bias.grad]

    assert F_.fp32_inits_ok(T, D, r, *pqk)
    fp32 = run()
    monkeypatch.setattr(F_, "fp32_inits_ok", lambda *a: False)
    cast = run()
    for name, a, b in zip(("q", "k", "v", "grad_x", "grad_weight", "grad_init_param",
                           "grad_logit_bias"), fp32, cast):
        assert torch.equal(a, b), f"{name} differs with pqk={pqk}"


@pytest.mark.parametrize("pqk", [(16, 16, 9), (64, 60, 5), (32, 8, 9), (128, 100, 5)], ids=str)
def test_shared_inits_match_expanded(pqk):
    """The (H, D) init parameter handed to the bf16 look-back filter directly
    (what the computer module does without a KV cache): q, k, v and the
    gradients of x, the weight and the logit bias bitwise those of the
    expanded (B, H, D) inits; the parameter's gradient bitwise the batch-order
    fp32 sum of the per-sequence gradients (which the library forms itself
    where the kernels take shared inits -- (128, 100, 5) does not, and is
    expanded by the filter)."""
    from nanochat_amd.ltv_look_back_qkv_computer_module import LtvLookBackQkvComputerModule
    NH, NKVH, D, r = 2, 1, 128, 128
    B, T = 5, 200
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, T, NH * D, generator=g).to(torch.bfloat16).to(DEV)
    gy = [torch.randn(B, T, n, D, generator=g).to(torch.bfloat16).to(DEV) for n in (NH, NKVH, NKVH)]

    def run(mode):
        f = _make("blelloch", NH, NKVH, D, r, pqk, seed=3)
        xd = x.clone().requires_grad_(True)
        per_seq = None
        if mode == "shared":
            q, k, v = f(xd, f.init_param, full_recurrence=False)
        elif mode == "module":
            q, k, v = LtvLookBackQkvComputerModule(0, f)(xd, None)
        else:  # per-sequence leaf inits: their (B, H, D) gradient
            per_seq = f.init_param.detach().unsqueeze(0).repeat(B, 1, 1).requires_grad_(True)
            q, k, v = f(xd, per_seq, full_recurrence=False)
        torch.autograd.backward([q, k, v], gy)
        gi = per_seq.grad if per_seq is not None else f.init_param.grad
        return [q, k, v, xd.grad, f.c.weight.grad, f.logit_bias.grad], gi

    ref, gi_seq = run("per_sequence")
    want = np.zeros(gi_seq.shape[1:], np.float32)
    for b in range(B):  # batch order, fp32
        want = (want + gi_seq[b].cpu().numpy()).astype(np.float32)
    for mode in ("shared", "module"):
        outs, gi = run(mode)
        for name, a, b in zip(("q", "k", "v", "grad_x", "grad_weight", "grad_logit_bias"),
                              outs, ref):
            assert torch.equal(a, b), f"{name} differs ({mode}, pqk={pqk})"
        got = gi.cpu().numpy()
        if pqk == (128, 100, 5):  # expanded by the filter: torch's batch reduction
            assert_close(got, want, 1e-6, f"grad_init_param ({mode})")
        else:
            assert np.array_equal(got, want), f"grad_init_param ({mode}, pqk={pqk})"


def _random_cases(n=12, seed=11):
    """Seeded look-back filter cases: chunk specs (P, Q, K) with short and long
    warm-ups, P = 0 and unbounded P, heads, head widths and gate group sizes,
    batch and sequence lengths off the kernels' tile sizes, both variants and
    both I/O dtypes; odd Blelloch cases hand over the (H, D) inits parameter."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        NH = int(rng.integers(1, 4))
        NKVH = int(rng.integers(1, NH + 1))
        D = int(rng.choice([12, 24, 32, 48, 64, 96, 128]))
        r = int(rng.choice([d for d in range(1, D + 1) if D % d == 0]))
        Q = int(rng.integers(1, 131))
        K = int(rng.integers(1, 40))
        P = O.UNBOUNDED_P if i % 5 == 4 else int(rng.choice([0, int(rng.integers(1, 200))]))
        B = int(rng.integers(1, 4))
        T = int(rng.integers(1, 301))
        variant = "blelloch" if i % 4 < 2 else "sequential"
        dtype = torch.bfloat16 if i % 2 else torch.float32
        shared = variant == "blelloch" and i % 2 == 1
        cases.append(pytest.param(variant, NH, NKVH, D, r, (P, Q, K), B, T, dtype, shared,
                                  id=f"{i}-{variant}-{'bf16' if i % 2 else 'f32'}-h{NH}.{NKVH}"
                                     f"-D{D}-r{r}-pqk{P}.{Q}.{K}-B{B}-T{T}"))
    return cases


@pytest.mark.parametrize("variant, NH, NKVH, D, r, pqk, B, T, dtype, shared", _random_cases())
def test_look_back_filter_random(variant, NH, NKVH, D, r, pqk, B, T, dtype, shared):
    io = "bf16" if dtype == torch.bfloat16 else "f32"
    f = _make(variant, NH, NKVH, D, r, pqk, seed=T)
    C = NH * D
    g = torch.Generator().manual_seed(B * 1000 + T)
    x = torch.randn(B, T, C, generator=g).to(dtype)
    gq = torch.randn(B, T, NH, D, generator=g).to(dtype)
    gk = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    gv = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    xd = x.to(DEV).requires_grad_(True)
    inits = f.init_param if shared else f.init_param.unsqueeze(0).expand(B, -1, -1)
    q, k, v = f(xd, inits, full_recurrence=False)
    torch.autograd.backward([q, k, v], [gq.to(DEV), gk.to(DEV), gv.to(DEV)])
    (eq, ek, ev), egx, egw, egi, egb = _oracle(f, x.float().numpy(), gq.float().numpy(),
                                              gk.float().numpy(), gv.float().numpy(), pqk, io)
    tol = TOL[dtype]
    for name, got, want in (("q", q, eq), ("k", k, ek), ("v", v, ev), ("grad_x", xd.grad, egx),
                            ("grad_weight", f.c.weight.grad, egw),
                            ("grad_init_param", f.init_param.grad, egi),
                            ("grad_logit_bias", f.logit_bias.grad, egb)):
        assert_close(np_of(got), want, tol, name)
        assert_norm_rel(np_of(got), want, tol, name)


@pytest.mark.parametrize("variant", ["blelloch", "sequential"])
@pytest.mark.parametrize("NH,NKVH,D,r", [(1, 1, 12, 4), (2, 1, 6, 2)])
def test_look_back_filter_shapes_outside_the_fused_path(variant, NH, NKVH, D, r):
    """bf16 with C not a multiple of 8 or D not of 4: the generic dataflow
    (projection in bf16 with the weight rounded to it, then the look-back op),
    forward and every gradient against the oracle."""
    pqk = (16, 16, 9)
    f = _make(variant, NH, NKVH, D, r, pqk, seed=D)
    B, T, C = 2, 70, NH * D
    g = torch.Generator().manual_seed(C)
    dtype = torch.bfloat16
    x = torch.randn(B, T, C, generator=g).to(dtype)
    gq = torch.randn(B, T, NH, D, generator=g).to(dtype)
    gk = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    gv = torch.randn(B, T, NKVH, D, generator=g).to(dtype)
    xd = x.to(DEV).requires_grad_(True)
    q, k, v = f(xd, f.init_param.unsqueeze(0).expand(B, -1, -1), full_recurrence=False)
    torch.autograd.backward([q, k, v], [gq.to(DEV), gk.to(DEV), gv.to(DEV)])
    (eq, ek, ev), egx, egw, egi, egb = _oracle(f, x.float().numpy(), gq.float().numpy(),
                                              gk.float().numpy(), gv.float().numpy(), pqk, "bf16")
    tol = TOL[dtype]
    for name, got, want in (("q", q, eq), ("k", k, ek), ("v", v, ev), ("grad_x", xd.grad, egx),
                            ("grad_weight", f.c.weight.grad, egw),
                            ("grad_init_param", f.init_param.grad, egi),
                            ("grad_logit_bias", f.logit_bias.grad, egb)):
        assert_close(np_of(got), want, tol, name)
        assert_norm_rel(np_of(got), want, tol, name)
