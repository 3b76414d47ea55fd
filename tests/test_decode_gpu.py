"""GPU parity of the decode (KV-cache) path: one token per sequence, no autograd.

The fused ``ltv_qkv_decode_step`` is pinned three ways:
* one step against the CPU oracle (``filter_forward`` at T = 1 from the same
  previous rows) and against the general GPU path at T = 1;
* a chain of decode steps through ``LtvCombinedQkvComputerModule`` and a KV
  cache (the reference protocol, ``ltv_combined_qkv_computer_module.py:28-41``)
  against the same chain on the general path: both carry the state as the bf16
  output row, so they agree to bf16 rounding;
* config 5's decode (B = 64, 256 steps after a prefill) against a full
  recompute of the whole sequence.  The cache holds bf16 rows, so every decode
  step re-quantises the state that the full scan keeps in fp32; with a constant
  decay a = 1 - alpha the difference is bounded by 2^-9 max|h| / alpha (the
  bound of the reference's own decode), which the test asserts; with
  data-dependent gates, by the largest per-step perturbation over the smallest
  alpha seen.
"""

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import assert_close, np_of

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2


def _make_filter(NH, NKVH, D, r, seed=0, gate_scale=1.0, bias=(-0.5, 0.5)):
    from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
        LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter,
    )
    torch.manual_seed(seed)
    f = Filter(NH, NKVH, D, r)
    C = NH * D  # the filter's input width is n_head * head_dim
    Da = D // r
    H = NH + 2 * NKVH
    assert f.c.weight.shape == (H * (D + Da), C)
    with torch.no_grad():
        f.c.weight.normal_(0.0, C ** -0.5)
        w = f.c.weight.view(H, D + Da, C)
        w[:, D:, :] *= gate_scale
        f.logit_bias.uniform_(*bias)
        f.init_param.uniform_(-0.5, 0.5)
    return f.to(DEV)


class _Cache:
    """The slice of nanochat's KV cache the filter uses (kv_cache.py:212-294)."""

    class _Slot:
        def __init__(self):
            self.special = {}

    class _Last:
        def __init__(self):
            self.q, self.k, self.v = _Cache._Slot(), _Cache._Slot(), _Cache._Slot()

    def __init__(self):
        self.last_qkv = _Cache._Last()

    def has_last_qkv(self, layer):
        return layer in self.last_qkv.q.special

    def update_last_qkv(self, layer, q, k, v):
        self.last_qkv.q.special[layer] = q
        self.last_qkv.k.special[layer] = k
        self.last_qkv.v.special[layer] = v

    def __bool__(self):
        return True


def _general_step(f, x, prev):
    """The general (autograd-capable) path at T = 1: projection GEMM + scan."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    with torch.enable_grad():
        q, k, v = f(x, prev if prev is not None else LtvInitValues())
    return q.detach(), k.detach(), v.detach()


@pytest.mark.parametrize("NH,NKVH,D,r,B", [(6, 6, 128, 128, 64), (4, 2, 128, 32, 37),
                                            (2, 1, 64, 1, 5), (3, 0, 64, 16, 33),
                                            # C = 24: not the fused step's multiple of 16, the
                                            # fused path at T = 1; C = 12, D = 6: the reference
                                            # dataflow in bf16
                                            (1, 1, 24, 24, 9), (1, 1, 12, 12, 5), (2, 1, 6, 2, 3)])
def test_decode_step_matches_oracle_and_general_path(NH, NKVH, D, r, B):
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    f = _make_filter(NH, NKVH, D, r, seed=NH + r)
    C = NH * D
    H = NH + 2 * NKVH
    Da = D // r
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, 1, C, generator=g).to(torch.bfloat16).to(DEV)
    prev_all = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV)
    prev = LtvInitValues(q=prev_all[:, :NH], k=prev_all[:, NH:NH + NKVH],
                         v=prev_all[:, NH + NKVH:])
    with torch.no_grad():
        q, k, v = f(x, prev)
    got = torch.cat([q, k, v], dim=2)[:, 0]  # (B, H, D)

    # oracle: the reference dataflow at T = 1 from the same rows, bf16 I/O
    w = O.bf16_round(f.c.weight.detach().float().cpu().numpy())
    bias = f.logit_bias.detach().float().cpu().numpy()
    ini = O.round_io(prev_all.float().cpu().numpy(), "bf16")
    eq, ek, ev, _, _ = O.filter_forward(x.float().cpu().numpy(), w, ini, bias, NH, NKVH, Da, r,
                                        "bf16")
    exp = np.concatenate([eq, ek, ev], axis=2)[:, 0]
    assert_close(np_of(got), exp, TOL, "decode vs oracle")

    gq, gk, gv = _general_step(f, x, prev)
    gen = torch.cat([gq, gk, gv], dim=2)[:, 0]
    assert_close(np_of(got), np_of(gen), TOL, "decode vs general path")


def test_decode_from_init_param_and_weight_updates():
    """Without cache rows the step starts from init_param; an in-place weight
    update (an optimizer step) invalidates the reused packed weight."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    f = _make_filter(2, 1, 128, 128, seed=3)
    x = torch.randn(9, 1, 256).to(torch.bfloat16).to(DEV)
    for _ in range(2):
        with torch.no_grad():
            got = torch.cat(f(x, LtvInitValues()), dim=2)
        gen = torch.cat(_general_step(f, x, None), dim=2)
        assert_close(np_of(got), np_of(gen), TOL, "decode from init_param")
        with torch.no_grad():
            f.c.weight.mul_(-1.5)


def test_decode_after_data_writes_and_load_state_dict():
    """A write through c.weight.data does not bump the parameter's version: the
    packed weight is refreshed by invalidate_packed_weight(); load_state_dict
    refreshes it by itself."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    f = _make_filter(2, 1, 128, 128, seed=4)
    x = torch.randn(5, 1, 256).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        f(x, LtvInitValues())  # fills the cache
    f.c.weight.data.mul_(-2.0)
    f.invalidate_packed_weight()
    with torch.no_grad():
        got = torch.cat(f(x, LtvInitValues()), dim=2)
    gen = torch.cat(_general_step(f, x, None), dim=2)
    assert_close(np_of(got), np_of(gen), TOL, "decode after a .data write")
    other = _make_filter(2, 1, 128, 128, seed=5)
    f.load_state_dict(other.state_dict())
    with torch.no_grad():
        got = torch.cat(f(x, LtvInitValues()), dim=2)
    gen = torch.cat(_general_step(other, x, None), dim=2)
    assert_close(np_of(got), np_of(gen), TOL, "decode after load_state_dict")


def _chain(module, xs, cache, fused):
    outs = []
    for t in range(xs.shape[1]):
        if fused:
            with torch.no_grad():
                q, k, v = module(xs[:, t:t + 1], cache)
        else:
            with torch.enable_grad():
                q, k, v = module(xs[:, t:t + 1], cache)
            q, k, v = q.detach(), k.detach(), v.detach()
            cache.update_last_qkv(module.layer_idx, q=q[:, -1], k=k[:, -1], v=v[:, -1])
        outs.append(torch.cat([q, k, v], dim=2))
    return torch.cat(outs, dim=1)


def test_decode_chain_matches_general_path_chain():
    from nanochat_amd.ltv_combined_qkv_computer_module import LtvCombinedQkvComputerModule
    f = _make_filter(6, 6, 128, 128, seed=5, gate_scale=1.0, bias=(-3.5, -2.5))
    m = LtvCombinedQkvComputerModule(0, f)
    g = torch.Generator().manual_seed(11)
    xs = torch.randn(16, 40, 768, generator=g).to(torch.bfloat16).to(DEV)
    ca, cb = _Cache(), _Cache()
    with torch.no_grad():
        m(xs[:, :8], ca)
        m(xs[:, :8], cb)
    fused = _chain(m, xs[:, 8:], ca, fused=True)
    general = _chain(m, xs[:, 8:], cb, fused=False)
    assert_close(np_of(fused), np_of(general), TOL, "decode chain")


def test_decode_config5_vs_full_recompute():
    """Config 5's decode: B = 64, 256 steps after a 16-token prefill, checked
    against the full sequence in one call.  Gate rows zeroed and bias -3 give a
    constant alpha = sigmoid(-3), so the bf16-state drift bound is exact."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    from nanochat_amd.ltv_combined_qkv_computer_module import LtvCombinedQkvComputerModule
    f = _make_filter(6, 6, 128, 128, seed=2, gate_scale=0.0, bias=(-3.0, -3.0))
    m = LtvCombinedQkvComputerModule(0, f)
    B, T0, N = 64, 16, 256
    g = torch.Generator().manual_seed(5)
    xs = torch.randn(B, T0 + N, 768, generator=g).to(torch.bfloat16).to(DEV)
    cache = _Cache()
    with torch.no_grad():
        m(xs[:, :T0], cache)
    dec = _chain(m, xs[:, T0:], cache, fused=True)
    with torch.no_grad():
        full = torch.cat(f(xs, LtvInitValues()), dim=2)[:, T0:]
    alpha = 1.0 / (1.0 + np.exp(3.0))
    hmax = float(full.float().abs().max())
    bound = 2.0 ** -9 * hmax / alpha
    err = (dec.float() - full.float()).abs()
    # the bound plus one bf16 rounding of the output
    assert float(err.max()) <= bound + 2.0 ** -8 * hmax, (float(err.max()), bound)
    # and the drift is far from the bound on average
    assert float(err.mean()) <= 0.25 * bound


def test_decode_config5_data_dependent_gates_vs_full_recompute():
    """Config 5's decode with data-dependent gates (gate rows at full scale,
    bias in [-3.5, -2.5]): B = 64, 256 steps after a 16-token prefill, against
    the full sequence in one call.  Per step the decode path can differ from
    the full scan by
      * the bf16 rounding of the carried state, <= 2^-8 max|h|;
      * its own projection of the new token, summed in another order than the
        GEMM's: a value or a logit can round to the neighbouring bf16 (<= 2^-7
        of it), which moves the step by <= alpha 2^-7 max|u|, and alpha by <=
        alpha (1 - alpha) 2^-7 |logit| <= 2^-9 |logit| (times |u - h|).
    Each perturbation then decays by (1 - alpha) per step, so the difference is
    bounded by the largest perturbation over the smallest alpha seen (the
    largest decay), plus one bf16 rounding of the output."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    from nanochat_amd.ltv_combined_qkv_computer_module import LtvCombinedQkvComputerModule
    from nanochat_amd.ops import ltv_hm_fast as F_
    NH, NKVH, D = 6, 6, 128
    H = NH + 2 * NKVH
    f = _make_filter(NH, NKVH, D, D, seed=3, gate_scale=1.0, bias=(-3.5, -2.5))
    m = LtvCombinedQkvComputerModule(0, f)
    B, T0, N = 64, 16, 256
    g = torch.Generator().manual_seed(6)
    xs = torch.randn(B, T0 + N, NH * D, generator=g).to(torch.bfloat16).to(DEV)
    cache = _Cache()
    with torch.no_grad():
        m(xs[:, :T0], cache)
    dec = _chain(m, xs[:, T0:], cache, fused=True)
    with torch.no_grad():
        full = torch.cat(f(xs, LtvInitValues()), dim=2)[:, T0:]
        vals, logits, _ = F_.project(xs, f.c.weight.detach(), H, D, 1)
    lg = logits[:, T0:, :H].float()
    alpha = torch.sigmoid(lg + f.logit_bias.detach().float().view(1, 1, H))
    a_min, a_max = float(alpha.min()), float(alpha.max())
    assert a_max - a_min > 0.05, "the gates should vary with the data"
    umax = float(vals[:, :, T0:].float().abs().max())
    lmax = float(lg.abs().max())
    hmax = float(full.float().abs().max())
    delta = 2.0 ** -8 * hmax + a_max * 2.0 ** -7 * umax + 2.0 ** -9 * lmax * (umax + hmax)
    bound = delta / a_min + 2.0 ** -8 * hmax
    err = (dec.float() - full.float()).abs()
    assert float(err.max()) <= bound, (float(err.max()), bound, a_min)
    assert float(err.mean()) <= 0.25 * bound, (float(err.mean()), bound)


def test_decode_writes_cache_rows_in_place():
    """Through LtvCombinedQkvComputerModule and a KVCache, the fused decode step
    stores the new last rows into the cache's row buffers itself
    (ltv_qkv_decode_step_rows): every step's q, k, v and the cache rows are
    bitwise those of the step with the module's copy (update_last_qkv), and the
    rows returned by earlier steps are never modified."""
    from nanochat_amd.gpt_config import ChunksAndHistory
    from nanochat_amd.kv_cache import KVCache
    from nanochat_amd.ltv_combined_qkv_computer_module import LtvCombinedQkvComputerModule
    f = _make_filter(6, 6, 128, 128, seed=8, gate_scale=1.0, bias=(-2.5, -1.5))
    m = LtvCombinedQkvComputerModule(0, f)
    B, T0, N = 8, 5, 12
    g = torch.Generator().manual_seed(9)
    xs = torch.randn(B, T0 + N, 768, generator=g).to(torch.bfloat16).to(DEV)

    def run(in_place):
        cache = KVCache(B, 6, 6, T0 + N, 128, 1, [ChunksAndHistory(2147483647, 1, 1)])
        if not in_place:
            f.decode_into_rows = lambda *args: None  # the module falls back to its copy
        try:
            outs, kept = [], []
            with torch.no_grad():
                m(xs[:, :T0], cache)
                for t in range(T0, T0 + N):
                    q, k, v = m(xs[:, t:t + 1], cache)
                    kept.append((q, q.clone()))
                    outs.append(torch.cat([q, k, v], dim=2))
            last = cache.last_qkv
            rows = [t.special[0].clone() for t in (last.q, last.k, last.v)]
        finally:
            if not in_place:
                del f.decode_into_rows
        for q, q0 in kept:
            assert torch.equal(q, q0), "a returned row changed after a later step"
        return torch.cat(outs, dim=1), rows

    a, rows_a = run(True)
    b, rows_b = run(False)
    assert torch.equal(a, b)
    for x, y in zip(rows_a, rows_b):
        assert torch.equal(x, y)
    assert torch.equal(rows_a[0], a[:, -1, :6])


def test_decode_into_rows_declines_rows_it_cannot_store():
    """decode_into_rows takes the fused in-place step only when every row
    buffer is bf16 on x's device with contiguous channels; for fp32 rows (a
    cache filled by an fp32 prefill) or channel-strided rows it returns None
    and writes nothing, so the module runs the general step and its own row
    update."""
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    NH, NKVH, D = 2, 1, 64
    f = _make_filter(NH, NKVH, D, D, seed=4)
    B = 3
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, 1, NH * D, generator=g).to(torch.bfloat16).to(DEV)

    def rows(dtype, strided=False):
        out = []
        for nh in (NH, NKVH, NKVH):
            if strided:
                t = torch.randn(B, nh, 2 * D, generator=g).to(dtype).to(DEV)[..., ::2]
            else:
                t = torch.randn(B, nh, D, generator=g).to(dtype).to(DEV)
            out.append(t)
        return out

    with torch.no_grad():
        for bad in (rows(torch.float32), rows(torch.bfloat16, strided=True)):
            before = [t.clone() for t in bad]
            prev = LtvInitValues(q=bad[0], k=bad[1], v=bad[2])
            assert f.decode_into_rows(x, prev, tuple(bad)) is None
            for t, t0 in zip(bad, before):
                assert torch.equal(t, t0), "declined call wrote the rows"
        good = rows(torch.bfloat16)
        prev = LtvInitValues(q=good[0].clone(), k=good[1].clone(), v=good[2].clone())
        out = f.decode_into_rows(x, prev, tuple(good))
        assert out is not None
        torch.cuda.synchronize()
        assert torch.equal(out[0][:, 0], good[0])
