"""CPU checks of the look-back filters' module layer: ``advance_kv_cache``, the
``KVCache`` state it keeps, and the filters' reference dataflow.

The filters take their projection and scan as injected ops (reference
``ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter.py:44-56``);
here they are the CPU oracle's, as the reference's own exhaustive test injects
its Python reference ops (``tests/test_look_back_advance_kv_cache_exhaustive.py:26-49``).
Checked, for both filter variants and every token grouping of short sequences:

* feeding the tokens all at once, step by step, or step by step through a
  prefilled copy of the cache gives the same rows (the reference's test);
* those rows equal the chunked scan without a cache (``full_recurrence=False``):
  the cache protocol reproduces the chunk windows exactly.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

import ltv_oracle as O
from nanochat_amd.gpt_config import UNBOUNDED_P, ChunksAndHistory
from nanochat_amd.kv_cache import KVCache
from nanochat_amd.ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
    LtvLookBackFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter,
)
from nanochat_amd.ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_qkv_filter import (
    LtvLookBackFusedConcatHeadMajorRegisterCastSequentialScanQkvFilter,
)
from nanochat_amd.ltv_look_back_qkv_computer_module import (
    LtvLookBackQkvComputerModule,
    advance_kv_cache,
)


def _oracle_transpose(x, w):
    return torch.from_numpy(O.linear_transpose_forward(x.detach().numpy(), w.detach().numpy(),
                                                       "f32"))


def _oracle_look_back(combined, inits, logit_bias, NH, NKVH, da, r, P, Q, K, *tuning_and_flag):
    outs = O.look_back_forward(combined.detach().numpy(), inits.detach().numpy(),
                               logit_bias.detach().numpy(), NH, NKVH, da, r, P, Q, K,
                               bool(tuning_and_flag[-1]), "f32")
    return tuple(torch.from_numpy(np.ascontiguousarray(o)) for o in outs)


def _blelloch(nh, nkvh, hd, r, spec):
    return LtvLookBackFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter(
        nh, nkvh, hd, r, spec, transpose_op=_oracle_transpose, look_back_op=_oracle_look_back)


def _sequential(nh, nkvh, hd, r, spec):
    return LtvLookBackFusedConcatHeadMajorRegisterCastSequentialScanQkvFilter(
        nh, nkvh, hd, r, spec, sequential_look_back_op=_oracle_look_back)


VARIANTS = [pytest.param(_blelloch, id="blelloch"), pytest.param(_sequential, id="sequential")]
CHUNKS = [(3, 2, 2), (5, 3, 2), (4, 2, 3), (1, 1, 1), (10, 2, 5), (2, 2, 6), (0, 2, 3),
          (UNBOUNDED_P, 1, 1)]


def _make(make_filter, p, q, k, random_weights, nh=1, nkvh=1, hd=2, r=1):
    f = make_filter(nh, nkvh, hd, r, ChunksAndHistory(p=p, q=q, k=k))
    with torch.no_grad():
        if random_weights:
            g = torch.Generator().manual_seed(p * 31 + q * 7 + k)
            f.c.weight.copy_(torch.randn(f.c.weight.shape, generator=g) * 0.5)
            f.logit_bias.copy_(torch.randn(f.logit_bias.shape, generator=g))
            f.init_param.copy_(torch.randn(f.init_param.shape, generator=g))
        else:  # the reference test's weights
            f.c.weight.fill_(1.0)
            f.logit_bias.fill_(0.0)
            f.init_param.fill_(0.0)
    return f


def _cache(B, nh, nkvh, hd, total, spec):
    return KVCache(batch_size=B, num_q_heads=nh, num_kv_heads=nkvh, seq_len=max(1, total) + 10,
                   head_dim=hd, num_layers=1, layer_specs=[spec])


@pytest.mark.parametrize("p,q,k", CHUNKS)
@pytest.mark.parametrize("make_filter", VARIANTS)
@pytest.mark.parametrize("random_weights", [False, True])
def test_advance_kv_cache_groupings_agree_with_chunked_scan(make_filter, p, q, k, random_weights):
    nh = nkvh = 1
    hd = 2
    C = nh * hd
    f = _make(make_filter, p, q, k, random_weights)
    spec = ChunksAndHistory(p=p, q=q, k=k)
    B = 1
    inits = f.init_param.unsqueeze(0).expand(B, -1, -1)
    for N, A in ((1, 3), (2, 3), (3, 3), (4, 2)):
        for counts in itertools.product(range(A), repeat=N):
            total = sum(counts)
            torch.manual_seed(42)
            x = torch.randn(1, total, C) if total else torch.empty(1, 0, C)
            with torch.no_grad():
                whole = advance_kv_cache(x, 0, f, inits, _cache(B, nh, nkvh, hd, total, spec))
                step_cache = _cache(B, nh, nkvh, hd, total, spec)
                prev = _cache(B, nh, nkvh, hd, total, spec)
                steps, steps3 = [], []
                start = 0
                for t in counts:
                    xs = x[:, start:start + t]
                    start += t
                    steps.append(advance_kv_cache(xs, 0, f, inits, step_cache))
                    steps3.append(advance_kv_cache(xs, 0, f, inits, prev))
                    fresh = _cache(B, nh, nkvh, hd, total, spec)
                    fresh.prefill(prev)
                    prev = fresh
                chunked = f(x, inits, full_recurrence=False) if total else None
            for i in range(3):
                s2 = torch.cat([s[i] for s in steps], dim=1)
                s3 = torch.cat([s[i] for s in steps3], dim=1)
                torch.testing.assert_close(whole[i], s2)
                torch.testing.assert_close(whole[i], s3)
                if chunked is not None:
                    torch.testing.assert_close(whole[i], chunked[i])


def test_computer_module_uses_chunked_scan_without_cache_and_advances_with_one():
    spec = ChunksAndHistory(p=4, q=3, k=3)
    f = _make(_blelloch, 4, 3, 3, True, nh=2, nkvh=1, hd=4, r=2)
    m = LtvLookBackQkvComputerModule(0, f)
    torch.manual_seed(0)
    x = torch.randn(2, 11, 8)
    with torch.no_grad():
        q, k, v = m(x, None)
        cache = _cache(2, 2, 1, 4, 11, spec)
        parts = [m(x[:, a:b], cache) for a, b in ((0, 5), (5, 6), (6, 11))]
    assert q.shape == (2, 11, 2, 4) and k.shape == (2, 11, 1, 4) and v.shape == (2, 11, 1, 4)
    for i, ref in enumerate((q, k, v)):
        torch.testing.assert_close(torch.cat([p[i] for p in parts], dim=1), ref)
    # the oracle's chunked scan of the projected input, directly
    combined = O.linear_transpose_forward(x.numpy(), f.c.weight.detach().numpy(), "f32")
    inits = np.broadcast_to(f.init_param.detach().numpy(), (2, 4, 4))
    eq, ek, ev = O.look_back_forward(np.ascontiguousarray(combined.transpose(0, 2, 1)), inits,
                                     f.logit_bias.detach().numpy(), 2, 1, 2, 2, 4, 3, 3, True)
    np.testing.assert_allclose(q.numpy(), eq.transpose(0, 2, 1, 3), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(v.numpy(), ev.transpose(0, 2, 1, 3), rtol=1e-6, atol=1e-6)


def test_chunks_and_history():
    s = ChunksAndHistory(p=224, q=100, k=125)
    assert s.deque_size() == 2  # warm-ups of 124 steps reach two boundaries ahead
    assert ChunksAndHistory(p=16, q=16, k=9).deque_size() == 1
    assert ChunksAndHistory(p=UNBOUNDED_P, q=1, k=1).deque_size() == 0
    assert ChunksAndHistory.from_dict(s.to_dict()).to_comma_separated_str() == "224,100,125"
    with pytest.raises(AssertionError):
        ChunksAndHistory(p=1, q=0, k=1)
