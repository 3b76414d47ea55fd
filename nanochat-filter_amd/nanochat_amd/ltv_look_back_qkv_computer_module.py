"""Adapter from a look-back filter to ``CausalSelfAttention``'s
``qkv_computer(x, kv_cache)`` protocol, and the KV-cache advance that lets
inference feed tokens in any grouping (reference
``nanochat/ltv_look_back_qkv_computer_module.py:15-209``).

Without a cache the filter runs its chunked scan (``full_recurrence=False``).
With one, ``advance_kv_cache`` reproduces the chunked scan piece by piece,
using only unchunked calls (``full_recurrence=True``, which the filters run as
one window, or as the fused decode kernel for one-token steps):

  * the cache's ``special`` rows are the state the current chunk continues
    from; ``countdown`` is the number of steps left in it (``p``, or ``q`` when
    ``p == 0``, for the first chunk);
  * ``d[i]`` is the warm-up state of the chunk boundary ``i + 1`` ahead: the
    recurrence from the inits over the ``k - 1`` steps before that boundary,
    advanced as those steps arrive (boundary ``i + 1`` ahead lies
    ``countdown + i q`` steps after the current position);
  * at a boundary the nearest warm-up state becomes ``special``, a fresh
    warm-up (the inits) joins the deque and ``countdown`` restarts at ``q``.

Tokens are consumed in segments that never cross a chunk boundary, so feeding
a sequence whole, token by token, or in any grouping gives the same rows.
"""

from __future__ import annotations

import collections
import logging
from typing import Optional

import torch
import torch.nn as nn

from nanochat_amd.kv_cache import KVCache, TypeDevice, make_empty_last_qkv_like_specials
from nanochat_amd.ltv_look_back_head_major_qkv_filter_base import LtvLookBackHeadMajorQkvFilter

logger = logging.getLogger(__name__)


def _init_layer_state(last_qkv, layer_idx, layer_spec, inits_qkv):
    for proj, x0 in zip((last_qkv.q, last_qkv.k, last_qkv.v), inits_qkv):
        layer = proj.layers[layer_idx]
        if layer.is_initialized():
            continue
        proj.special[layer_idx, :, :, :] = x0
        layer.countdown = layer_spec.p or layer_spec.q
        if layer_spec.is_unbounded():
            layer.d = collections.deque(maxlen=0)
        else:
            ml = layer_spec.deque_size()
            layer.d = collections.deque([x0] * ml, maxlen=ml)


def advance_kv_cache(x: torch.Tensor, layer_idx: int, ltv_filter: LtvLookBackHeadMajorQkvFilter,
                     resolved_inits: torch.Tensor, kv_cache: KVCache):
    """Run the layer's filter over ``x`` (B, T, C) from the cached state and
    advance that state; returns q (B, T, NH, D), k, v (B, T, NKVH, D)."""
    last = kv_cache.last_qkv
    if last is None:
        assert not layer_idx
        td = TypeDevice(x.dtype, x.device)
        last = kv_cache.last_qkv = make_empty_last_qkv_like_specials(
            kv_cache.last_q_shape, kv_cache.last_k_v_shape, td, td, td,
            mls=[spec.deque_size() for spec in kv_cache.layer_specs])
    else:
        assert last.q and last.k and last.v
    spec = kv_cache.layer_specs[layer_idx]
    NH, NKVH = ltv_filter.n_head, ltv_filter.n_kv_head
    # per-head split of the (B, NH + 2 NKVH, D) inits
    inits_qkv = torch.split(resolved_inits, [NH, NKVH, NKVH], dim=1)
    _init_layer_state(last, layer_idx, spec, inits_qkv)

    layers = [proj.layers[layer_idx] for proj in (last.q, last.k, last.v)]
    specials = [proj.special for proj in (last.q, last.k, last.v)]
    n = x.shape[1]
    pieces = []
    start = 0
    while start < n:
        (countdown,) = {layer.countdown for layer in layers}
        seg = min(countdown, n - start)  # never crosses the next chunk boundary
        state = torch.cat([s[layer_idx] for s in specials], dim=1)
        out = ltv_filter.forward(x=x[:, start:start + seg], resolved_inits=state,
                                 full_recurrence=True)
        pieces.append(out)

        # advance the warm-ups of the boundaries ahead over this segment's steps
        for i, warm in enumerate(zip(*(layer.d for layer in layers), strict=True)):
            # first step of this segment inside boundary i's warm-up window
            first = max(countdown + i * spec.q - spec.k + 1, 0)
            if first >= seg:
                continue
            wq, wk, wv = ltv_filter.forward(x=x[:, start + first:start + seg],
                                            resolved_inits=torch.cat(warm, dim=1),
                                            full_recurrence=True)
            for layer, rows in zip(layers, (wq, wk, wv)):
                layer.d[i] = rows[:, -1, :, :]

        if seg == countdown:
            # chunk boundary: continue from the nearest warm-up, start a new one
            for layer, s, x0 in zip(layers, specials, inits_qkv):
                nxt = layer.d[0] if layer.d else x0
                layer.d.append(x0)
                s[layer_idx, :, :, :] = nxt
                layer.countdown = spec.q
        else:
            for layer, s, rows in zip(layers, specials, out):
                layer.countdown = countdown - seg
                s[layer_idx, :, :, :] = rows[:, -1, :, :]
        start += seg

    assert last.m == layer_idx or last.m == kv_cache.num_ltv_layers()
    if last.m != kv_cache.num_ltv_layers():
        last.m += 1

    B, D = x.shape[0], ltv_filter.head_dim
    parts = [[torch.empty(B, 0, nh, D, dtype=x.dtype, device=x.device)] for nh in (NH, NKVH, NKVH)]
    for out in pieces:
        for p, t in zip(parts, out):
            p.append(t)
    return tuple(torch.cat(p, dim=1) for p in parts)


class LtvLookBackQkvComputerModule(nn.Module):
    def __init__(self, layer_idx: int, ltv_filter: LtvLookBackHeadMajorQkvFilter):
        super().__init__()
        self.ltv_filter = ltv_filter
        self.layer_idx = layer_idx
        self.advance_last_qkv = lambda kv_cache, resolved_inits, x: advance_kv_cache(
            x, layer_idx, self.ltv_filter, resolved_inits, kv_cache)

    def forward(self, x, kv_cache: Optional[KVCache]):
        B = x.size(0)
        if kv_cache is None and hasattr(self.ltv_filter, "takes_shared_inits"):
            # the (H, D) parameter itself: the filter broadcasts it to every
            # sequence and its gradient comes back summed over the batch
            # (the reference expands it to (B, H, D) here; same values)
            return self.ltv_filter(x, self.ltv_filter.init_param, full_recurrence=False)
        resolved_inits = self.ltv_filter.init_param.unsqueeze(0).expand(B, -1, -1)
        if kv_cache is not None:
            return self.advance_last_qkv(kv_cache, resolved_inits, x)
        return self.ltv_filter(x, resolved_inits, full_recurrence=False)

    def init_weights(self, alpha_mlp_bias_init: float, weight_s: float, bias_s: float,
                     init_s: float):
        self.ltv_filter.init_weights(alpha_mlp_bias_init=alpha_mlp_bias_init,
                                     weight_s=weight_s, bias_s=bias_s, init_s=init_s)

    def get_matrix_linear_params(self):
        return self.ltv_filter.get_matrix_linear_params()

    def estimate_flops(self, sequence_len: int) -> int:
        return self.ltv_filter.estimate_flops(sequence_len)

    def ltv_parameter_count(self) -> int:
        return self.ltv_filter.ltv_parameter_count()
