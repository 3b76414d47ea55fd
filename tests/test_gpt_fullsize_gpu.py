"""configs[3] at full size: one training step of the 12-layer d12 GPT
(768 wide, 6 heads of 128, vocabulary 65536, T = 1024) on B = 16 token ids
~ U[0, 65536), random-init weights, bf16 autocast, the LTV filter in every
layer (the model of nanochat/gpt.py:631-706, the harness of
nanochat/bench/bench_gpt_ltv.py:345-428).

Checks:
  * the step-0 loss is ln(65536) within 1%: lm_head ~ N(0, 0.001) makes the
    logits nearly zero, so the predicted distribution is nearly uniform
    whatever the layers compute;
  * every filter's parameters receive finite, non-zero gradients;
  * layer 0's filter outputs on a sampled batch row equal the oracle's
    (projection + sequential scan of the same bf16 input and weights) within
    the bf16 tolerance;
  * layer 0's gradients: the model's gradients of the filter's input and of
    its three parameters are bitwise what the filter computes from the
    captured input and the upstream gradients of its q, k, v (the wiring of
    the step), and the filter's backward on a sampled row alone equals the
    oracle's (grad_x, and the row's grad_weight, grad_init_param and
    grad_logit_bias) within the bf16 tolerance.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import ltv_oracle as O
from ltv_test_utils import assert_close, assert_norm_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_gpt_d12_full_size_training_step():
    from nanochat_amd.gpt import GPT, GPTConfig
    B, T = 16, 1024
    cfg = GPTConfig()
    assert (cfg.n_layer, cfg.n_embd, cfg.n_head, cfg.vocab_size, cfg.sequence_len) == (
        12, 768, 6, 65536, 1024)
    torch.manual_seed(0)
    model = GPT(cfg).to(DEV)
    model.init_weights(randomise_output_projections=True)
    model.wte.to(dtype=torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(0)
    idx = torch.randint(0, cfg.vocab_size, (B, T), generator=g, device=DEV)
    tgt = torch.randint(0, cfg.vocab_size, (B, T), generator=g, device=DEV)

    seen = {}

    def hook(module, args, output):
        seen["x"] = args[0].detach()
        seen["qkv"] = [o.detach() for o in output]
        # the gradients that reach the filter: its input's, and its outputs'
        args[0].register_hook(lambda g: seen.__setitem__("gx", g.detach()))
        for i, o in enumerate(output):
            o.register_hook(lambda g, i=i: seen.__setitem__(f"g{i}", g.detach()))

    f0 = model.filters()[0]
    handle = f0.register_forward_hook(hook)
    try:
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss = model(idx, tgt)
        loss.backward()
        torch.cuda.synchronize()
    finally:
        handle.remove()

    assert torch.isfinite(loss)
    assert abs(float(loss) - math.log(cfg.vocab_size)) <= 0.01 * math.log(cfg.vocab_size), float(loss)
    for i, f in enumerate(model.filters()):
        for name, p in (("c.weight", f.c.weight), ("logit_bias", f.logit_bias),
                        ("init_param", f.init_param)):
            assert p.grad is not None, f"layer {i} {name}: no gradient"
            assert torch.isfinite(p.grad).all(), f"layer {i} {name}: non-finite gradient"
            assert float(p.grad.abs().sum()) > 0, f"layer {i} {name}: zero gradient"

    # layer 0 on batch row 5 against the oracle (the filter computes in bf16
    # under autocast: bf16 input, the fp32 master weight rounded to bf16)
    b = 5
    NH, NKVH, D, r = cfg.n_head, cfg.n_kv_head, cfg.n_embd // cfg.n_head, cfg.ltv_r
    H, Da = NH + 2 * NKVH, D // r
    x = seen["x"][b:b + 1].to(torch.bfloat16).float().cpu().numpy()
    w = O.bf16_round(f0.c.weight.detach().float().cpu().numpy())
    ini = O.round_io(np.broadcast_to(f0.init_param.detach().float().cpu().numpy(),
                                     (1, H, D)).copy(), "bf16")
    bias = f0.logit_bias.detach().float().cpu().numpy()
    eq, ek, ev, _, _ = O.filter_forward(x, w, ini, bias, NH, NKVH, Da, r, "bf16")
    q, k, v = (t[b:b + 1].float().cpu().numpy() for t in seen["qkv"])
    assert_close(q, eq, 2e-2, "layer 0 q, row 5")
    assert_close(k, ek, 2e-2, "layer 0 k, row 5")
    assert_close(v, ev, 2e-2, "layer 0 v, row 5")

    # ---- layer 0's gradients
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    params = (f0.c.weight, f0.logit_bias, f0.init_param)
    ups = [seen[f"g{i}"] for i in range(3)]

    def filter_grads(rows):
        xr = seen["x"][rows].clone().requires_grad_(True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            outs = f0(xr, LtvInitValues())
        return torch.autograd.grad(outs, (xr,) + params, [u[rows] for u in ups])

    # the step's wiring: the same filter on the captured tensors, all rows
    gx_all, *gp_all = filter_grads(slice(None))
    assert torch.equal(gx_all, seen["gx"]), "grad of the filter input"
    for name, got, p in zip(("c.weight", "logit_bias", "init_param"), gp_all, params):
        assert torch.equal(got, p.grad), f"layer 0 {name}: gradient differs from the filter's own"

    # the filter's backward on row 5 alone against the oracle
    gx5, gw5, gb5, gi5 = filter_grads(slice(b, b + 1))
    _, _, _, comb, saved = O.filter_forward(x, w, ini, bias, NH, NKVH, Da, r, "bf16")
    dq, dk, dv = (u[b:b + 1].float().cpu().numpy() for u in ups)
    egx, egw, egi, egb = O.filter_backward(x, w, ini, bias, comb, saved, dq, dk, dv, NH, NKVH,
                                           Da, r, "bf16")
    np_ = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    assert_close(np_(gx5), egx, 2e-2, "layer 0 grad_x, row 5")
    assert_norm_rel(np_(gx5), egx, 2e-2, "layer 0 grad_x, row 5")
    assert_norm_rel(np_(gw5), egw, 2e-2, "layer 0 grad_weight, row 5")
    assert_norm_rel(np_(gi5), egi.sum(axis=0), 2e-2, "layer 0 grad_init_param, row 5")
    assert_close(np_(gb5), egb, 2e-2, "layer 0 grad_logit_bias, row 5")
