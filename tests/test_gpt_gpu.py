"""GPU tests of the GPT harness (configs[3]'s model, reduced in depth and
vocabulary): a training step under bf16 autocast runs the filter's bf16 path in
every layer, the loss is finite, and gradients reach every filter parameter;
each layer's q, k, v equal the standalone filter's on the same input; and in a
training step every filter's outputs and parameter gradients equal the
oracle's on the input and upstream gradients the filter saw."""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model(n_layer=2, vocab=1000):
    from nanochat_amd.gpt import GPT, GPTConfig
    torch.manual_seed(0)
    m = GPT(GPTConfig(sequence_len=256, vocab_size=vocab, n_layer=n_layer)).to(DEV)
    m.init_weights(randomise_output_projections=True)
    m.wte.to(dtype=torch.bfloat16)
    return m


def test_gpt_training_step_reaches_every_filter():
    from nanochat_amd import _native as N
    m = _model()
    g = torch.Generator(device=DEV).manual_seed(1)
    idx = torch.randint(0, 1000, (4, 256), generator=g, device=DEV)
    tgt = torch.randint(0, 1000, (4, 256), generator=g, device=DEV)
    with N.KernelRecorder() as rec:
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss = m(idx, tgt)
        loss.backward()
        torch.cuda.synchronize()
    spans = rec.durations_ms()
    # the bf16 fast path ran in both layers, forward and backward
    assert len(spans.get("qkv_project_fwd", [])) == 2 and len(spans.get("scan_bwd", [])) == 2
    assert torch.isfinite(loss)
    for f in m.filters():
        for p in (f.c.weight, f.logit_bias, f.init_param):
            assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().sum() > 0


def test_gpt_layer_qkv_equals_standalone_filter():
    from nanochat_amd.gpt import norm
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    m = _model(n_layer=1)
    idx = torch.randint(0, 1000, (2, 128), device=DEV)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        x = norm(m.wte(idx))
        q1, k1, v1 = m.h[0].attn.qkv_computer(norm(x), None)
        q2, k2, v2 = m.filters()[0](norm(x), LtvInitValues())
    for a, b in ((q1, q2), (k1, k2), (v1, v2)):
        assert torch.equal(a, b)


def test_gpt_filter_gradients_match_oracle():
    """In a 2-layer training step under bf16 autocast, every filter's output
    and parameter gradients equal the oracle's filter forward and backward on
    the input the filter saw and the upstream q/k/v gradients it received
    (captured with hooks), within the bf16 tolerance."""
    import numpy as np

    import ltv_oracle as O
    from ltv_test_utils import TOL, assert_close, assert_norm_rel, np_of
    m = _model(n_layer=2)
    seen = {}

    def capture(i):
        def hook(module, args, out):
            seen[i] = {"x": args[0].detach().clone(), "out": [t.detach().clone() for t in out]}
            for name, t in zip("qkv", out):
                t.register_hook(lambda g, name=name: seen[i].__setitem__("g" + name,
                                                                          g.detach().clone()))
        return hook

    handles = [f.register_forward_hook(capture(i)) for i, f in enumerate(m.filters())]
    g = torch.Generator(device=DEV).manual_seed(3)
    idx = torch.randint(0, 1000, (2, 128), generator=g, device=DEV)
    tgt = torch.randint(0, 1000, (2, 128), generator=g, device=DEV)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        loss = m(idx, tgt)
    loss.backward()
    torch.cuda.synchronize()
    for h in handles:
        h.remove()
    tol = TOL[torch.bfloat16]
    for i, f in enumerate(m.filters()):
        s = seen[i]
        NH, NKVH, Da, r = f.n_head, f.n_kv_head, f.num_alpha_groups, f.r
        x = O.bf16_round(np_of(s["x"]))  # the fast path multiplies the bf16 input
        B = x.shape[0]
        w = O.bf16_round(np_of(f.c.weight))
        ini = np.broadcast_to(np_of(f.init_param), (B,) + tuple(f.init_param.shape))
        ini = O.round_io(np.ascontiguousarray(ini), "bf16")
        bias = np_of(f.logit_bias)
        q, k, v, comb, saved = O.filter_forward(x, w, ini, bias, NH, NKVH, Da, r, "bf16")
        for name, got, want in zip("qkv", s["out"], (q, k, v)):
            assert_close(np_of(got), want, tol, f"layer {i} {name}")
        _, gw, gi, gb = O.filter_backward(x, w, ini, bias, comb, saved, np_of(s["gq"]),
                                          np_of(s["gk"]), np_of(s["gv"]), NH, NKVH, Da, r, "bf16")
        # the loss is a mean over tokens, so the gradients are small: the
        # normwise check (max|a - e| <= tol max|e|) is the one that binds
        for name, got, want in (("grad_weight", f.c.weight.grad, gw),
                                ("grad_init_param", f.init_param.grad, gi.sum(axis=0)),
                                ("grad_logit_bias", f.logit_bias.grad, gb)):
            assert_close(np_of(got), want, tol, f"layer {i} {name}")
            assert_norm_rel(np_of(got), want, tol, f"layer {i} {name}")
