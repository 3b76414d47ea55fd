"""GPU smoke of the GPT harness (configs[3]'s model, reduced in depth and
vocabulary): a training step under bf16 autocast runs the filter's bf16 path in
every layer, the loss is finite, and gradients reach every filter parameter.
Each layer's q, k, v equal the standalone filter's on the same input."""

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
