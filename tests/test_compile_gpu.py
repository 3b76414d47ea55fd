"""torch.compile compatibility of the drop-in path.

The reference compiles its model with ``torch.compile(model, dynamic=False)``
(scripts/base_train.py:468-470) and ships fake (meta) implementations of its
ops for that (nanochat/ops/ltv_cuda_meta.py:155-252, 341-377).  Here:
  * the filter module compiles with ``fullgraph=True`` (no graph break) in its
    bf16 and fp32 paths, and the compiled forward and backward equal eager
    bitwise (the custom ops are opaque to the compiler: the same HIP kernels
    run on the same inputs);
  * a one-layer GPT of the harness compiles with ``fullgraph=True`` and gives
    the eager loss and filter gradients (the other ops may fuse, so within
    bf16 tolerance);
  * ``torch.library.opcheck`` passes for the ops (schema, fake tensors,
    autograd registration, AOT dispatch);
  * in eager mode the modules run the fused op's implementations through a
    plain autograd function: its outputs and every gradient equal the library
    op's bitwise (shared and per-sequence inits, one upstream gradient absent).
"""

from __future__ import annotations

import pytest
import torch

from ltv_test_utils import assert_norm_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _filter(NH, NKVH, D, r, seed=0):
    from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
        LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter,
    )
    torch.manual_seed(seed)
    C = NH * D
    f = Filter(NH, NKVH, D, r)
    with torch.no_grad():
        f.c.weight.normal_(0.0, C ** -0.5)
        f.logit_bias.uniform_(-0.5, 0.5)
        f.init_param.uniform_(-0.5, 0.5)
    return f.to(DEV)


def _run_filter(f, x, grads):
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    for p in f.parameters():
        p.grad = None
    x = x.detach().clone().requires_grad_(True)
    q, k, v = f(x, LtvInitValues())
    torch.autograd.backward([q, k, v], list(grads))
    torch.cuda.synchronize()
    return [q, k, v, x.grad] + [p.grad.clone() for p in f.parameters()]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_compiled_filter_matches_eager(dtype):
    torch._dynamo.reset()
    NH, NKVH, D, r = 2, 1, 128, 128
    B, T = 2, 192
    f = _filter(NH, NKVH, D, r)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, NH * D, generator=g).to(dtype).to(DEV)
    grads = (torch.randn(B, T, NH, D, generator=g).to(dtype).to(DEV),
             torch.randn(B, T, NKVH, D, generator=g).to(dtype).to(DEV),
             torch.randn(B, T, NKVH, D, generator=g).to(dtype).to(DEV))
    want = _run_filter(f, x, grads)
    fc = torch.compile(f, fullgraph=True, dynamic=False)
    got = _run_filter(fc, x, grads)
    got2 = _run_filter(fc, x, grads)  # the cached graph, second call
    names = ["q", "k", "v", "grad_x", "grad_weight", "grad_init_param", "grad_logit_bias"]
    for name, a, b, c in zip(names, got, got2, want):
        assert torch.equal(a, c), f"{name}: compiled differs from eager"
        assert torch.equal(b, c), f"{name}: second compiled call differs from eager"


def test_compiled_gpt_layer_matches_eager():
    torch._dynamo.reset()
    from nanochat_amd.gpt import GPT, GPTConfig
    torch.manual_seed(0)
    m = GPT(GPTConfig(sequence_len=256, vocab_size=1024, n_layer=1)).to(DEV)
    m.init_weights(randomise_output_projections=True)
    m.wte.to(dtype=torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(2)
    idx = torch.randint(0, 1024, (2, 256), generator=g, device=DEV)
    tgt = torch.randint(0, 1024, (2, 256), generator=g, device=DEV)

    def step(model):
        for p in m.parameters():
            p.grad = None
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss = model(idx, tgt)
        loss.backward()
        torch.cuda.synchronize()
        f = m.filters()[0]
        return loss.detach().float(), [f.c.weight.grad.clone(), f.logit_bias.grad.clone(),
                                       f.init_param.grad.clone()]

    loss_e, grads_e = step(m)
    mc = torch.compile(m, fullgraph=True, dynamic=False)
    loss_c, grads_c = step(mc)
    assert torch.isfinite(loss_c)
    assert abs(float(loss_c) - float(loss_e)) <= 1e-2 * abs(float(loss_e))
    for name, a, b in zip(("grad_weight", "grad_logit_bias", "grad_init_param"), grads_c, grads_e):
        assert_norm_rel(a.cpu().numpy(), b.cpu().numpy(), 5e-2, name)


def _opcheck(op, args):
    # test_aot_dispatch_dynamic compiles with dynamic shapes, which the
    # reference's training never uses; the others are the op contract
    return torch.library.opcheck(op, args, test_utils=("test_schema", "test_autograd_registration",
                                                       "test_faketensor",
                                                       "test_aot_dispatch_static"))


def test_opcheck_fused_qkv_filter_ops():
    import nanochat_amd.ops  # noqa: F401
    NH, NKVH, D, r, B, T = 2, 1, 64, 64, 2, 80
    H, Da, C = NH + 2 * NKVH, D // r, NH * D
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, T, C, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(H * (D + Da), C, generator=g) / C ** 0.5).to(DEV).requires_grad_(True)
    inits = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    bias = torch.zeros(H, Da, device=DEV, requires_grad=True)
    _opcheck(torch.ops.nanochat_amd.qkv_filter.default, (x, w, inits, bias, NH, NKVH, Da, r))


def test_opcheck_reference_namespace_ops():
    import nanochat_amd.ops  # noqa: F401
    NH, NKVH, Da, r, B, T = 2, 1, 2, 32, 2, 40
    H, D = NH + 2 * NKVH, Da * r
    g = torch.Generator().manual_seed(4)
    comb = torch.randn(B, T, H * (D + Da), generator=g).to(DEV).requires_grad_(True)
    inits = torch.randn(B, H, D, generator=g).to(DEV).requires_grad_(True)
    bias = torch.zeros(H, Da, device=DEV, requires_grad=True)
    op = torch.ops.nanochat_cuda.ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op
    _opcheck(op.default, (comb, inits, bias, NH, NKVH, Da, r, 8, 8, 4, 32, 2, 8, True))
    x = torch.randn(B, T, 64, generator=g).to(DEV).requires_grad_(True)
    w = torch.randn(96, 64, generator=g).to(DEV).requires_grad_(True)
    _opcheck(torch.ops.nanochat_cuda.fused_linear_transpose_cuda_op.default, (x, w))


@pytest.mark.parametrize("shared", [False, True], ids=["batch_inits", "shared_inits"])
def test_eager_function_matches_library_op(shared):
    from nanochat_amd.ops import ltv_hm_fast as hm
    NH, NKVH, D, r, B, T = 2, 1, 64, 16, 3, 150
    H, Da, C = NH + 2 * NKVH, D // r, NH * D
    g = torch.Generator().manual_seed(5)
    x0 = torch.randn(B, T, C, generator=g).to(torch.bfloat16).to(DEV)
    w0 = (torch.randn(H * (D + Da), C, generator=g) / C ** 0.5).to(DEV)
    i0 = torch.randn(H, D, generator=g) if shared else torch.randn(B, H, D, generator=g)
    i0 = i0.to(torch.bfloat16).to(DEV)
    b0 = (torch.rand(H, Da, generator=g) - 0.5).to(DEV)
    gq = torch.randn(B, NH, T, D, generator=g).to(torch.bfloat16).to(DEV)
    gv = torch.randn(B, NKVH, T, D, generator=g).to(torch.bfloat16).to(DEV)

    def run(fn):
        x, w, i, b = (t.detach().clone().requires_grad_(True) for t in (x0, w0, i0, b0))
        q, k, v, *_ = fn(x, w, i, b, NH, NKVH, Da, r)
        torch.autograd.backward([q, v], [gq, gv])  # k's gradient absent
        torch.cuda.synchronize()
        return [q, k, v, x.grad, w.grad, i.grad, b.grad]

    want = run(torch.ops.nanochat_amd.qkv_filter)
    got = run(hm.qkv_filter_call)
    names = ["q", "k", "v", "grad_x", "grad_weight", "grad_inits", "grad_logit_bias"]
    for name, a, e in zip(names, got, want):
        assert torch.equal(a, e), f"{name}: eager function differs from the library op"
