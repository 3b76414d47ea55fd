"""CPU pins of the filter module's parameter bookkeeping and seeded init.

Reference: nanochat/ltv_combined_qkv_filter_base.py:14-71 (parameters,
optimiser grouping, FLOP estimate, LTV parameter count) and
nanochat/ltv_combined_head_major_qkv_filter.py:21-66 with
nanochat/ltv/ltv_fused_scan_filter.py:17-39 (seeded init: value rows of q, k,
v, then the gate rows, interleaved per head; then logit_bias; then init_param
q, k, v).
"""

from __future__ import annotations

import pytest
import torch

from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
    LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter,
)

SHAPES = [(6, 6, 128, 128), (4, 2, 16, 4), (2, 1, 8, 1), (3, 3, 12, 3)]


@pytest.mark.parametrize("NH,NKVH,D,r", SHAPES)
def test_parameter_shapes_and_grouping(NH, NKVH, D, r):
    f = Filter(NH, NKVH, D, r)
    H, Da, C = NH + 2 * NKVH, D // r, NH * D
    assert tuple(f.c.weight.shape) == (H * (D + Da), C)
    assert f.c.bias is None
    assert tuple(f.logit_bias.shape) == (H, Da)
    assert tuple(f.init_param.shape) == (H, D)
    # state_dict keys the reference's checkpoints carry
    assert set(f.state_dict()) == {"c.weight", "logit_bias", "init_param"}
    matrix, linear = f.get_matrix_linear_params()
    # c.weight goes to Muon, the two small parameters to AdamW; every
    # parameter lands in exactly one group
    assert [id(p) for p in matrix] == [id(f.c.weight)]
    assert [id(p) for p in linear] == [id(f.logit_bias), id(f.init_param)]
    assert sorted(map(id, matrix + linear)) == sorted(map(id, f.parameters()))
    assert [id(p) for p in f.get_init_parameters()] == [id(f.init_param)]
    assert f.split_sections == [NH * D, NKVH * D, NKVH * D, H * Da]


def test_d12_flops_and_parameter_count():
    """d12 (6 + 2*6 heads of 128, r = 128): 6 * 18 * 768 gate-projection
    FLOPs + 7 * 18 * 128 scan FLOPs per token; the LTV parameters are the 18
    gate rows of c.weight, logit_bias and init_param."""
    f = Filter(6, 6, 128, 128)
    assert f.estimate_flops(1024) == 99_072
    assert f.ltv_parameter_count() == 16_146


@pytest.mark.parametrize("NH,NKVH,D,r", SHAPES)
def test_flops_and_parameter_count_by_counting(NH, NKVH, D, r):
    """Both figures from an independent count: the LTV parameters are every
    parameter except the value rows of c.weight, found by walking the
    interleaved rows; the gate-projection FLOPs are 6 per gate-row weight, the
    scan 7 per filtered channel (per token, independent of T)."""
    f = Filter(NH, NKVH, D, r)
    H, Da, C = NH + 2 * NKVH, D // r, NH * D
    rows = f.c.weight.shape[0]
    gate_rows = sum(1 for i in range(rows) if i % (D + Da) >= D)
    value_rows = rows - gate_rows
    assert f.ltv_parameter_count() == gate_rows * C + f.logit_bias.numel() + f.init_param.numel()
    assert value_rows == H * D
    for T in (1, 7, 1024):
        assert f.estimate_flops(T) == 6 * gate_rows * C + 7 * H * D


@pytest.mark.parametrize("NH,NKVH,D,r", SHAPES)
def test_seeded_init_consumes_one_uniform_stream_in_reference_order(NH, NKVH, D, r):
    """With every draw on the CPU generator, the seeded init equals one stream
    of uniforms read in the order: the value rows of q, k, v heads (row-major),
    the H*Da gate rows, the H*Da biases, the H*D inits (q, k, v).  The weight
    is checked through the per-head interleave [values D | gates Da], read back
    row by row, so a wrong interleave or draw order fails."""
    ambi, ws, bs, init_s = -1.5, 0.07, 0.3, 0.2
    H, Da, C = NH + 2 * NKVH, D // r, NH * D
    f = Filter(NH, NKVH, D, r)
    torch.manual_seed(1234)
    f.init_weights(ambi, ws, bs, init_s)

    torch.manual_seed(1234)
    values = torch.empty(H * D, C).uniform_(-ws, ws)   # q, k, v value rows
    gates = torch.empty(H * Da, C).uniform_(-ws, ws)
    bias = torch.empty(H, Da).uniform_(ambi - bs, ambi + bs)
    inits = torch.empty(H, D).uniform_(-init_s, init_s)

    W = f.c.weight.detach()
    for h in range(H):
        base = h * (D + Da)
        assert torch.equal(W[base:base + D], values[h * D:(h + 1) * D]), f"value rows of head {h}"
        assert torch.equal(W[base + D:base + D + Da], gates[h * Da:(h + 1) * Da]), f"gate rows of head {h}"
    assert torch.equal(f.logit_bias.detach(), bias)
    assert torch.equal(f.init_param.detach(), inits)
    # ranges (up to the float32 rounding of the bounds)
    eps = 1e-6
    assert float(W.abs().max()) <= ws + eps
    assert float((f.logit_bias.detach() - ambi).abs().max()) <= bs + eps
    assert float(f.init_param.detach().abs().max()) <= init_s + eps


def test_uniform_stream_splits_like_one_draw():
    """The property the init test leans on: on the CPU generator, consecutive
    uniform_ draws read one stream (a draw of n + m values equals a draw of n
    then a draw of m, before scaling)."""
    torch.manual_seed(7)
    one = torch.empty(1000).uniform_(0.0, 1.0)
    torch.manual_seed(7)
    a = torch.empty(300).uniform_(0.0, 1.0)
    b = torch.empty(700).uniform_(0.0, 1.0)
    assert torch.equal(one, torch.cat([a, b]))


def test_load_state_dict_drops_the_packed_weight_cache():
    """The decode path caches a packed copy of c.weight on the module; loading a
    state dict must drop it (checked on the CPU: the cache attribute only)."""
    f = Filter(2, 1, 16, 4)
    f._wpack_cache = ("stale-key", torch.zeros(1))
    g = Filter(2, 1, 16, 4)
    f.load_state_dict(g.state_dict())
    assert f._wpack_cache is None
    f._wpack_cache = ("stale-key", torch.zeros(1))
    f.invalidate_packed_weight()
    assert f._wpack_cache is None
