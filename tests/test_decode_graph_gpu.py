"""The decode step captured in a HIP graph and replayed.

Serving loops capture their per-token step (``torch.cuda.CUDAGraph``) to remove
the host dispatch around it.  ``ltv_qkv_decode_step`` is one kernel launch on
the caller's stream: it allocates nothing, synchronises nothing and records no
memset, so it can be captured.  The graph is replayed several times with new
contents in its static inputs and eager decode steps between the replays; every
replay must equal the eager step on the same inputs bit for bit (same kernel,
same inputs).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("NH,NKVH,D,r,B", [(6, 6, 128, 128, 64), (2, 1, 64, 4, 8)])
def test_decode_step_replays_in_a_graph(NH, NKVH, D, r, B):
    from nanochat_amd.ops import ltv_hm_fast as F

    g = torch.Generator(device=DEV).manual_seed(NH * 100 + D + r)
    Da = D // r
    H = NH + 2 * NKVH
    C = NH * D
    bf = torch.bfloat16
    weight = torch.randn(H * (D + Da), C, generator=g, device=DEV) * C ** -0.5
    wpack = F.pack_weight(weight, H, D, Da)
    bias = torch.rand(H, Da, generator=g, device=DEV) - 0.5

    def fresh_inputs():
        x = torch.randn(B, C, generator=g, device=DEV).to(bf)
        prev = tuple(torch.randn(B, nh, D, generator=g, device=DEV).to(bf)
                     for nh in (NH, NKVH, NKVH))
        return x, prev

    # static inputs of the graph
    x_s, prev_s = fresh_inputs()
    prev_s = tuple(t.clone() for t in prev_s)

    def step():
        return F.decode_step(x_s, wpack, prev_s, bias, NH, NKVH, Da, r, True)

    # warm up on a side stream, as torch's graph capture expects
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = step()
    torch.cuda.synchronize()

    for i in range(4):
        x_n, prev_n = fresh_inputs()
        x_s.copy_(x_n)
        for dst, src in zip(prev_s, prev_n):
            dst.copy_(src)
        want = F.decode_step(x_n, wpack, prev_n, bias, NH, NKVH, Da, r, True)  # eager
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert out_g.shape == (B, H, D)
        assert torch.equal(out_g, want), f"replay {i}: max diff {(out_g.float() - want.float()).abs().max()}"
        # the eager step keeps working between replays
        again = F.decode_step(x_n, wpack, prev_n, bias, NH, NKVH, Da, r, True)
        torch.cuda.synchronize()
        assert torch.equal(again, want)
