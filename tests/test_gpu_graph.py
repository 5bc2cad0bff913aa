"""A training step of TritonMoEMLP captured into a HIP graph (torch.cuda.graph)
and replayed: every kernel launch goes through the C ABI on torch's current
stream, the expert path needs no host sync, and the backward's second stream
(forced on here; by default only large layers take it) joins the capture
through stream waits. Each replay (with eager steps run in between) must
reproduce the eager step's output and gradients bit for bit."""

from __future__ import annotations

import pytest
import torch

from triton_moe import TritonMoEConfig, TritonMoEMLP

from _util import bits_equal, make_problem

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[None, True], ids=["default", "side_stream"])
def side_stream_mode(request):
    from triton_moe.kernels import grouped_gemm as gg

    gg.BACKWARD_SIDE_STREAM = request.param
    yield request.param
    gg.BACKWARD_SIDE_STREAM = None


@pytest.mark.parametrize("B,S,d,sizes,k", [(4, 256, 256, [(4, 512), (4, 256)], 2),
                                           (8, 1024, 768, [(8, 512)], 2)])
def test_graph_replay_matches_eager(B, S, d, sizes, k, side_stream_mode, device):
    p = make_problem(B * S, d, sizes, k, 64, seed=3, device=device)
    cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=64)
    m = TritonMoEMLP(cfg).to(device).to(torch.bfloat16)
    with torch.no_grad():
        m.router.weight.copy_(p["wr"])
        m.w1.copy_(p["w1"])
        m.w2.copy_(p["w2"])
    x = p["x"].view(B, S, d).to(device).requires_grad_(True)
    gout = torch.randn(B, S, d, generator=torch.Generator().manual_seed(5)).to(
        torch.bfloat16).to(device)

    def step():
        m.zero_grad(set_to_none=True)
        x.grad = None
        out, _, _ = m(x)
        out.backward(gout)
        return out

    ref_out = step().detach().clone()
    ref = [x.grad.clone(), m.w1.grad.clone(), m.w2.grad.clone()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = step()
    static_grads = [x.grad, m.w1.grad, m.w2.grad]
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert bits_equal(static_out, ref_out), f"replay {r}: output"
        for got, want, name in zip(static_grads, ref, ("x", "w1", "w2")):
            assert bits_equal(got, want), f"replay {r}: grad {name}"
        with torch.no_grad():
            m(x)  # eager work between replays
        torch.cuda.synchronize()
