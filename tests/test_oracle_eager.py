"""Pins the eager per-expert-loop oracle (oracle/eager.py) on the CPU.

* fp32 mode (run in float64) against a dense all-experts formulation with a
  routing-weight matrix (no sorting, padding or gather), forward and torch
  autograd gradients.
* bf16 mode against hand-computed values where each rounding point changes
  the result, and against the fp32 mode within bf16 precision.
"""

from __future__ import annotations

import pytest
import torch

from oracle import eager


def _problem(seed, T, d, sizes, k, b, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    widths, offsets = eager.expert_layout(sizes)
    E, W = len(widths), offsets[-1]
    x = torch.randn(T, d, generator=g, dtype=dtype)
    w1 = torch.randn(d, W, generator=g, dtype=dtype) * 0.3
    w2 = torch.randn(W, d, generator=g, dtype=dtype) * 0.3
    logits = torch.randn(T, E, generator=g)
    wts, sel = torch.topk(torch.sigmoid(logits), k, dim=-1)
    wts = (wts / wts.sum(-1, keepdim=True)).to(torch.bfloat16).to(dtype)
    return eager.Problem(x, w1, w2, widths, offsets, sel, wts, b)


def _dense(prob, x, w1, w2):
    E = prob.num_experts
    R = torch.zeros(x.shape[0], E, dtype=x.dtype)
    R.scatter_add_(1, prob.selected, prob.weights.to(x.dtype))
    out = torch.zeros_like(x)
    for e, (w, o) in enumerate(zip(prob.widths, prob.offsets)):
        h = torch.relu(x @ w1[:, o:o + w]) ** 2
        out = out + R[:, e:e + 1] * (h @ w2[o:o + w])
    return out


@pytest.mark.parametrize("sizes,k,b", [([(4, 16)], 2, 4), ([(2, 24), (3, 8), (1, 16)], 3, 8),
                                       ([(8, 8)], 8, 16)])
def test_fp32_forward_backward_vs_dense(sizes, k, b):
    prob = _problem(0, 37, 12, sizes, k, b)
    fwd = eager.forward(prob, "fp32")
    x = prob.x.clone().requires_grad_(True)
    w1 = prob.w1.clone().requires_grad_(True)
    w2 = prob.w2.clone().requires_grad_(True)
    ref = _dense(prob, x, w1, w2)
    torch.testing.assert_close(fwd["out"], ref.detach(), rtol=1e-10, atol=1e-12)
    G = torch.randn(ref.shape, generator=torch.Generator().manual_seed(1), dtype=ref.dtype)
    ref.backward(G)
    bwd = eager.backward(prob, fwd, G, "fp32")
    torch.testing.assert_close(bwd["grad_x"], x.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(bwd["grad_w1"], w1.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(bwd["grad_w2"], w2.grad, rtol=1e-10, atol=1e-12)


def test_fp32_gradcheck_dense():
    """The dense formulation's autograd against finite differences (float64)."""
    prob = _problem(3, 5, 4, [(3, 4)], 2, 2)

    def f(x, w1, w2):
        return _dense(prob, x, w1, w2)

    args = [prob.x.clone().requires_grad_(True), prob.w1.clone().requires_grad_(True),
            prob.w2.clone().requires_grad_(True)]
    assert torch.autograd.gradcheck(f, args)


def test_bf16_rounding_points_by_hand():
    # One token, one expert of width 1: pre = 1 + 2^-7 (exact in bf16),
    # pre^2 = 1 + 2^-6 + 2^-14 rounds to 1 + 2^-6 when H is stored as bf16.
    f = torch.float32
    pre = 1.0 + 2.0 ** -7
    x = torch.tensor([[1.0]], dtype=f)
    w1 = torch.tensor([[pre]], dtype=f)
    w2 = torch.tensor([[1.0]], dtype=f)
    prob = eager.Problem(x, w1, w2, [1], [0, 1], torch.tensor([[0]]),
                         torch.tensor([[1.0]], dtype=f), 1)
    out_bf = eager.forward(prob, "bf16")["out"].item()
    out_fp = eager.forward(prob, "fp32")["out"].item()
    assert out_bf == 1.0 + 2.0 ** -6
    assert out_fp == pytest.approx(pre * pre, rel=1e-7) and out_fp != out_bf
    # GA = bf16(2 * GH * PRE): GH = 1 + 2^-7 (w2 = that, G = 1) -> 2 * (1+2^-7)^2
    # = 2 + 2^-5 + 2^-13 -> bf16 2 + 2^-5
    w2b = torch.tensor([[pre]], dtype=f)
    prob2 = eager.Problem(x, w1, w2b, [1], [0, 1], torch.tensor([[0]]),
                          torch.tensor([[1.0]], dtype=f), 1)
    fw = eager.forward(prob2, "bf16")
    bw = eager.backward(prob2, fw, torch.ones(1, 1), "bf16")
    assert bw["grad_a"][0, 0].item() == 2.0 + 2.0 ** -5
    # combine: slot = bf16(y * w); y = 1 + 2^-7, w = 1 + 2^-7 -> 1 + 2^-6 + 2^-14 -> 1 + 2^-6
    y = torch.tensor([[pre]], dtype=f)
    out = eager.combine(y, [0], torch.tensor([pre], dtype=f), 1, 1, "bf16")
    assert out.item() == 1.0 + 2.0 ** -6


def test_bf16_mode_close_to_fp32_mode():
    prob = _problem(5, 64, 32, [(2, 32), (4, 16)], 2, 8, dtype=torch.float32)
    prob.x = prob.x.to(torch.bfloat16).float()
    prob.w1 = prob.w1.to(torch.bfloat16).float()
    prob.w2 = prob.w2.to(torch.bfloat16).float()
    a = eager.forward(prob, "fp32")["out"]
    b = eager.forward(prob, "bf16")["out"]
    assert (a - b).abs().max() / a.abs().max() < 2e-2
    assert (a - b).abs().mean() / a.abs().mean() < 1e-2


def test_bf16w_rounding_points_by_hand():
    """Mode "bf16w" puts the routing weight on H: H' = bf16(w relu(z)^2),
    out = bf16(H' @ W2) (unweighted combine), GH = bf16(w (G @ W2^T))."""
    f = torch.float32
    a = 1.0 + 2.0 ** -7  # exact in bf16
    x = torch.tensor([[1.0]], dtype=f)
    one = torch.tensor([[1.0]], dtype=f)
    # relu(z) = 1, w = a: H' = a exactly; W2 = a: out = bf16(a * a) = 1 + 2^-6
    prob = eager.Problem(x, one, torch.tensor([[a]], dtype=f), [1], [0, 1],
                         torch.tensor([[0]]), torch.tensor([[a]], dtype=f), 1)
    fw = eager.forward(prob, "bf16w")
    assert fw["h"][0, 0].item() == a
    assert fw["out"].item() == 1.0 + 2.0 ** -6
    # the reference order rounds y = a first, then bf16(y * w): the same here
    assert eager.forward(prob, "bf16")["out"].item() == 1.0 + 2.0 ** -6
    # G = a: GH = bf16(w * (G @ W2^T)) = bf16(a^3) = 1 + 3 * 2^-7 (exact: 1 + 3*2^-7
    # + 3*2^-14 + 2^-21 rounds down), and the reference's GY = bf16(a * a) = 1 + 2^-6,
    # GH = bf16(GY * a) = bf16(1 + 3*2^-7 + 2^-13) = 1 + 3 * 2^-7: same, by another path
    bw = eager.backward(prob, fw, torch.tensor([[a]], dtype=f), "bf16w")
    assert bw["grad_h"][0, 0].item() == 1.0 + 3 * 2.0 ** -7
    # dW2 = H'^T G = a * a -> bf16 1 + 2^-6
    assert bw["grad_w2"][0, 0].item() == 1.0 + 2.0 ** -6


@pytest.mark.parametrize("seed", [0, 1])
def test_bf16w_mode_no_less_accurate_than_bf16(seed):
    """Both bf16 orders against the unrounded fp32 mode: the row-weighted
    order (fewer roundings per product) is within bf16 tolerance and no
    worse than the reference's order by more than a little."""
    prob = _problem(seed, 128, 64, [(2, 64), (4, 32)], 2, 8, dtype=torch.float32)
    prob.x = prob.x.to(torch.bfloat16).float()
    prob.w1 = prob.w1.to(torch.bfloat16).float()
    prob.w2 = prob.w2.to(torch.bfloat16).float()
    ff, fb, fw = (eager.forward(prob, m) for m in ("fp32", "bf16", "bf16w"))
    G = torch.randn(prob.x.shape, generator=torch.Generator().manual_seed(seed + 3))
    bf_, bb, bw = (eager.backward(prob, f_, G, m)
                   for f_, m in ((ff, "fp32"), (fb, "bf16"), (fw, "bf16w")))

    def mean_err(a, b):
        return ((a - b).abs().mean() / b.abs().mean()).item()

    pairs = [(fw["out"], fb["out"], ff["out"])] + [
        (bw[key], bb[key], bf_[key]) for key in ("grad_x", "grad_w1", "grad_w2")]
    for w_, b_, ref in pairs:
        assert mean_err(w_, ref) < 6e-3
        assert mean_err(w_, ref) <= 1.1 * mean_err(b_, ref) + 1e-4


def test_aux_losses_uniform_and_grouped():
    g = torch.Generator().manual_seed(0)
    L = torch.randn(50, 8, generator=g)
    tpe = [5, 7, 0, 10, 12, 6, 4, 6]
    a = eager.aux_losses(L, tpe, [64] * 8, [(8, 64)])
    p = torch.sigmoid(L.double())
    f = (torch.tensor(tpe, dtype=torch.float64) / sum(tpe)).to(torch.bfloat16).double()
    assert torch.allclose(a["load_balance_loss"], 8 * (f * p.mean(0)).sum())
    b = eager.aux_losses(L, tpe, [64] * 4 + [32] * 4, [(4, 64), (4, 32)])
    fp = f * p.mean(0)
    assert torch.allclose(b["load_balance_loss"], (4 * fp[:4].sum() + 4 * fp[4:].sum()) / 2)


@pytest.mark.parametrize("T,k,d,P", [(7, 3, 5, 30), (64, 8, 32, 700)])
def test_combine_weight_grad_matches_autograd(T, k, d, P):
    """The opt-in routing-weight gradient equals torch autograd of the fp32
    combine with respect to the weights (float64), slots without a row
    included; a transposed operand or a wrong slot index fails it."""
    g = torch.Generator().manual_seed(T * 31 + k)
    y = torch.randn(P, d, generator=g, dtype=torch.float64)
    G = torch.randn(T, d, generator=g, dtype=torch.float64)
    ar = torch.randperm(P, generator=g)[:T * k].clone()
    ar[::4] = -1
    w = torch.rand(T * k, generator=g, dtype=torch.float64).requires_grad_(True)
    out = eager.combine(y, ar.numpy(), w, k, T, "fp32")
    (out * G).sum().backward()
    got = eager.combine_weight_grad(G, y, ar.numpy(), k, T)
    assert torch.allclose(got, w.grad, rtol=1e-12, atol=1e-12)
    assert bool((got[::4] == 0).all())


def test_router_weight_logit_grad_gradcheck():
    """The routing weights' chain into the logits: torch.autograd.gradcheck
    (finite differences) of the weights for a fixed selection, normalised and
    not, and the closed form dp_j = (g_j - sum_i g_i w_i) / S, dL = dp p (1 - p)
    on the selected experts (0 elsewhere)."""
    g = torch.Generator().manual_seed(5)
    L = torch.randn(6, 10, generator=g, dtype=torch.float64)
    sel = torch.topk(L, 3, dim=-1).indices
    gw = torch.randn(6, 3, generator=g, dtype=torch.float64)
    for norm in (True, False):
        assert torch.autograd.gradcheck(
            lambda x: eager.router_weights(x, sel, norm), (L.clone().requires_grad_(True),))
        got = eager.router_weight_logit_grad(L, sel, gw, norm)
        p = torch.sigmoid(L).gather(1, sel)
        S = p.sum(-1, keepdim=True) + 1e-20
        dp = (gw - (gw * p / S).sum(-1, keepdim=True)) / S if norm else gw
        want = torch.zeros_like(L).scatter_(1, sel, dp * p * (1 - p))
        assert torch.allclose(got, want, rtol=1e-12, atol=1e-14)
        assert bool((got.gather(1, sel) != 0).all())
        assert int((got != 0).sum()) == sel.numel()


def test_module_weight_gradient_decomposes():
    """dL/dlogits of sum(out * G) through the fp32 oracle's forward with the
    weights a function of the logits equals router_weight_logit_grad of
    combine_weight_grad(G, y): the per-row gradient the module computes from
    the dH GEMM, then the router chain."""
    prob = _problem(3, 29, 12, [(2, 24), (3, 8)], 2, 8)
    g = torch.Generator().manual_seed(4)
    L = torch.randn(29, 5, generator=g, dtype=torch.float64)
    sel = prob.selected
    Lr = L.clone().requires_grad_(True)
    prob.weights = eager.router_weights(Lr, sel)
    fwd = eager.forward(prob, "fp32")
    G = torch.randn(fwd["out"].shape, generator=g, dtype=torch.float64)
    (fwd["out"] * G).sum().backward()
    r = fwd["route"]
    gw = eager.combine_weight_grad(G, fwd["y"].detach(), r["assignment_row"], 2, 29)
    got = eager.router_weight_logit_grad(L, sel, gw.view(29, 2))
    assert torch.allclose(got, Lr.grad, rtol=1e-10, atol=1e-12)


def test_swiglu_oracle_layout_and_silu():
    """swiglu_up against torch.nn.functional.silu on a dense single-expert
    problem and, for two experts of different widths, against column slices
    taken by hand: a swapped gate/up half or a wrong column offset fails it."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(12, 16, generator=g, dtype=torch.float64)
    w1 = torch.randn(16, 2 * 8 + 2 * 16, generator=g, dtype=torch.float64)
    h, gate = eager.swiglu_up(x[:5], w1[:, :16], [(0, 5)], [8], [0], 8)
    ref = torch.nn.functional.silu(x[:5] @ w1[:, :8]) * (x[:5] @ w1[:, 8:16])
    assert torch.allclose(h, ref, rtol=1e-12, atol=1e-12)
    assert torch.allclose(gate, x[:5] @ w1[:, :8], rtol=1e-12, atol=1e-12)
    rows, widths, offs = [(0, 5), (5, 12)], [8, 16], [0, 16]
    h2, _ = eager.swiglu_up(x, w1, rows, widths, offs, 16)
    ref1 = torch.nn.functional.silu(x[5:] @ w1[:, 16:32]) * (x[5:] @ w1[:, 32:48])
    assert torch.allclose(h2[5:], ref1, rtol=1e-12, atol=1e-12)
    assert torch.allclose(h2[:5, :8], ref, rtol=1e-12, atol=1e-12)
    assert (h2[:5, 8:] == 0).all()
