"""A float32 TritonMoEMLP on the fp32 kernels, against the fp32 eager oracle.

The reference builds its module in float32 for training validation
(benchmarks/validate_training.py: `TritonMoEMLP(cfg).to(device).to(torch.float32)`,
n_embd 128, 4 experts of 256, k = 2, block 128, batch 4 x 64, Adam on an MSE
loss). Here the same module runs the fp32 router kernels (sigmoid, top-k,
normalisation, auxiliary losses), the routing, the fp32 grouped GEMMs and the
fp32 permutation kernels. Its routing is first held to the reference's chain
run by PyTorch on the same fp32 logits; the oracle is then fed that chain's
decision and the outputs and gradients must agree within 1e-4 normwise (max)
and 1e-5 (mean): fp32 arithmetic in another summation order.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import eager
from triton_moe import TritonMoEConfig, TritonMoEMLP

from _util import assert_close_norm

pytestmark = pytest.mark.gpu

F32_TOL = (1e-4, 1e-5)

# name: (batch, seq, n_embd, expert_sizes, top_k, block_size)
SHAPES = {
    "validate_training": (4, 64, 128, [(4, 256)], 2, 128),
    "ref_variable": (4, 256, 256, [(4, 512), (4, 256)], 2, 128),
    "cfg2_small": (2, 512, 768, [(4, 512), (8, 256), (4, 128)], 2, 64),
    "k8_64": (1, 2048, 256, [(64, 128)], 8, 64),
    # hidden and offsets off every vector width (rows of 98 floats are 8-byte
    # aligned at best), widths of 4 to 20 (blocks of 4 rows), an odd top_k
    "unaligned": (1, 300, 98, [(3, 12), (2, 20), (1, 4)], 3, 4),
}


def _model(d, sizes, k, b, device, seed=42):
    torch.manual_seed(seed)
    cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=b)
    return TritonMoEMLP(cfg).to(device).to(torch.float32)


def _reference_routing(m, x_flat, k):
    """The reference's routing chain in PyTorch (moe.py:166-176), fp32."""
    with torch.no_grad():
        logits = F.linear(x_flat, m.router.weight)
        probs = torch.sigmoid(logits.float())
        w, sel = torch.topk(probs, k, dim=-1)
        w = w / (w.sum(dim=-1, keepdim=True) + 1e-20)
    return logits, w, sel


def _problem(m, x_flat, sel, w, b):
    return eager.Problem(x_flat.detach().cpu().float(), m.w1.detach().cpu().float(),
                         m.w2.detach().cpu().float(), m.expert_widths, m.expert_offsets,
                         sel.cpu(), w.cpu().float(), b)


@pytest.mark.parametrize("name", list(SHAPES))
def test_f32_module_forward_backward_vs_oracle(name, device):
    B, S, d, sizes, k, b = SHAPES[name]
    m = _model(d, sizes, k, b, device)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, S, d, generator=g).to(device).requires_grad_(True)
    out, aux, f_i = m(x)
    assert out.dtype == torch.float32 and f_i.dtype == torch.float32
    G = torch.randn(B, S, d, generator=g)
    out.backward(G.to(device))
    x_flat = x.detach().reshape(-1, d)
    logits, w_ref, sel_ref = _reference_routing(m, x_flat, k)
    with torch.no_grad():
        lg, probs, w_mod, sel_mod = m._router(x_flat)
    assert torch.equal(lg, logits)
    assert torch.equal(sel_mod, sel_ref), f"{name}: routing differs from the reference chain"
    assert w_mod.dtype == torch.float32
    assert ((w_mod - w_ref).abs() <= 2e-7 * w_ref.abs() + 1e-12).all(), name
    assert torch.allclose(probs, torch.sigmoid(logits), rtol=2e-7, atol=0)
    prob = _problem(m, x_flat, sel_ref, w_ref, b)
    ff = eager.forward(prob, "fp32")
    T = B * S
    Gf = G.reshape(T, d).float()
    bf = eager.backward(prob, ff, Gf, "fp32")
    assert_close_norm(out.detach().reshape(T, d), ff["out"], F32_TOL, f"{name} out")
    for got, key in ((x.grad.reshape(T, d), "grad_x"), (m.w1.grad, "grad_w1"),
                     (m.w2.grad, "grad_w2")):
        assert got.dtype == torch.float32
        assert_close_norm(got, bf[key], F32_TOL, f"{name} {key}")
    assert m.router.weight.grad is None
    ref = eager.aux_losses(logits.cpu(), ff["route"]["tokens_per_expert"], m.expert_widths,
                           sizes, dtype=torch.float32)
    assert torch.equal(f_i.cpu(), ref["f_i"])
    for key in ("router_z_loss", "load_balance_loss", "compute_loss"):
        assert aux[key].dtype == torch.float32, key
        assert abs(aux[key].item() - ref[key].item()) <= 1e-5 * abs(ref[key].item()) + 1e-7, key


def test_f32_aux_loss_gradient(device):
    """The auxiliary losses differentiate into the fp32 router logits like
    float64 autograd of the oracle's formulas."""
    B, S, d, sizes, k, b = SHAPES["ref_variable"]
    m = _model(d, sizes, k, b, device)
    x = torch.randn(B, S, d, generator=torch.Generator().manual_seed(3)).to(device)
    store = {}

    def hook(mod, inp, out):
        out.register_hook(lambda gl: store.__setitem__("g", gl))
        store["logits"] = out.detach()
        return out

    m.router.register_forward_hook(hook)
    out, aux, f_i = m(x)
    (aux["router_z_loss"] * 0.5 + aux["load_balance_loss"] * 2.0 +
     aux["compute_loss"] * 0.25).backward()
    L = store["logits"].cpu().double().requires_grad_(True)
    tpe = torch.bincount(torch.topk(torch.sigmoid(store["logits"]), k, dim=-1).indices.reshape(-1),
                         minlength=m.num_experts).cpu()
    ref = eager.aux_losses(L, tpe, m.expert_widths, sizes, dtype=torch.float32)
    (ref["router_z_loss"] * 0.5 + ref["load_balance_loss"] * 2.0 +
     ref["compute_loss"] * 0.25).backward()
    assert store["g"].dtype == torch.float32
    assert_close_norm(store["g"], L.grad, F32_TOL, "aux logit gradient")


def test_f32_routing_weight_grad(device):
    """TritonMoEConfig(routing_weight_grad=True) in fp32: the logit gradient
    of the output through the weights, held to float64 autograd of the
    reference's chain (sigmoid, top-k, normalise, weighted combine of the
    oracle's fp32 Y)."""
    B, S, d, sizes, k, b = SHAPES["validate_training"]
    torch.manual_seed(42)
    cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=b,
                          routing_weight_grad=True)
    m = TritonMoEMLP(cfg).to(device).to(torch.float32)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, S, d, generator=g).to(device)
    store = {}

    def hook(mod, inp, out):
        out.register_hook(lambda gl: store.__setitem__("g", gl))
        return out

    m.router.register_forward_hook(hook)
    out, _, _ = m(x)
    G = torch.randn(B, S, d, generator=g)
    out.backward(G.to(device))
    T = B * S
    x_flat = x.reshape(T, d)
    logits, w_ref, sel_ref = _reference_routing(m, x_flat, k)
    prob = _problem(m, x_flat, sel_ref, w_ref, b)
    ff = eager.forward(prob, "fp32")
    gw = eager.combine_weight_grad(G.reshape(T, d).float(), ff["y"], ff["route"]["assignment_row"],
                                   k, T).view(T, k)
    ref = eager.router_weight_logit_grad(logits.cpu().float(), sel_ref.cpu(), gw)
    assert store["g"].dtype == torch.float32
    assert_close_norm(store["g"], ref, F32_TOL, "routing-weight logit gradient")


def test_f32_training_tracks_oracle(device):
    """validate_training's loop (Adam 1e-3 on an MSE loss, fresh N(0, 1)
    inputs and targets each step) for 10 steps, beside a twin whose gradients
    come from the fp32 oracle (routing from the reference's chain on the
    twin's own weights): per-step losses within 1e-5 relative, and w1 / w2
    within 1e-4 normwise at the end."""
    B, S, d, sizes, k, b = SHAPES["validate_training"]
    m = _model(d, sizes, k, b, device)
    twin_w1 = torch.nn.Parameter(m.w1.detach().cpu().clone())
    twin_w2 = torch.nn.Parameter(m.w2.detach().cpu().clone())
    opt = torch.optim.Adam(m.parameters(), lr=1e-3)
    opt_t = torch.optim.Adam([twin_w1, twin_w2], lr=1e-3)
    T = B * S
    for step in range(10):
        torch.manual_seed(42 + step)
        x = torch.randn(B, S, d, device=device)
        target = torch.randn(B, S, d, device=device)
        opt.zero_grad()
        out, _, _ = m(x)
        loss = F.mse_loss(out, target)
        loss.backward()
        opt.step()
        # twin: the same step through the oracle
        logits, w_ref, sel_ref = _reference_routing(m, x.reshape(T, d), k)
        prob = eager.Problem(x.reshape(T, d).cpu(), twin_w1.detach(), twin_w2.detach(),
                             m.expert_widths, m.expert_offsets, sel_ref.cpu(), w_ref.cpu(), b)
        ff = eager.forward(prob, "fp32")
        tgt = target.reshape(T, d).cpu()
        loss_t = F.mse_loss(ff["out"], tgt)
        gout = 2.0 * (ff["out"] - tgt) / ff["out"].numel()
        bf = eager.backward(prob, ff, gout, "fp32")
        opt_t.zero_grad()
        twin_w1.grad, twin_w2.grad = bf["grad_w1"].clone(), bf["grad_w2"].clone()
        opt_t.step()
        assert abs(loss.item() - loss_t.item()) <= 1e-5 * loss_t.item(), (step, loss.item(),
                                                                          loss_t.item())
    assert_close_norm(m.w1.detach(), twin_w1.detach(), F32_TOL, "w1 after 10 steps")
    assert_close_norm(m.w2.detach(), twin_w2.detach(), F32_TOL, "w2 after 10 steps")
