"""Router kernel (sigmoid, top-k, normalisation, auxiliary losses and their
gradient) against PyTorch and the float64 oracle (reference moe.py:166-182,
253-303).

Top-k: torch.topk leaves the order of equal values open, so the test checks
the properties that define a top-k (the selected values are the k largest,
in descending order) plus this build's tie rule (ascending expert index), and
compares values and weights with torch on the same probabilities.
"""

from __future__ import annotations

import pytest
import torch

from oracle import eager
from triton_moe import TritonMoEConfig, TritonMoEMLP
from triton_moe.kernels.router import RouterLinear, load_balance_coef, router_topk

from _util import LOOSE, assert_close_norm, bits_equal, make_problem

pytestmark = pytest.mark.gpu


def _logits(T, E, seed, ties):
    g = torch.Generator().manual_seed(seed)
    L = torch.randn(T, E, generator=g) * 1.5
    if ties:
        L = (L * 4).round() / 4  # many exactly equal logits per row
    return L.to(torch.bfloat16)


@pytest.mark.parametrize("T,E,k,norm,ties", [
    (1000, 4, 2, True, False), (4096, 8, 2, True, True), (2048, 16, 4, False, True),
    (16384, 64, 8, True, False), (3000, 64, 8, True, True), (1024, 128, 8, True, True),
    (512, 1000, 16, True, False), (256, 2048, 8, False, True), (300, 7, 7, True, True),
    (333, 64, 1, True, False)])
def test_router_topk_is_a_topk(T, E, k, norm, ties, device):
    L = _logits(T, E, seed=T + E + k, ties=ties).to(device)
    st = router_topk(L, k, norm, want_probs=True, index_dtype=torch.int64)
    st32 = router_topk(L, k, norm)
    assert torch.equal(st32.selected.long(), st.selected)
    assert bits_equal(st32.weights, st.weights)
    p_ref = torch.sigmoid(L.float())
    torch.testing.assert_close(st.probs, p_ref, rtol=1e-6, atol=1e-7)
    p = st.probs
    sel = st.selected
    assert sel.shape == (T, k) and int(sel.min()) >= 0 and int(sel.max()) < E
    # distinct experts per token
    srt = sel.sort(dim=1).values
    assert bool((srt[:, 1:] != srt[:, :-1]).all())
    vals = p.gather(1, sel)
    if k > 1:
        a, b = vals[:, :-1], vals[:, 1:]
        ia, ib = sel[:, :-1], sel[:, 1:]
        assert bool(((a > b) | ((a == b) & (ia < ib))).all()), "descending, ties by index"
    # the k largest: nothing unselected beats the k-th value, and an equal
    # unselected value has a larger index than the selected ones equal to it
    kth = vals[:, -1:]
    unsel = torch.ones_like(p, dtype=torch.bool).scatter_(1, sel, False)
    assert bool((p.masked_fill(~unsel, -1.0) <= kth).all())
    idx = torch.arange(E, device=device).expand(T, E)
    tie_sel = (~unsel) & (p == kth)
    tie_uns = unsel & (p == kth)
    max_sel = idx.masked_fill(~tie_sel, -1).max(dim=1).values
    min_uns = idx.masked_fill(~tie_uns, E).min(dim=1).values
    assert bool((min_uns > max_sel).all())
    # torch.topk picks the same values (its tie order aside)
    tv = torch.topk(p, k, dim=-1).values
    assert torch.equal(tv, vals)
    # weights: the reference's normalisation of the selected values
    w_ref = vals / (vals.sum(dim=-1, keepdim=True) + 1e-20) if norm else vals
    d = (st.weights.float() - w_ref.to(torch.bfloat16).float()).abs()
    ulp = w_ref.to(torch.bfloat16).float().abs() * 2.0 ** -7
    assert bool((d <= ulp).all())
    # lse: bf16-rounded logsumexp of the bf16 logits
    lse_ref = torch.logsumexp(L.float(), dim=-1).to(torch.bfloat16).float()
    d = (st.lse - lse_ref).abs()
    assert bool((d <= lse_ref.abs() * 2.0 ** -7 + 1e-6).all())


AUX_CASES = {
    "uniform": (2048, 256, [(16, 256)], 4),
    "grouped": (4096, 256, [(4, 512), (8, 256), (4, 128)], 2),
    "lone_experts": (2048, 128, [(1, 256), (1, 128), (1, 64)], 2),
    "mixed": (2048, 128, [(1, 512), (6, 256), (3, 128)], 3),
}


def _module(name, device, seed=0):
    T, d, sizes, k = AUX_CASES[name]
    p = make_problem(T, d, sizes, k, 64, seed=seed, device=device)
    cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=64)
    m = TritonMoEMLP(cfg).to(device).to(torch.bfloat16)
    with torch.no_grad():
        m.router.weight.copy_(p["wr"])
        m.w1.copy_(p["w1"])
        m.w2.copy_(p["w2"])
    return m, p


@pytest.mark.parametrize("name", list(AUX_CASES))
def test_aux_losses_vs_oracle(name, device):
    m, p = _module(name, device)
    T, d, sizes, k = AUX_CASES[name]
    x = p["x"].view(1, T, d).to(device)
    out, aux, f_i = m(x)
    with torch.no_grad():
        logits = m.router(x.reshape(T, d))
        _, _, wts, sel = m._router(x.reshape(T, d))
    tpe = torch.bincount(sel.reshape(-1), minlength=sum(c for c, _ in sizes)).cpu().numpy()
    ref = eager.aux_losses(logits.float().cpu(), tpe, p["widths"], sizes)
    assert f_i.dtype == torch.bfloat16 and torch.equal(f_i.cpu(), ref["f_i"])
    assert aux["router_z_loss"].dtype == torch.bfloat16
    assert aux["load_balance_loss"].dtype == torch.float32
    assert aux["compute_loss"].dtype == torch.float32
    # z_loss carries the bf16 rounding of the reference's bf16 chain (2^-8
    # relative); the other two are fp32 sums of the same terms.
    for key, tol in (("router_z_loss", 1e-2), ("load_balance_loss", 1e-4),
                     ("compute_loss", 1e-4)):
        got, want = float(aux[key].detach()), float(ref[key])
        assert abs(got - want) <= tol * abs(want) + 1e-7, (key, got, want)
    # the coefficient form equals the reference's three formulas
    coef = torch.tensor(load_balance_coef(sizes), dtype=torch.float64)
    pr = torch.sigmoid(logits.double().cpu()).mean(0)
    lb = float((coef * ref["f_i"].double() * pr).sum())
    assert abs(lb - float(ref["load_balance_loss"])) <= 1e-9 * max(1.0, abs(lb))


@pytest.mark.parametrize("name", ["uniform", "grouped", "mixed"])
def test_aux_losses_backward_vs_oracle(name, device):
    """Router weight gradient of 0.7 z + 0.2 lb + 0.1 cl against float64
    autograd through the oracle's loss formulas on the same logits."""
    m, p = _module(name, device, seed=1)
    T, d, sizes, k = AUX_CASES[name]
    x = p["x"].view(1, T, d).to(device)
    out, aux, f_i = m(x)
    loss = 0.7 * aux["router_z_loss"].float() + 0.2 * aux["load_balance_loss"] \
        + 0.1 * aux["compute_loss"]
    loss.backward()
    with torch.no_grad():
        logits = m.router(x.reshape(T, d)).float().cpu()
        _, _, _, sel = m._router(x.reshape(T, d))
    tpe = torch.bincount(sel.reshape(-1), minlength=sum(c for c, _ in sizes)).cpu().numpy()
    L = logits.double().requires_grad_(True)
    ref = eager.aux_losses(L, tpe, p["widths"], sizes)
    (0.7 * ref["router_z_loss"] + 0.2 * ref["load_balance_loss"]
     + 0.1 * ref["compute_loss"]).backward()
    gw_ref = L.grad.T @ p["x"].double()
    assert_close_norm(m.router.weight.grad, gw_ref, LOOSE, f"{name} router.weight.grad")
    # no gradient reaches the expert weights through the auxiliary losses
    assert m.w1.grad is None and m.w2.grad is None


def test_router_deterministic(device):
    L = _logits(8192, 64, seed=5, ties=True).to(device)
    a = router_topk(L, 8, True)
    b = router_topk(L, 8, True)
    assert torch.equal(a.selected, b.selected) and bits_equal(a.weights, b.weights)
    assert torch.equal(a.partial, b.partial) and torch.equal(a.lse, b.lse)


@pytest.mark.parametrize("T,d,E", [(16384, 1024, 64), (1000, 768, 8), (333, 2048, 128),
                                   (512, 256, 16), (97, 512, 24), (64, 64, 8), (4096, 768, 7)])
def test_router_linear(T, d, E, device):
    """RouterLinear = nn.Linear(d, E, bias=False): the kernel's logits are one
    bf16 rounding of the fp32 product (E = 7 is outside the kernel's shapes and
    runs nn.Linear's own path); gradients as the linear layer's; forward hooks
    still apply."""
    g = torch.Generator().manual_seed(T + d + E)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, d, generator=g) * 0.05).to(torch.bfloat16)
    lin = RouterLinear(d, E, bias=False).to(device).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(w)
    xd = x.to(device).requires_grad_(True)
    out = lin(xd)
    assert out.shape == (T, E) and out.dtype == torch.bfloat16
    ref = x.float() @ w.float().t()
    bound = ref.abs() * 2.0 ** -8 + (x.float().abs() @ w.float().abs().t()) * 2.0 ** -20
    assert bool(((out.float().cpu() - ref).abs() <= bound).all())
    gout = torch.randn(T, E, generator=g).to(torch.bfloat16)
    out.backward(gout.to(device))
    assert_close_norm(xd.grad, gout.float() @ w.float(), LOOSE, "router x.grad")
    assert_close_norm(lin.weight.grad, gout.float().t() @ x.float(), LOOSE, "router weight.grad")
    h = lin.register_forward_hook(lambda mod, inp, o: o + 1.0)
    with torch.no_grad():
        assert torch.equal(lin(xd), (out + 1.0).detach())
    h.remove()
    # a [B, S, d] input keeps its leading shape
    assert lin(xd.detach().reshape(1, T, d)).shape == (1, T, E)
