"""Router kernel (sigmoid, top-k, normalisation, auxiliary losses and their
gradient) against PyTorch and the float64 oracle (reference moe.py:166-182,
253-303).

Top-k: the reference routes with torch.topk(torch.sigmoid(L.float()), k),
normalised and rounded to bf16 (moe.py:168-176). The kernel is held to that
chain bit for bit on the same bf16 logits: probabilities, expert ids in slot
order (ties included: the order PyTorch's GPU sort leaves equal values in),
and bf16 weights (the sum in torch's reduction order).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import eager
from triton_moe import TritonMoEConfig, TritonMoEMLP
from triton_moe.kernels.router import RouterLinear, load_balance_coef, router_topk

from _util import LOOSE, assert_close_norm, bits_equal, make_problem

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "topk_cases.json"


def _logits(T, E, seed, ties):
    g = torch.Generator().manual_seed(seed)
    L = torch.randn(T, E, generator=g) * 1.5
    if ties:
        L = (L * 4).round() / 4  # many exactly equal logits per row
    return L.to(torch.bfloat16)


def _torch_chain(L, k, norm):
    """The reference's routing chain (moe.py:168-176) run by PyTorch."""
    probs = torch.sigmoid(L.float())
    w, sel = torch.topk(probs, k, dim=-1)
    if norm:
        w = w / (w.sum(dim=-1, keepdim=True) + 1e-20)
    return probs, w.to(L.dtype), sel


def _assert_same_routing(L, k, norm, what):
    st = router_topk(L, k, norm, want_probs=True, index_dtype=torch.int64)
    st32 = router_topk(L, k, norm)
    probs, w, sel = _torch_chain(L, k, norm)
    assert bits_equal(st.probs, probs), f"{what}: sigmoid bits"
    bad = (st.selected != sel).any(dim=1)
    assert int(bad.sum()) == 0, (
        f"{what}: {int(bad.sum())} of {L.shape[0]} tokens routed differently from torch.topk; "
        f"first {bad.nonzero()[:1].tolist()}")
    assert torch.equal(st32.selected.long(), sel), f"{what}: int32 ids"
    assert bits_equal(st.weights, w), f"{what}: bf16 weights"
    assert bits_equal(st32.weights, w), f"{what}: bf16 weights (int32 ids)"
    return st


@pytest.mark.parametrize("T,E,k,norm,ties", [
    (1000, 4, 2, True, False), (4096, 8, 2, True, True), (2048, 16, 4, False, True),
    (16384, 64, 8, True, False), (3000, 64, 8, True, True), (1024, 128, 8, True, True),
    (512, 1000, 16, True, False), (256, 2048, 8, False, True), (300, 7, 7, True, True),
    (333, 64, 1, True, False), (2000, 64, 3, True, True), (2000, 64, 5, True, True),
    (2000, 64, 6, True, True), (500, 40, 12, True, True), (400, 256, 16, True, True),
    (300, 64, 32, True, True), (200, 256, 48, True, True), (200, 96, 64, False, True)])
def test_router_topk_matches_torch(T, E, k, norm, ties, device):
    L = _logits(T, E, seed=T + E + k, ties=ties).to(device)
    st = _assert_same_routing(L, k, norm, f"T={T} E={E} k={k}")
    assert st.selected.shape == (T, k)
    # lse: bf16-rounded logsumexp of the bf16 logits
    lse_ref = torch.logsumexp(L.float(), dim=-1).to(torch.bfloat16).float()
    d = (st.lse - lse_ref).abs()
    assert bool((d <= lse_ref.abs() * 2.0 ** -7 + 1e-6).all())


# BASELINE configurations 1-4 (tokens, n_embd, experts, top-k); logits as the
# module makes them (bf16 nn.Linear of N(0,1) tokens with N(0,0.02) router
# weights); configuration 3 adds the benchmark's Zipf bias at alpha 1 and 3.
ROUTER_SHAPES = {
    "cfg1": (8192, 768, 8, 2, None),
    "cfg2": (16384, 768, 16, 2, None),
    "cfg3_a1": (16384, 1024, 64, 8, 1.0),
    "cfg3_a3": (16384, 1024, 64, 8, 3.0),
    "cfg4": (32768, 2048, 128, 8, None),
}


@pytest.mark.parametrize("name", list(ROUTER_SHAPES))
def test_router_topk_config_shapes(name, device):
    T, d, E, k, alpha = ROUTER_SHAPES[name]
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16).to(device)
    wr = (torch.randn(E, d, generator=g) * 0.02).to(torch.bfloat16).to(device)
    L = F.linear(x, wr)
    if alpha is not None:
        ranks = np.random.default_rng(0).permutation(E) + 1
        bias = torch.tensor(-1.2 * alpha * np.log(ranks), dtype=torch.float32)
        L = L + bias.to(torch.bfloat16).to(device)
    _assert_same_routing(L, k, True, name)


def test_router_sigmoid_every_bf16(device):
    """All 65536 bf16 patterns but NaN: the kernel's probabilities are
    torch.sigmoid's bits."""
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    L = bits.view(torch.bfloat16)
    L = torch.where(torch.isnan(L.float()), torch.zeros_like(L), L)
    L = L.reshape(1024, 64).to(device)
    st = router_topk(L, 8, True, want_probs=True)
    assert bits_equal(st.probs, torch.sigmoid(L.float()))


def test_router_topk_golden(device):
    """The recorded torch.topk chain on tie-heavy rows (tests/golden/topk_cases.json)."""
    data = json.loads(GOLDEN.read_text())
    for c in data["cases"]:
        lev = torch.tensor(c["levels_bf16"], dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
        L = lev[torch.tensor(c["idx"])].to(device)
        st = router_topk(L, c["k"], c["norm"], index_dtype=torch.int64)
        assert st.selected.cpu().tolist() == c["selected"], c["name"]
        wb = st.weights.cpu().view(torch.int16).to(torch.int32) & 0xFFFF
        assert wb.tolist() == c["weights_bf16"], c["name"]
        _assert_same_routing(L, c["k"], c["norm"], c["name"])


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
    """RouterLinear = nn.Linear(d, E, bias=False); with use_logits_kernel the
    kernel's logits are one bf16 rounding of the fp32 product (E = 7 is outside the kernel's shapes and
    runs nn.Linear's own path); gradients as the linear layer's; forward hooks
    still apply."""
    g = torch.Generator().manual_seed(T + d + E)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, d, generator=g) * 0.05).to(torch.bfloat16)
    lin = RouterLinear(d, E, bias=False).to(device).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(w)
    xd = x.to(device).requires_grad_(True)
    # default: nn.Linear's own logits, bit for bit
    with torch.no_grad():
        assert bits_equal(lin(xd), F.linear(xd, lin.weight))
    lin.use_logits_kernel = True
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


@pytest.mark.parametrize("T,E,k,norm", [(300, 64, 8, True), (257, 16, 2, True),
                                        (128, 40, 5, False), (64, 128, 33, True)])
def test_router_weight_bwd_vs_oracle(T, E, k, norm, device):
    """Opt-in routing-weight gradient into the logits (the reference has none,
    scatter.py:176) against float64 autograd of the reference's chain
    (sigmoid, gather of the selected, normalisation; moe.py:168-176) for the
    kernel's own selection: non-zero exactly on the selected experts, within
    bf16 rounding of the output elsewhere."""
    from triton_moe.kernels.router import RouterWeightOp

    L = _logits(T, E, seed=T + E, ties=False).to(device)
    for dt in (torch.int32, torch.int64):
        st = router_topk(L, k, norm, index_dtype=dt)
        Lg = L.clone().requires_grad_(True)
        w = RouterWeightOp.apply(Lg, st.weights, st.selected, norm)
        assert bits_equal(w, st.weights)
        gw = torch.randn(T, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
        w.backward(gw.to(device))
        ref = eager.router_weight_logit_grad(L.float().cpu(), st.selected.cpu(), gw.float(), norm)
        got = Lg.grad.float().cpu()
        mask = torch.zeros(T, E, dtype=torch.bool).scatter_(1, st.selected.long().cpu(), True)
        assert bool((got[~mask] == 0).all())
        # one bf16 rounding of an fp32 value, |d| <= 2^-8 |ref|, plus fp32
        # cancellation in g_j - sum_i g_i w_i, bounded by the gradient's scale
        d = (got - ref.float()).abs()
        bound = ref.abs().float() * 2.0 ** -8 + 1e-5 * ref.abs().max().float()
        assert bool((d <= bound).all()), float((d - bound).max())


HIST_SHAPES = {  # tokens, experts, k, Zipf alpha (None: plain logits)
    "cfg1": (8192, 8, 2, None),
    "cfg2": (16384, 16, 2, None),
    "cfg3_a1": (16384, 64, 8, 1.0),
    "cfg4": (32768, 128, 8, None),
    "partial_tile": (1000, 64, 8, None),
    "k4": (3001, 16, 4, 2.0),
    "k1": (333, 64, 1, None),
    "one_token": (1, 64, 8, None),
    "fallback_k3": (2000, 64, 3, None),
    "fallback_e256": (500, 256, 8, None),
}


@pytest.mark.parametrize("name", list(HIST_SHAPES))
def test_router_topk_hist_routes_like_two_launches(name, device):
    """router_topk(route_hist=True) + route_device(workspace=) (the top-k
    kernel counts each 1024-assignment tile, the routing skips its counting
    launch) gives the outputs of router_topk + route_device bit for bit; the
    workspace holds each tile's expert histogram; the auxiliary losses, whose
    per-token terms are then summed in other blocks, agree to fp32 rounding."""
    from triton_moe import _lib
    from triton_moe.kernels.fused_cumsum import route_device
    from triton_moe.kernels.router import RouterAuxOp

    T, E, k, alpha = HIST_SHAPES[name]
    L = _logits(T, E, seed=T + E, ties=True)
    if alpha is not None:
        ranks = np.random.default_rng(0).permutation(E) + 1
        L = (L.float() + torch.tensor(-1.2 * alpha * np.log(ranks))).to(torch.bfloat16)
    L = L.to(device)
    blocks = int(_lib.lib().vmoe_router_topk_hist_blocks(T, E, k))
    assert (blocks > 0) == (not name.startswith("fallback"))
    a = router_topk(L, k, True, want_probs=True, index_dtype=torch.int64)
    h = router_topk(L, k, True, want_probs=True, index_dtype=torch.int64, route_hist=True)
    for f in ("weights", "selected", "probs", "lse"):
        assert bits_equal(getattr(h, f), getattr(a, f)), f"{name}: {f}"
    if blocks == 0:
        assert h.route_ws is None
        return
    assert h.partial_rows == blocks
    A = T * k
    ntiles = -(-A // 1024)
    S = blocks // ntiles  # count columns per routing tile
    assert blocks == ntiles * S and S in (1, 2, 4, 8)
    span = 1024 // S
    counts = h.route_ws[:E * blocks].view(E, blocks).cpu()
    bad = h.route_ws[E * blocks:E * blocks + blocks].cpu()
    flat = a.selected.reshape(-1).cpu()
    for t in range(blocks):
        want = torch.bincount(flat[t * span:(t + 1) * span], minlength=E)
        assert torch.equal(counts[:, t], want.to(torch.int32)), f"{name}: block {t} histogram"
    assert int(bad.abs().sum()) == 0
    wf = a.weights.reshape(-1)
    r1 = route_device(a.selected.reshape(-1), E, k, 64, "up", map_pad=-1, weights=wf)
    r2 = route_device(h.selected.reshape(-1), E, k, 64, "up", map_pad=-1, weights=wf,
                      workspace=h.route_ws)
    torch.cuda.synchronize()
    P = int(r1.info[_lib.INFO_ROWS])
    assert torch.equal(r1.info, r2.info)
    for f in ("bin_ids", "indices", "tokens_per_expert", "bins", "padded_bins",
              "assignment_row", "expert_offsets", "padded_counts"):
        assert torch.equal(getattr(r1, f), getattr(r2, f)), f"{name}: {f}"
    for f in ("row_src", "gather_map", "row_weight"):
        assert bits_equal(getattr(r1, f)[:P], getattr(r2, f)[:P]), f"{name}: {f}"
    # auxiliary losses from the two blockings of the per-token sums
    coef = torch.full((E,), float(E), device=device)
    wn = torch.ones(E, device=device)
    la = RouterAuxOp.apply(L, a.lse, a.partial, a.partial_rows, r1.tokens_per_expert, coef, wn)
    lh = RouterAuxOp.apply(L, h.lse, h.partial, h.partial_rows, r2.tokens_per_expert, coef, wn)
    # z_loss is bf16 (one rounding step apart at most), the two losses fp32
    # sums of T terms, f_i a function of the counts alone
    for x, y, what, rtol in zip(la, lh, ("z", "lb", "cl", "f_i"), (2.0 ** -7, 1e-5, 1e-5, 0)):
        assert torch.allclose(x.float(), y.float(), rtol=rtol, atol=0), f"{name}: aux {what}"
