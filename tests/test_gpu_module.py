"""TritonMoEMLP on the GPU against the eager per-expert-loop oracle.

Protocol: the module's routing (logits, expert ids in slot order, bf16
weights) is first checked bit for bit against the reference's routing chain
run by PyTorch on the same inputs (nn.Linear, sigmoid, torch.topk,
normalisation, moe.py:166-176); the oracle then consumes that decision,
upcasts the bf16 parameters exactly to fp32, and detaches
the routing weights (the reference gives them no gradient, scatter.py:176).
Tolerances are normwise (max|d|/max|ref|, mean|d|/mean|ref|): TIGHT against
the oracle rounding to bf16 where the module does (mode "bf16w": the routing
weight applied to H, the same products as the reference with other rounding
points), LOOSE against the unrounded fp32 oracle.
"""

from __future__ import annotations

import contextlib

import numpy as np
import pytest
import torch

from oracle import eager
from triton_moe import TritonMoEConfig, TritonMoEMLP

from _util import (LOOSE, TIGHT, assert_close_norm, bf16_ulps, bits_equal, make_problem,
                   parity_stats, zipf_bias)

pytestmark = pytest.mark.gpu

# name: (batch, seq, n_embd, expert_sizes, top_k, block_size, Zipf alpha or None)
CONFIGS = {
    "ref_small": (2, 64, 128, [(4, 256)], 2, 128, None),
    "ref_uniform": (4, 256, 256, [(8, 512)], 2, 128, None),
    "ref_variable": (4, 256, 256, [(4, 512), (4, 256)], 2, 128, None),
    "cfg0_shape": (8, 512, 256, [(8, 512)], 2, 64, None),
    "cfg1": (8, 1024, 768, [(8, 512)], 2, 64, None),
    "cfg2": (8, 2048, 768, [(4, 512), (8, 256), (4, 128)], 2, 64, None),
    "cfg3": (1, 16384, 1024, [(64, 256)], 8, 64, 3.0),
    "cfg3_a1": (1, 16384, 1024, [(64, 256)], 8, 64, 1.0),  # the benchmark's alpha
    # more than 64 experts: the layer's auxiliary losses take a launch of their
    # own instead of riding in the routing launch
    "e128": (2, 1024, 256, [(96, 128), (32, 64)], 4, 64, 1.0),
    "one_token": (1, 1, 256, [(2, 256), (2, 128)], 2, 64, None),
    # hidden a multiple of 8 only (every K = hidden loop ends in a partial
    # stage), widths that cut the 256-wide tiles, top_k 1 and an odd top_k,
    # token counts that fill no tile
    "odd_k1": (1, 300, 200, [(3, 64), (2, 128)], 1, 64, 2.0),
    "odd_k3": (3, 100, 136, [(5, 64), (3, 192)], 3, 64, None),
}


def _module(p, d, sizes, k, b, device):
    cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=b)
    m = TritonMoEMLP(cfg).to(device).to(torch.bfloat16)
    with torch.no_grad():
        m.router.weight.copy_(p["wr"])
        m.w1.copy_(p["w1"])
        m.w2.copy_(p["w2"])
    return m


def _run(name, device, seed=0):
    B, S, d, sizes, k, b, alpha = CONFIGS[name]
    E = sum(c for c, _ in sizes)
    bias = zipf_bias(E, alpha=alpha) if alpha is not None else None
    p = make_problem(B * S, d, sizes, k, b, seed=seed, skew=bias, device=device)
    m = _module(p, d, sizes, k, b, device)
    if bias is not None:
        m.router.register_forward_hook(lambda mod, inp, out: out + bias.to(out.device, out.dtype))
    x = p["x"].view(B, S, d).to(device).requires_grad_(True)
    out, aux, f_i = m(x)
    with torch.no_grad():
        logits, _, wts, sel = m._router(x.detach().reshape(-1, d))
    # The module routes exactly as the reference's chain on the same inputs
    # (logits, expert ids in slot order, bf16 weights); the oracle is fed
    # that chain's decision.
    assert bits_equal(logits, p["logits"]), f"{name}: router logits"
    bad = int((sel != p["sel"]).any(dim=1).sum())
    assert bad == 0, f"{name}: {bad} tokens routed differently from the reference chain"
    assert bits_equal(wts, p["wts"]), f"{name}: routing weights"
    prob = eager.Problem(p["x"].float(), p["w1"].float(), p["w2"].float(), p["widths"],
                         p["offsets"], p["sel"].cpu(), p["wts"].cpu().float(), b)
    return m, x, out, aux, f_i, prob


def term_magnitudes(prob, fb, bb) -> dict:
    """For out, grad_x, grad_w1 and grad_w2: the sum of the magnitudes of the
    products each element sums, through the last GEMM before it (out[t] sums
    the rows H'_e W2_e of its slots, so its magnitude is the slots' |H'_e| |W2_e|;
    grad_x likewise with |GA_e| |W1_e^T|; grad_w1 = |X_e^T| |GA_e|,
    grad_w2 = |H'_e^T| |G_e|), from the bf16w oracle's intermediates."""
    r = fb["route"]
    T, d = prob.x.shape
    k = prob.top_k
    P = r["P"]
    ya = torch.zeros(P, d)
    gxa = torch.zeros(P, d)
    w1a = torch.zeros_like(prob.w1)
    w2a = torch.zeros_like(prob.w2)
    h, ga, xg, gy = fb["h"].abs(), bb["grad_a"].abs(), fb["x_gathered"].abs(), bb["grad_y"].abs()
    for e, (w, o) in enumerate(zip(prob.widths, prob.offsets)):
        r0 = int(r["padded_bins"][e - 1]) if e else 0
        r1 = int(r["padded_bins"][e])
        if r1 == r0:
            continue
        ya[r0:r1] = h[r0:r1, :w] @ prob.w2[o:o + w].abs()
        gxa[r0:r1] = ga[r0:r1, :w] @ prob.w1[:, o:o + w].abs().T
        w1a[:, o:o + w] = xg[r0:r1].T @ ga[r0:r1, :w]
        w2a[o:o + w] = h[r0:r1, :w].T @ gy[r0:r1]
    return {"out": eager.combine(ya, r["assignment_row"], None, k, T, "fp32"),
            "grad_x": eager.combine(gxa, r["assignment_row"], None, k, T, "fp32"),
            "grad_w1": w1a, "grad_w2": w2a}


def _assert_ulp_level(got, ref, mag, what, ulp1=0.999, ulp2=0.9995):
    """The module against the oracle that rounds where it does: at least
    99.9 % of the elements within 1 bf16 ulp and 99.95 % within 2 (by
    default), and every element within 4 of its conditioned error
    (|d| - ulp) / (2^-8 M), M the magnitudes of the terms it sums: elements
    whose sums cancel (their ulp distance can be large, a few flip sign near
    zero) are held to the rounding of their terms."""
    st = parity_stats(got, ref, mag)
    assert st["ulp1"] >= ulp1 and st["ulp2"] >= ulp2 and st["cond"] <= 4.0, (what, st)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_forward_backward_vs_oracle(name, device):
    m, x, out, aux, f_i, prob = _run(name, device)
    T, d = prob.x.shape
    assert out.shape == x.shape and out.dtype == torch.bfloat16
    # The module rounds in the "bf16w" order (routing weight applied to H,
    # so the combine and the backward need no weighted copies): held to the
    # oracle in that order with only summation order free, and to the
    # unrounded fp32 oracle with the bf16 tolerance.
    fb = eager.forward(prob, "bf16w")
    ff = eager.forward(prob, "fp32")
    o = out.detach().reshape(T, d)
    assert_close_norm(o, fb["out"], TIGHT, f"{name} out vs bf16w oracle")
    assert_close_norm(o, ff["out"], LOOSE, f"{name} out vs fp32 oracle")
    # upstream gradient: random (exercises the weighted gather) for small
    # configs, ones (out.sum()) for the large ones
    if T <= 4096:
        G = torch.randn(T, d, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
        out.backward(G.to(device).view_as(out))
    else:
        G = torch.ones(T, d, dtype=torch.bfloat16)
        out.sum().backward()
    bb = eager.backward(prob, fb, G.float(), "bf16w")
    bf_ = eager.backward(prob, ff, G.float(), "fp32")
    for got, key in ((x.grad.reshape(T, d), "grad_x"), (m.w1.grad, "grad_w1"),
                     (m.w2.grad, "grad_w2")):
        assert_close_norm(got, bb[key], TIGHT, f"{name} {key} vs bf16w oracle")
        assert_close_norm(got, bf_[key], LOOSE, f"{name} {key} vs fp32 oracle")
    assert m.router.weight.grad is None
    mags = term_magnitudes(prob, fb, bb)
    _assert_ulp_level(o, fb["out"], mags["out"], f"{name} out")
    for got, key in ((x.grad.reshape(T, d), "grad_x"), (m.w1.grad, "grad_w1"),
                     (m.w2.grad, "grad_w2")):
        _assert_ulp_level(got, bb[key], mags[key], f"{name} {key}")


@pytest.mark.parametrize("name", ["ref_variable", "cfg1"])
def test_broadcast_gradient_scale(name, device):
    """A loss c * out.sum() hands the backward a broadcast scalar c: the dH
    and dW2 GEMMs read a row of ones and scale by c on the device. Held to the
    oracle with G = c everywhere (c = 0.75, not a power of two)."""
    m, x, out, aux, f_i, prob = _run(name, device)
    T, d = prob.x.shape
    (out.sum() * 0.75).backward()
    fb = eager.forward(prob, "bf16w")
    bb = eager.backward(prob, fb, torch.full((T, d), 0.75), "bf16w")
    for got, key in ((x.grad.reshape(T, d), "grad_x"), (m.w1.grad, "grad_w1"),
                     (m.w2.grad, "grad_w2")):
        assert_close_norm(got, bb[key], TIGHT, f"{name} {key} with c = 0.75")


def test_aux_losses_and_f_i(device):
    m, x, out, aux, f_i, prob = _run("cfg2", device)
    with torch.no_grad():
        logits = m.router(x.detach().reshape(-1, x.shape[-1]))
    r = eager.route(prob)
    ref = eager.aux_losses(logits.float().cpu(), r["tokens_per_expert"], prob.widths,
                           CONFIGS["cfg2"][3])
    assert torch.equal(f_i.cpu(), ref["f_i"])
    # router_z_loss is computed from the bf16 router logits (logsumexp and the
    # square stay in bf16, as in the reference), so it carries bf16 rounding
    # (relative 2^-8); the other two are fp32 reductions.
    rel = {"router_z_loss": 1e-2, "load_balance_loss": 1e-3, "compute_loss": 1e-3}
    for key, tol in rel.items():
        assert abs(aux[key].item() - ref[key].item()) <= tol * abs(ref[key].item()) + 1e-6, key


def test_forward_with_intermediates(device):
    m, x, out, aux, f_i, prob = _run("ref_variable", device)
    with torch.no_grad():
        inter = m.forward_with_intermediates(x.detach())
    r = eager.route(prob)
    for key in ("bin_ids", "indices", "tokens_per_expert", "bins", "padded_bins"):
        assert torch.equal(inter[key].cpu(), torch.from_numpy(r[key])), key
    fb = eager.forward(prob, "bf16", r)
    assert bits_equal(inter["x_gathered"], fb["x_gathered"].to(torch.bfloat16))
    assert_close_norm(inter["x_after_up"], fb["h"], TIGHT, "x_after_up")
    assert_close_norm(inter["x_after_down"], fb["y"], TIGHT, "x_after_down")
    assert_close_norm(inter["output"].reshape(fb["out"].shape), fb["out"], TIGHT, "output")
    # the public-API path rounds in the reference's order, the fused module
    # path with the routing weight on H: the same products, to bf16 accuracy
    assert_close_norm(out.detach().reshape(fb["out"].shape), fb["out"], LOOSE,
                      "module vs public-API order")
    assert set(inter) >= {"x_flat", "router_logits", "router_probs", "top_k_weights",
                          "top_k_weights_flat", "selected_experts", "selected_experts_flat",
                          "x_scattered"}


def test_forward_deterministic(device):
    m, x, out1, _, _, _ = _run("cfg1", device)
    out1.sum().backward()
    g1 = (x.grad.clone(), m.w1.grad.clone(), m.w2.grad.clone())
    x.grad = None
    m.zero_grad(set_to_none=True)
    out2, _, _ = m(x)
    out2.sum().backward()
    assert bits_equal(out1, out2)
    for a, b in zip(g1, (x.grad, m.w1.grad, m.w2.grad)):
        assert bits_equal(a, b)


@pytest.mark.parametrize("fused", [True, False])
def test_backward_twice_with_retain_graph(fused, device):
    """backward(retain_graph=True) twice through one forward: the backward
    only reads what the forward saved, so the second pass gives the first
    pass's gradients again and the accumulated .grad is exactly twice them
    (x, w1, w2 and, through the auxiliary losses, the router weight)."""
    from triton_moe.kernels import grouped_gemm as gg

    gg.FUSED_EXPERT_PATH = fused
    try:
        m, x, out, aux, _, _ = _run("ref_variable", device)
        G = torch.randn(x.shape, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
        loss = (out.float() * G.to(device).float()).sum() + sum(aux.values())
        params = (x, m.w1, m.w2, m.router.weight)
        loss.backward(retain_graph=True)
        first = [p.grad.clone() for p in params]
        loss.backward()
        torch.cuda.synchronize()
        for p, g1, what in zip(params, first, ("x", "w1", "w2", "router")):
            assert torch.isfinite(g1.float()).all() and int(torch.count_nonzero(g1)) > 0, what
            assert bits_equal(p.grad, g1 * 2), what
    finally:
        gg.FUSED_EXPERT_PATH = True


@pytest.mark.parametrize("fused", [True, False])
def test_column_slice_input_same_bits(fused, device):
    """An input that is a column slice of a wider tensor (rows start 2 bytes
    past a 16-byte boundary) gives the bits of the same values stored
    contiguously: output, losses and every gradient (the GEMMs' operands are
    copied to aligned rows first). The router Linear is fed a contiguous copy
    in both runs, since hipBLASLt may pick another kernel for another layout."""
    from triton_moe.kernels import grouped_gemm as gg

    B, S, d, sizes, k, b, _ = CONFIGS["ref_variable"]
    g = torch.Generator().manual_seed(11)
    wide = torch.randn(B, S, d + 8, generator=g).to(torch.bfloat16).to(device)
    G = torch.randn(B, S, d, generator=g).to(torch.bfloat16).to(device)
    p = make_problem(B * S, d, sizes, k, b, seed=0, device=device)
    gg.FUSED_EXPERT_PATH = fused
    try:
        res = []
        for sliced in (True, False):
            m = _module(p, d, sizes, k, b, device)
            m.router.register_forward_pre_hook(lambda mod, args: (args[0].contiguous(),))
            src = wide.detach().clone().requires_grad_(True)
            x = src[:, :, 1:1 + d] if sliced else src[:, :, 1:1 + d].contiguous()
            if sliced:
                assert x.data_ptr() % 16 == 2
            out, aux, f_i = m(x)
            loss = (out.float() * G.float()).sum() + sum(aux.values())
            loss.backward()
            res.append([out, f_i, *aux.values(), src.grad, m.w1.grad, m.w2.grad,
                        m.router.weight.grad])
        torch.cuda.synchronize()
        for a, c in zip(*res):
            assert bits_equal(a, c)
    finally:
        gg.FUSED_EXPERT_PATH = True


def test_strided_router_logits_same_bits(device):
    """Router logits handed on as a strided view (a forward hook on the
    router returning a column slice of a wider tensor) give the bits of the
    plain logits: output, losses, f_i and the x / router gradients."""
    B, S, d, sizes, k, b, _ = CONFIGS["ref_variable"]
    E = sum(c for c, _ in sizes)
    p = make_problem(B * S, d, sizes, k, b, seed=2, device=device)
    G = torch.randn(B, S, d, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    res = []
    for strided in (True, False):
        m = _module(p, d, sizes, k, b, device)
        if strided:
            def hook(mod, inp, out):
                wide = torch.cat([out[:, :1], out, out[:, :7]], dim=1)
                return wide[:, 1:1 + E]
            m.router.register_forward_hook(hook)
        x = p["x"].view(B, S, d).to(device).requires_grad_(True)
        out, aux, f_i = m(x)
        loss = (out.float() * G.to(device).float()).sum() + sum(aux.values())
        loss.backward()
        res.append([out, f_i, *aux.values(), x.grad, m.router.weight.grad, m.w1.grad])
    torch.cuda.synchronize()
    for a, c in zip(*res):
        assert bits_equal(a, c)


@pytest.mark.parametrize("fused,dtype", [(True, torch.bfloat16), (False, torch.bfloat16),
                                         (True, torch.float32)])
def test_no_tokens(fused, dtype, device):
    """A batch with no tokens: an empty output, zero weight gradients (the
    reference's grouped-GEMM backward returns zeros for empty inputs), an
    empty input gradient."""
    from triton_moe.kernels import grouped_gemm as gg

    d, sizes, k, b = 128, [(2, 128), (2, 64)], 2, 64
    cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=b)
    m = TritonMoEMLP(cfg).to(device).to(dtype)
    gg.FUSED_EXPERT_PATH = fused
    try:
        x = torch.zeros(1, 0, d, dtype=dtype, device=device, requires_grad=True)
        out, aux, f_i = m(x)
        assert out.shape == (1, 0, d)
        out.sum().backward()
        torch.cuda.synchronize()
        assert x.grad is not None and x.grad.shape == (1, 0, d)
        assert m.w1.grad is not None and int(torch.count_nonzero(m.w1.grad)) == 0
        assert m.w2.grad is not None and int(torch.count_nonzero(m.w2.grad)) == 0
    finally:
        gg.FUSED_EXPERT_PATH = True


def test_autocast_region_same_bits(device):
    """A bf16 layer run inside torch.autocast (bf16), forward and backward,
    gives the bits it gives outside: nothing in the layer after the router
    Linear is an op autocast would change, and the Linear is already bf16."""
    B, S, d, sizes, k, b, _ = CONFIGS["ref_variable"]
    p = make_problem(B * S, d, sizes, k, b, seed=11, device=device)
    m = _module(p, d, sizes, k, b, device)
    G = torch.randn(B, S, d, generator=torch.Generator().manual_seed(12)).to(
        torch.bfloat16).to(device)
    res = []
    for ctx in (contextlib.nullcontext(), torch.autocast("cuda", dtype=torch.bfloat16)):
        x = p["x"].view(B, S, d).to(device).requires_grad_(True)
        m.zero_grad(set_to_none=True)
        with ctx:
            out, aux, f_i = m(x)
            loss = (out * G).sum() + aux["router_z_loss"] + aux["load_balance_loss"]
        loss.backward()
        res.append((out.detach().clone(), aux["router_z_loss"].detach().clone(), f_i.clone(),
                    x.grad.clone(), m.w1.grad.clone(), m.w2.grad.clone(),
                    m.router.weight.grad.clone()))
    for a, c, what in zip(res[0], res[1], ("out", "z", "f_i", "x", "w1", "w2", "router")):
        assert bits_equal(a, c), what


@pytest.mark.parametrize("name", ["cfg1", "cfg3"])
def test_backward_stream_modes(name, device):
    """The backward runs its weight-gradient GEMMs on a second stream beside
    dH and dX, or (one stream) in one launch with each of them on half of the
    CUs. x.grad is the same bits in both modes; the split-K dW GEMMs cut their
    K ranges by the launch's workgroup count, so w1 / w2 gradients differ
    between the modes in fp32 summation order only (held at the ulp level),
    and each mode gives the same bits in every one of three steps in a row
    (stream reuse, workspaces per stream)."""
    from triton_moe.kernels import grouped_gemm as gg

    m, x, _, _, _, _ = _run(name, device)
    G = torch.randn(x.shape, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    G = G.to(device)

    def grads(side):
        gg.BACKWARD_SIDE_STREAM = side
        try:
            out = []
            for _ in range(3):
                x.grad = None
                m.zero_grad(set_to_none=True)
                y, _, _ = m(x)
                y.backward(G)
                out.append((x.grad.clone(), m.w1.grad.clone(), m.w2.grad.clone()))
            torch.cuda.synchronize()
            return out
        finally:
            gg.BACKWARD_SIDE_STREAM = None

    one, two = grads(False), grads(True)
    for mode in (one, two):
        for step in mode[1:]:
            for ga, gb in zip(mode[0], step):
                assert bits_equal(ga, gb)
    for a, b in zip(one, two):
        assert bits_equal(a[0], b[0])
        for ga, gb, what in ((a[1], b[1], "w1"), (a[2], b[2], "w2")):
            st = parity_stats(ga, gb, gb.abs().float() + 1e-30)
            assert st["ulp1"] >= 0.999 and st["ulp2"] >= 0.9995, (name, what, st)


def test_forward_profiled(device):
    m, x, out, aux, f_i, _ = _run("ref_small", device)

    class StepRecorder:
        """Event-timed steps, as the reference's CUDAStepProfiler."""

        def __init__(self):
            self.steps = []

        @contextlib.contextmanager
        def step(self, name):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            try:
                yield
            finally:
                e1.record()
                self.steps.append((name, e0, e1))

    rec = StepRecorder()
    out2, aux2, f2 = m.forward_profiled(x.detach(), rec)
    torch.cuda.synchronize()
    names = [n for n, _, _ in rec.steps]
    assert names == ["flatten", "routing", "fused_route", "gather", "gemm_up", "gemm_down",
                     "scatter", "reshape", "aux_loss"]
    ms = {n: a.elapsed_time(b) for n, a, b in rec.steps}
    # each expert-path step holds a launch of its own
    for n in ("gemm_up", "gemm_down", "scatter"):
        assert ms[n] > 0.0, (n, ms)
    assert bits_equal(out2, out.detach()) and torch.equal(f2, f_i)
    assert not out2.requires_grad


def test_config4_full_size_sampled(device):
    """BASELINE config 4 at full size (d=2048, 128 variable experts, k=8,
    T=32768): outputs and x.grad are row-local, so 2048 sampled tokens are
    checked against the oracle restricted to those tokens; the weight
    gradients on the columns of 18 experts, 6 from each width group (1024,
    512, 256), with all their rows. Against the bf16w oracle: normwise
    TIGHT and the ulp-level bounds of test_forward_backward_vs_oracle;
    against the unrounded fp32 chain: normwise LOOSE."""
    B, S, d, sizes, k, b = 1, 32768, 2048, [(32, 1024), (64, 512), (32, 256)], 8, 64
    p = make_problem(B * S, d, sizes, k, b, seed=4, device=device)
    m = _module(p, d, sizes, k, b, device)
    x = p["x"].view(B, S, d).to(device).requires_grad_(True)
    out, _, _ = m(x)
    out.sum().backward()
    with torch.no_grad():
        logits, _, wts, sel = m._router(x.detach().reshape(-1, d))
    assert bits_equal(logits, p["logits"]) and torch.equal(sel, p["sel"])
    assert bits_equal(wts, p["wts"])
    g = torch.Generator().manual_seed(0)
    tok = torch.randperm(S, generator=g)[:2048].sort().values
    sub = eager.Problem(p["x"][tok].float(), p["w1"].float(), p["w2"].float(), p["widths"],
                        p["offsets"], sel.cpu()[tok], wts.cpu()[tok].float(), b)
    out_s = out.detach().reshape(S, d)[tok.to(device)]
    gx_s = x.grad.reshape(S, d)[tok.to(device)]
    ones = torch.ones(len(tok), d)
    fb = eager.forward(sub, "bf16w")
    bb = eager.backward(sub, fb, ones, "bf16w")
    mags = term_magnitudes(sub, fb, bb)
    assert_close_norm(out_s, fb["out"], TIGHT, "cfg4 out")
    assert_close_norm(gx_s, bb["grad_x"], TIGHT, "cfg4 x.grad")
    # d = 2048, k = 8 and widths up to 1024: each output element is the end
    # of longer chains of rounded sums, and 99.88 % of out lands within 1 ulp
    _assert_ulp_level(out_s, fb["out"], mags["out"], "cfg4 out", 0.998, 0.999)
    _assert_ulp_level(gx_s, bb["grad_x"], mags["grad_x"], "cfg4 x.grad", 0.998, 0.999)
    ff = eager.forward(sub, "fp32")
    assert_close_norm(out_s, ff["out"], LOOSE, "cfg4 out vs fp32 oracle")
    bf_ = eager.backward(sub, ff, ones, "fp32")
    assert_close_norm(gx_s, bf_["grad_x"], LOOSE, "cfg4 x.grad vs fp32 oracle")
    # weight gradients: the oracle on 18 experts' columns (all their tokens)
    full = eager.Problem(p["x"].float(), p["w1"].float(), p["w2"].float(), p["widths"],
                         p["offsets"], sel.cpu(), wts.cpu().float(), b)
    r = eager.route(full)
    experts = [0, 5, 11, 17, 23, 31, 32, 45, 58, 71, 84, 95, 96, 102, 108, 114, 120, 127]
    assert {p["widths"][e] for e in experts} == {1024, 512, 256}
    gw1_g, gw1_b, gw1_f, gw1_m = [], [], [], []
    gw2_g, gw2_b, gw2_f, gw2_m = [], [], [], []
    for e in experts:
        w, o = p["widths"][e], p["offsets"][e]
        r0 = int(r["padded_bins"][e - 1]) if e else 0
        r1 = int(r["padded_bins"][e])
        rs = torch.from_numpy(r["row_src"][r0:r1]).long()
        ok = rs >= 0
        xe = torch.zeros(r1 - r0, d)
        xe[ok] = p["x"][rs[ok] // k].float()
        we = torch.zeros(r1 - r0)
        we[ok] = wts.cpu().float().reshape(-1)[rs[ok]]
        z = xe @ p["w1"][:, o:o + w].float()
        # the "bf16w" order: H' = bf16(w relu(z)^2), GH = bf16(w (G @ W2^T))
        pre = eager.bf(torch.relu(z))
        h = eager.bf(we[:, None] * torch.relu(z) ** 2)
        g_rows = torch.zeros(r1 - r0, d)
        g_rows[ok] = 1.0
        gh = eager.bf(we[:, None] * (g_rows @ p["w2"][o:o + w].float().T))
        ga = eager.bf(torch.where(pre > 0, gh * 2.0 * pre, torch.zeros_like(pre)))
        gw2_g.append(m.w2.grad[o:o + w].cpu().reshape(-1))
        gw2_b.append(eager.bf(h.T @ g_rows).reshape(-1))
        gw2_m.append((h.abs().T @ g_rows).reshape(-1))
        gw1_g.append(m.w1.grad[:, o:o + w].cpu().reshape(-1))
        gw1_b.append(eager.bf(xe.T @ ga).reshape(-1))
        gw1_m.append((xe.abs().T @ ga.abs()).reshape(-1))
        # unrounded fp32 chain (the tolerance oracle)
        h32 = we[:, None] * torch.relu(z) ** 2
        gh32 = we[:, None] * (g_rows @ p["w2"][o:o + w].float().T)
        ga32 = torch.where(z > 0, gh32 * 2.0 * torch.relu(z), torch.zeros_like(z))
        gw2_f.append((h32.T @ g_rows).reshape(-1))
        gw1_f.append((xe.T @ ga32).reshape(-1))
        assert_close_norm(m.w2.grad[o:o + w], gw2_b[-1].view(w, d), TIGHT, f"cfg4 gw2 e{e}")
        assert_close_norm(m.w1.grad[:, o:o + w], gw1_b[-1].view(d, w), TIGHT, f"cfg4 gw1 e{e}")
        assert_close_norm(m.w2.grad[o:o + w], gw2_f[-1].view(w, d), LOOSE, f"cfg4 gw2 e{e} fp32")
        assert_close_norm(m.w1.grad[:, o:o + w], gw1_f[-1].view(d, w), LOOSE,
                          f"cfg4 gw1 e{e} fp32")
    _assert_ulp_level(torch.cat(gw1_g), torch.cat(gw1_b), torch.cat(gw1_m), "cfg4 gw1", 0.998,
                      0.999)
    _assert_ulp_level(torch.cat(gw2_g), torch.cat(gw2_b), torch.cat(gw2_m), "cfg4 gw2", 0.998,
                      0.999)


def _norm_err(got, ref):
    d = (got.double() - ref.double()).abs()
    return (d.max() / ref.abs().max()).item(), (d.mean() / ref.abs().mean()).item()


@pytest.mark.parametrize("name", ["ref_small", "ref_variable", "cfg1", "cfg3_a1"])
def test_routing_weight_grad(name, device):
    """TritonMoEConfig(routing_weight_grad=True) differentiates the output
    through the routing weights into the router (the reference's weights get
    no gradient, scatter.py:176). The logit gradient is held to the float64
    chain of the fp32 oracle's weight gradient (combine_weight_grad of the
    unrounded Y, then router_weight_logit_grad): its normwise error must stay
    within twice that of the same chain fed the reference's rounding order
    (Y = bf16(H W2), bf16 H), the yardstick of what bf16 storage costs here.
    W1 and W2 gradients are unchanged, bit for bit."""
    B, S, d, sizes, k, b, alpha = CONFIGS[name]
    E = sum(c for c, _ in sizes)
    bias = zipf_bias(E, alpha=alpha) if alpha is not None else None
    p = make_problem(B * S, d, sizes, k, b, seed=0, skew=bias, device=device)
    T = B * S
    G = torch.randn(T, d, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    grads = {}
    for flag in (False, True):
        cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=b,
                              routing_weight_grad=flag)
        m = TritonMoEMLP(cfg).to(device).to(torch.bfloat16)
        with torch.no_grad():
            m.router.weight.copy_(p["wr"])
            m.w1.copy_(p["w1"])
            m.w2.copy_(p["w2"])
        store = {}

        def hook(mod, inp, out):
            out = out + bias.to(out.device, out.dtype) if bias is not None else out
            if out.requires_grad:
                out.register_hook(lambda g: store.__setitem__("glogits", g))
            store["logits"] = out.detach()
            return out

        m.router.register_forward_hook(hook)
        x = p["x"].view(B, S, d).to(device).requires_grad_(True)
        out, _, _ = m(x)
        out.backward(G.to(device).view_as(out))
        grads[flag] = (x.grad, m.w1.grad, m.w2.grad, m.router.weight.grad, store)
    for a, b_ in zip(grads[False][1:3], grads[True][1:3]):
        assert bits_equal(a, b_)
    assert grads[False][3] is None and grads[True][3] is not None
    store = grads[True][4]
    # x also reaches the loss through the router Linear now: x.grad gains
    # dlogits @ Wr (the two bf16 contributions summed by autograd)
    xr = store["glogits"].float() @ p["wr"].to(device).float()
    assert_close_norm(grads[True][0].reshape(T, d).float(),
                      grads[False][0].reshape(T, d).float() + xr, TIGHT, f"{name} x.grad")
    assert bits_equal(store["logits"], p["logits"])
    prob = eager.Problem(p["x"].float(), p["w1"].float(), p["w2"].float(), p["widths"],
                         p["offsets"], p["sel"].cpu(), p["wts"].cpu().float(), b)
    ff = eager.forward(prob, "fp32")
    f16 = eager.forward(prob, "bf16")
    ar = ff["route"]["assignment_row"]
    Gf = G.float()
    L = p["logits"].float().cpu()
    ref = eager.router_weight_logit_grad(
        L, prob.selected, eager.combine_weight_grad(Gf, ff["y"], ar, k, T).view(T, k))
    yard = eager.router_weight_logit_grad(
        L, prob.selected, eager.combine_weight_grad(Gf, f16["y"], ar, k, T).view(T, k))
    got = store["glogits"].float().cpu()
    e_got, e_yard = _norm_err(got, ref), _norm_err(yard, ref)
    # + 4e-3: the two bf16 roundings the yardstick leaves out (the bf16
    # weight gradient autograd hands the router, and the bf16 logit gradient)
    assert e_got[0] <= 2 * e_yard[0] + 4e-3 and e_got[1] <= 2 * e_yard[1] + 4e-3, (e_got, e_yard)
    # the router weight's gradient is the linear layer's backward of it
    wr_ref = store["glogits"].float().t() @ p["x"].to(device).float()
    assert_close_norm(grads[True][3], wr_ref, TIGHT, f"{name} router weight grad")


@pytest.mark.parametrize("name", ["ref_small", "ref_variable", "cfg2"])
def test_routing_weight_grad_at_zero_and_denormal_weights(name, device):
    """The routing-weight gradient where the bf16 weight is 0 or a denormal:
    the module forms dL/dw from the dH GEMM's row sums of w * (G W2^T) *
    relu(z)^2 divided by w, which cannot recover these, so they take the
    direct form sum_c (G[t] . W2[c]) relu(z)[c]^2. Checked entry by entry
    against the fp32 oracle's G[t] . Y[row] (Y = relu(x W1_e)^2 W2_e
    unweighted), which does not depend on w; the forward output is checked
    too (a zero weight removes that slot's contribution)."""
    B, S, d, sizes, k, b, _alpha = CONFIGS[name]
    T = B * S
    p = make_problem(T, d, sizes, k, b, seed=3, device=device)
    wts = p["wts"].cpu().clone().reshape(-1)
    A = wts.numel()
    zero = torch.zeros(A, dtype=torch.bool)
    zero[::7] = True
    den = torch.zeros(A, dtype=torch.bool)
    den[3::11] = True
    den &= ~zero
    wts[zero] = 0
    # bf16 denormals (below 2^-126): 2^-130 and 2^-133
    wts[den] = torch.tensor([2.0 ** -130, 2.0 ** -133], dtype=torch.bfloat16).repeat(
        int(den.sum()) // 2 + 1)[:int(den.sum())]
    assert (wts[den].float() < 2.0 ** -126).all() and (wts[den] != 0).all()
    m = _module(p, d, sizes, k, b, device)
    x_flat = p["x"].to(device)
    w = wts.to(device).requires_grad_(True)
    sel = p["sel"].reshape(-1).to(device)
    out, _tpe = m._experts(x_flat, w, sel)
    G = torch.randn(T, d, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    out.backward(G.to(device))
    got = w.grad.float().cpu()
    prob = eager.Problem(p["x"].float(), p["w1"].float(), p["w2"].float(), p["widths"],
                         p["offsets"], p["sel"].cpu(), wts.view(T, k).float(), b)
    ff = eager.forward(prob, "fp32")
    ar = ff["route"]["assignment_row"]
    ref = eager.combine_weight_grad(G.float(), ff["y"], ar, k, T)
    assert_close_norm(out.float(), ff["out"], LOOSE, f"{name} out")
    scale = ref.abs().max().item()
    tiny = zero | den
    err = (got - ref).abs()
    # every entry: within 3 % of itself plus 1 % of the largest entry (bf16
    # PRE and bf16 GH against the unrounded chain; a lost gradient fails)
    bad = err > 3e-2 * ref.abs() + 1e-2 * scale
    assert not bad.any(), (name, int(bad.sum()), err[bad][:8], ref[bad][:8])
    assert_close_norm(got, ref, LOOSE, f"{name} all entries")
    # the tiny-weight entries are real gradients, not zeros, and equal the
    # direct form on the module's own bf16 PRE (float64 here) up to fp32 sums
    assert (got[tiny] != 0).float().mean() > 0.99
    pre = eager.forward(prob, "bf16", ff["route"])["pre_act"].double()
    G64, W2 = G.double(), p["w2"].double()
    ar_t = torch.as_tensor(ar, dtype=torch.int64)
    rows_ = ar_t[tiny]
    toks = torch.nonzero(tiny).reshape(-1) // k
    ends = torch.as_tensor(np.asarray(ff["route"]["padded_bins"], np.int64))
    exp_of = torch.searchsorted(ends, rows_, right=True)  # rows [ends[e-1], ends[e]) are e's
    ref_b = torch.zeros(int(tiny.sum()), dtype=torch.float64)
    mag = torch.zeros_like(ref_b)  # sum of the terms' magnitudes
    for e, (w_, o) in enumerate(zip(p["widths"], p["offsets"])):
        sel_e = exp_of == e
        if sel_e.any():
            terms = (G64[toks[sel_e]] @ W2[o:o + w_].T) * pre[rows_[sel_e], :w_] ** 2
            ref_b[sel_e] = terms.sum(1)
            mag[sel_e] = terms.abs().sum(1)
    # the entries are bf16: 99.9 % within one unit in the last place of the
    # rounded float64 value; the rest (sums that cancel) within 1e-4 of their
    # terms' magnitude (fp32 sums, and PRE bits that may differ by one ulp)
    ulps = bf16_ulps(w.grad[tiny.to(device)], ref_b.to(torch.bfloat16))
    assert float((ulps <= 1).double().mean()) >= 0.999, (name, int(ulps.max()))
    err_b = (got[tiny].double() - ref_b).abs()
    assert (err_b <= 2.0 ** -8 * ref_b.abs() + 1e-4 * mag).all(), (name, int(ulps.max()))


@pytest.mark.parametrize("name,grad", [("ref_variable", "random"), ("cfg1", "sum"),
                                       ("cfg2", "scaled"), ("cfg3_a1", "random"),
                                       ("e128", "random"), ("odd_k3", "random")])
def test_fused_expert_path_same_bits_as_per_kernel_path(name, grad, device):
    """The module after its router Linear as one library call per direction
    (vmoe_moe_forward / _backward, the default) gives the bits of the
    per-kernel calls (router_topk, RoutedMoEOp, RouterAuxOp,
    RouterWeightOp): output, auxiliary losses, f_i, the x / w1 / w2 / router
    gradients with the opt-in routing-weight gradient, over three steps (the
    output's loss, plus the auxiliary losses, the auxiliary losses alone),
    with and without the backward's second stream. Without it the fused path
    pairs each weight-gradient GEMM with dH / dX in one launch on half of
    the CUs, which cuts the split-K ranges of dW differently: w1 / w2
    gradients are then held at the ulp level."""
    from triton_moe.kernels import grouped_gemm as gg

    B, S, d, sizes, k, b, alpha = CONFIGS[name]
    E = sum(c for c, _ in sizes)
    bias = zipf_bias(E, alpha=alpha) if alpha is not None else None
    p = make_problem(B * S, d, sizes, k, b, seed=5, skew=bias, device=device)
    G = torch.randn(B, S, d, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    results = {}
    for fused in (False, True):
        for side in (False, True):
            gg.FUSED_EXPERT_PATH, gg.BACKWARD_SIDE_STREAM = fused, side
            try:
                cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k,
                                      block_size=b, routing_weight_grad=True)
                m = TritonMoEMLP(cfg).to(device).to(torch.bfloat16)
                with torch.no_grad():
                    m.router.weight.copy_(p["wr"])
                    m.w1.copy_(p["w1"])
                    m.w2.copy_(p["w2"])
                if bias is not None:
                    m.router.register_forward_hook(
                        lambda mod, inp, out: out + bias.to(out.device, out.dtype))
                x = p["x"].view(B, S, d).to(device).requires_grad_(True)
                steps = []
                for step in range(3):
                    x.grad = None
                    m.zero_grad(set_to_none=True)
                    out, aux, f_i = m(x)
                    if grad == "random":
                        loss = (out * G.to(device)).sum()
                    elif grad == "sum":
                        loss = out.sum()
                    else:
                        loss = out.sum() * 0.75
                    if step == 1:  # the auxiliary losses too
                        loss = loss + aux["router_z_loss"] * 0.1 + \
                            aux["load_balance_loss"] * 0.01 + aux["compute_loss"] * 0.01
                    if step == 2:  # the auxiliary losses alone
                        loss = aux["router_z_loss"] + aux["load_balance_loss"]
                    loss.backward()
                    grads = [t.grad.clone() if t.grad is not None else None
                             for t in (x, m.w1, m.w2, m.router.weight)]
                    steps.append((out.detach().clone(), f_i.clone(),
                                  aux["router_z_loss"].detach().clone(),
                                  aux["load_balance_loss"].detach().clone(),
                                  aux["compute_loss"].detach().clone(), *grads))
                torch.cuda.synchronize()
                results[(fused, side)] = steps
            finally:
                gg.FUSED_EXPERT_PATH, gg.BACKWARD_SIDE_STREAM = True, None
    ref = results[(False, False)]
    for key, steps in results.items():
        for i, (s_ref, s_got) in enumerate(zip(ref, steps)):
            for j, (a, b_) in enumerate(zip(s_ref, s_got)):
                if a is None or b_ is None:
                    assert a is None and b_ is None, (name, key, i, j)
                    continue
                if key == (True, False) and j in (6, 7):  # paired dW: w1 / w2 gradients
                    st = parity_stats(b_, a, a.abs().float() + 1e-30)
                    assert st["ulp1"] >= 0.999 and st["ulp2"] >= 0.9995, (name, key, i, j, st)
                    continue
                assert bits_equal(a, b_), (name, key, i, j)


@pytest.mark.parametrize("name", ["ref_variable", "cfg2", "cfg4_small"])
def test_compact_intermediates(name, device):
    """TritonMoEConfig(compact_intermediates=True): H', PRE and GA per width
    group, sum_e rows_e w_e elements. The row-tiled GEMMs compute every tile
    as the padded layout does, so out and x.grad are the same bits; the dW
    GEMMs cut their K ranges per launch, so w1 / w2 gradients may differ in
    fp32 summation order (held to the padded run at the ulp level, and to
    the bf16w oracle normwise). The saved intermediates shrink to the
    compact size."""
    from triton_moe.kernels import grouped_gemm as gg

    shapes = dict(CONFIGS, cfg4_small=(1, 4096, 512, [(4, 1024), (8, 512), (4, 256)], 8, 64,
                                        None))
    B, S, d, sizes, k, b, _alpha = shapes[name]
    T = B * S
    p = make_problem(T, d, sizes, k, b, seed=2, device=device)
    G = torch.randn(B, S, d, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    res, saved_elems = {}, {}
    orig = gg.CompactRoutedMoEOp.forward

    def spy(ctx, *a):
        out = orig(ctx, *a)
        hs = ctx.to_save[6:]  # the tensors forward passed to save_for_backward: H', PRE
        saved_elems["compact"] = sum(t.numel() for t in hs)
        return out

    for compact in (False, True):
        cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=b,
                              compact_intermediates=compact)
        m = TritonMoEMLP(cfg).to(device).to(torch.bfloat16)
        with torch.no_grad():
            m.router.weight.copy_(p["wr"])
            m.w1.copy_(p["w1"])
            m.w2.copy_(p["w2"])
        x = p["x"].view(B, S, d).to(device).requires_grad_(True)
        gg.CompactRoutedMoEOp.forward = staticmethod(spy)
        try:
            out, aux, f_i = m(x)
        finally:
            gg.CompactRoutedMoEOp.forward = staticmethod(orig)
        out.backward(G.to(device))
        res[compact] = (out.detach(), x.grad, m.w1.grad, m.w2.grad, f_i,
                        aux["load_balance_loss"].detach())
    a, c = res[False], res[True]
    assert bits_equal(a[0], c[0]) and bits_equal(a[1], c[1])
    assert bits_equal(a[4], c[4]) and bits_equal(a[5], c[5])
    for ga, gc, what in ((a[2], c[2], "w1"), (a[3], c[3], "w2")):
        st = parity_stats(gc, ga, ga.abs().float() + 1e-30)
        assert st["ulp1"] >= 0.999 and st["ulp2"] >= 0.9995, (name, what, st)
    prob = eager.Problem(p["x"].float(), p["w1"].float(), p["w2"].float(), p["widths"],
                         p["offsets"], p["sel"].cpu(), p["wts"].cpu().float(), b)
    fb = eager.forward(prob, "bf16w")
    bb = eager.backward(prob, fb, G.reshape(T, d).float(), "bf16w")
    assert_close_norm(c[2], bb["grad_w1"], TIGHT, f"{name} compact grad_w1")
    assert_close_norm(c[3], bb["grad_w2"], TIGHT, f"{name} compact grad_w2")
    # H' and PRE: 2 x sum over groups of rows_g x w_g, against 2 x rows x max_width padded
    r = fb["route"]
    pb = [0] + [int(v) for v in r["padded_bins"]]
    widths = p["widths"]
    compact_elems = 2 * sum((pb[e + 1] - pb[e]) * widths[e] for e in range(len(widths)))
    assert saved_elems["compact"] == compact_elems
    assert compact_elems < 2 * pb[-1] * max(widths)


@pytest.mark.parametrize("mode", ["no_grad", "inference_mode"])
def test_forward_without_autograd_same_bits(mode, device):
    """Under torch.no_grad() and torch.inference_mode() the module's forward
    (one library call after the router Linear) gives the bits of the
    forward that records the graph, and nothing requires grad."""
    B, S, d, sizes, k, b, _alpha = CONFIGS["cfg2"]
    p = make_problem(B * S, d, sizes, k, b, seed=6, device=device)
    m = _module(p, d, sizes, k, b, device)
    x = p["x"].view(B, S, d).to(device)
    out_g, aux_g, f_g = m(x.clone().requires_grad_(True))
    ctx = torch.no_grad() if mode == "no_grad" else torch.inference_mode()
    with ctx:
        out, aux, f_i = m(x)
    assert not out.requires_grad and not aux["router_z_loss"].requires_grad
    assert bits_equal(out, out_g.detach()) and bits_equal(f_i, f_g)
    for key in aux:
        assert bits_equal(aux[key], aux_g[key].detach()), key
