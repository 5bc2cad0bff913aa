"""fp32 grouped GEMMs (csrc/gemm_f32.hip) through the public API, against a
float64 per-expert restatement and its torch autograd gradients.

The reference's grouped-GEMM kernels are dtype-generic and its own autograd
tests run fp32 (tests/test_grouped_gemm_backward.py:151-208, forward against
autograd at rtol = atol = 1e-3). Here fp32 products are held to float64 at
F32 below: fp32 accumulation over k <= 1024 terms leaves ~1e-6 relative error,
so a dropped term, a wrong operand or a transposed index fails by orders of
magnitude. Gradients come from float64 autograd of the forward restatement,
not from a restated backward.
"""

from __future__ import annotations

import pytest
import torch

from triton_moe.kernels import (
    grouped_gemm_down,
    grouped_gemm_down_autograd,
    grouped_gemm_down_backward,
    grouped_gemm_up,
    grouped_gemm_up_autograd,
    grouped_gemm_up_backward,
)

from _util import assert_close_norm

pytestmark = pytest.mark.gpu

# normwise (max|d| / max|ref|, mean|d| / mean|ref|) against float64
F32 = (1e-4, 1e-5)

# (rows per expert, widths, hidden, rows covered = tpe < rows where marked)
CASES = {
    "ref_fixture": ([128, 128], [128, 128], 64, False),      # reference test shapes
    "ragged": ([70, 0, 133, 64, 1], [64, 128, 32, 96, 8], 96, False),
    "uncovered": ([100, 64, 37], [48, 64, 16], 128, True),  # tpe < row range
    "wide": ([300, 257], [256, 512], 256, False),
    # hidden, widths and offsets off the bf16 kernels' multiple-of-8 rule
    "unaligned": ([50, 33, 0, 17], [12, 20, 36, 5], 100, False),
}


def _meta(rows, widths, tpe_short, mult=1):
    eto = [0]
    for r in rows:
        eto.append(eto[-1] + r)
    tpe = [max(0, r - (r // 3 if tpe_short else 0)) for r in rows]
    offs = [0]
    for w in widths:
        offs.append(offs[-1] + mult * w)
    return eto, tpe, offs


def _dev(v, device):
    return torch.tensor(v, dtype=torch.int32, device=device)


def _ref_chain(xg, w1, w2, eto, tpe, widths, offs1, offs2, act):
    """float64 H = act(x_e W1_e) and Y = H_e W2_e per expert (rows
    eto[e] + [0, min(tpe, eto[e+1] - eto[e])), zero elsewhere)."""
    P, d = xg.shape
    max_w = max(widths)
    h = torch.zeros(P, max_w, dtype=torch.float64)
    pre = torch.zeros(P, max_w, dtype=torch.float64)
    y = torch.zeros(P, d, dtype=torch.float64)
    for e, w in enumerate(widths):
        r0 = eto[e]
        r1 = r0 + max(0, min(tpe[e], eto[e + 1] - eto[e]))
        if r1 == r0 or w == 0:
            continue
        o = offs1[e]
        z = xg[r0:r1] @ w1[:, o:o + w]
        if act == "swiglu":
            u = xg[r0:r1] @ w1[:, o + w:o + 2 * w]
            he, pe = z * torch.sigmoid(z) * u, z
        elif act == "relu_squared":
            he, pe = torch.relu(z) ** 2, torch.relu(z)
        else:
            he, pe = z, torch.zeros_like(z)
        h[r0:r1, :w] = he
        pre[r0:r1, :w] = pe
        y[r0:r1] = he @ w2[offs2[e]:offs2[e] + w]
    return h, pre, y


def _inputs(rows, widths, d, act, seed):
    g = torch.Generator().manual_seed(seed)
    P = sum(rows)
    m1 = 2 if act == "swiglu" else 1
    xg = torch.randn(P, d, generator=g, dtype=torch.float64)
    w1 = torch.randn(d, m1 * sum(widths), generator=g, dtype=torch.float64) * 0.1
    w2 = torch.randn(sum(widths), d, generator=g, dtype=torch.float64) * 0.1
    return xg, w1, w2


@pytest.mark.parametrize("act", ["none", "relu_squared", "swiglu"])
@pytest.mark.parametrize("name", list(CASES))
def test_f32_forward(name, act, device):
    rows, widths, d, short = CASES[name]
    m1 = 2 if act == "swiglu" else 1
    eto, tpe, offs1 = _meta(rows, widths, short, m1)
    _, _, offs2 = _meta(rows, widths, short)
    xg, w1, w2 = _inputs(rows, widths, d, act, seed=len(rows) + d)
    h_ref, pre_ref, y_ref = _ref_chain(xg, w1, w2, eto, tpe, widths, offs1, offs2, act)
    args = (_dev(eto, device), _dev(offs1, device), _dev(widths, device), _dev(tpe, device))
    h, pre = grouped_gemm_up(xg.float().to(device), w1.float().to(device), *args, max(widths),
                             activation=act, save_pre_act=True)
    assert h.dtype == torch.float32 and pre.dtype == torch.float32
    assert_close_norm(h, h_ref, F32, f"{name} {act} H")
    assert_close_norm(pre, pre_ref, F32, f"{name} {act} pre_act")
    y = grouped_gemm_down(h_ref.float().to(device), w2.float().to(device), args[0],
                          _dev(offs2, device), args[2], args[3], d)
    assert_close_norm(y, y_ref, F32, f"{name} down Y")
    # rows outside every expert's covered range and columns past w_e stay 0
    cover = torch.zeros(sum(rows), dtype=torch.bool)
    for e, w in enumerate(widths):
        n = max(0, min(tpe[e], eto[e + 1] - eto[e]))
        cover[eto[e]:eto[e] + n] = True
        assert h[eto[e]:eto[e + 1], w:].abs().sum().item() == 0
    assert h.cpu()[~cover].abs().sum().item() == 0
    assert y.cpu()[~cover].abs().sum().item() == 0


@pytest.mark.parametrize("use_map", [False, True])
@pytest.mark.parametrize("act", ["none", "relu_squared", "swiglu"])
@pytest.mark.parametrize("name", ["ref_fixture", "ragged", "uncovered", "unaligned"])
def test_f32_autograd_chain(name, act, use_map, device):
    """up_autograd -> down_autograd -> (Y * G).sum() -> backward (the
    reference's test_grouped_gemm_backward flow in fp32; with x_flat and
    gather_map as the reference module calls it, moe.py:214-225)."""
    rows, widths, d, short = CASES[name]
    m1 = 2 if act == "swiglu" else 1
    eto, tpe, offs1 = _meta(rows, widths, short, m1)
    _, _, offs2 = _meta(rows, widths, short)
    xg, w1, w2 = _inputs(rows, widths, d, act, seed=7 + len(rows))
    P = xg.shape[0]
    gen = torch.Generator().manual_seed(11)
    G = torch.randn(P, d, generator=gen, dtype=torch.float64)
    kw = {}
    if use_map:
        # token rows read through a gather map: xg = x_flat[gm]
        T = max(P // 2, 1)
        x_flat = torch.randn(T, d, generator=gen, dtype=torch.float64)
        gm = torch.randint(0, T, (P,), generator=gen, dtype=torch.int32)
        xg = x_flat[gm.long()]
        kw = dict(x_flat=x_flat.float().to(device), gather_map=gm.to(device))
    x64 = xg.clone().requires_grad_(True)
    w164 = w1.clone().requires_grad_(True)
    w264 = w2.clone().requires_grad_(True)
    _, _, y_ref = _ref_chain(x64, w164, w264, eto, tpe, widths, offs1, offs2, act)
    (y_ref * G).sum().backward()

    args = (_dev(eto, device), _dev(offs1, device), _dev(widths, device), _dev(tpe, device))
    x = xg.float().to(device).requires_grad_(True)
    w1d = w1.float().to(device).requires_grad_(True)
    w2d = w2.float().to(device).requires_grad_(True)
    h = grouped_gemm_up_autograd(x, w1d, *args, max(widths), d, act, **kw)
    y = grouped_gemm_down_autograd(h, w2d, args[0], _dev(offs2, device), args[2], args[3], d,
                                   max(widths))
    (y * G.float().to(device)).sum().backward()
    assert_close_norm(y, y_ref.detach(), F32, f"{name} {act} Y")
    assert_close_norm(x.grad, x64.grad, F32, f"{name} {act} grad_x")
    assert_close_norm(w1d.grad, w164.grad, F32, f"{name} {act} grad_w1")
    assert_close_norm(w2d.grad, w264.grad, F32, f"{name} {act} grad_w2")


@pytest.mark.parametrize("act", ["relu_squared", "swiglu"])
def test_f32_backward_functions_match_autograd(act, device):
    """grouped_gemm_up_backward / grouped_gemm_down_backward give the autograd
    functions' gradients bit for bit (same kernels, same inputs)."""
    rows, widths, d, short = CASES["ragged"]
    m1 = 2 if act == "swiglu" else 1
    eto, tpe, offs1 = _meta(rows, widths, short, m1)
    _, _, offs2 = _meta(rows, widths, short)
    xg, w1, w2 = _inputs(rows, widths, d, act, seed=5)
    args = (_dev(eto, device), _dev(offs1, device), _dev(widths, device), _dev(tpe, device))
    e2 = _dev(offs2, device)
    x = xg.float().to(device).requires_grad_(True)
    w1d = w1.float().to(device).requires_grad_(True)
    w2d = w2.float().to(device).requires_grad_(True)
    h = grouped_gemm_up_autograd(x, w1d, *args, max(widths), d, act)
    y = grouped_gemm_down_autograd(h, w2d, args[0], e2, args[2], args[3], d, max(widths))
    G = torch.randn(y.shape, generator=torch.Generator().manual_seed(3)).to(device)
    y.backward(G)
    h2, pre = grouped_gemm_up(x.detach(), w1d.detach(), *args, max(widths), activation=act,
                              save_pre_act=True)
    assert torch.equal(h2, h.detach())
    gh, gw2 = grouped_gemm_down_backward(G, h2, w2d.detach(), args[0], e2, args[2], args[3], d,
                                         max(widths))
    gx, gw1 = grouped_gemm_up_backward(gh, x.detach(), w1d.detach(), pre, *args, d,
                                       activation=act)
    assert torch.equal(gw2, w2d.grad)
    assert torch.equal(gx, x.grad)
    assert torch.equal(gw1, w1d.grad)


def test_f32_reference_fixture_forward_vs_autograd(device):
    """The reference's fp32 check (tests/test_grouped_gemm_backward.py:140-175):
    grouped_gemm_up against grouped_gemm_up_autograd, 256 tokens, hidden 64,
    two experts of width 128; here they are the same kernel, so equal."""
    torch.manual_seed(42)
    eto = torch.tensor([0, 128, 256], dtype=torch.int32, device=device)
    wid = torch.tensor([128, 128], dtype=torch.int32, device=device)
    x = torch.randn(256, 64, device=device, dtype=torch.float32)
    w1 = torch.randn(64, 256, device=device, dtype=torch.float32)
    fused = grouped_gemm_up(x, w1, eto, eto, wid, wid, 128, activation="relu_squared")
    auto = grouped_gemm_up_autograd(x.clone().requires_grad_(True), w1.clone().requires_grad_(True),
                                    eto, eto, wid, wid, 128, 64, "relu_squared")
    torch.testing.assert_close(fused, auto, rtol=1e-3, atol=1e-3)
    assert torch.equal(fused, auto.detach())


def test_f32_bf16_activations_widened(device):
    """bf16 x with fp32 weights is widened to fp32, as the reference's
    autograd casts x to the weights' dtype (grouped_gemm.py:1427)."""
    eto = torch.tensor([0, 64, 128], dtype=torch.int32, device=device)
    wid = torch.tensor([64, 64], dtype=torch.int32, device=device)
    g = torch.Generator().manual_seed(9)
    xb = torch.randn(128, 32, generator=g).to(torch.bfloat16)
    w1 = torch.randn(32, 128, generator=g)
    a = grouped_gemm_up(xb.to(device), w1.to(device), eto, eto, wid, wid, 64)
    b = grouped_gemm_up(xb.float().to(device), w1.to(device), eto, eto, wid, wid, 64)
    assert torch.equal(a, b)


def test_f32_empty_routing(device):
    """No rows at all (every expert empty): zero-row outputs, zero weight
    gradients, nothing launched."""
    E, d, w = 3, 32, 16
    eto = torch.zeros(E + 1, dtype=torch.int32, device=device)
    ewo = torch.arange(0, E * w + 1, w, dtype=torch.int32, device=device)
    wid = torch.full((E,), w, dtype=torch.int32, device=device)
    tpe = torch.zeros(E, dtype=torch.int32, device=device)
    x = torch.randn(0, d, device=device, requires_grad=True)
    w1 = torch.randn(d, E * w, device=device, requires_grad=True)
    w2 = torch.randn(E * w, d, device=device, requires_grad=True)
    h = grouped_gemm_up_autograd(x, w1, eto, ewo, wid, tpe, w, d, "relu_squared")
    y = grouped_gemm_down_autograd(h, w2, eto, ewo, wid, tpe, d, w)
    assert h.shape == (0, w) and y.shape == (0, d)
    y.sum().backward()
    assert w1.grad.abs().sum().item() == 0 and w2.grad.abs().sum().item() == 0
    assert x.grad.shape == (0, d)


@pytest.mark.parametrize("act", ["relu_squared", "swiglu"])
def test_f32_gather_map_pad_rows_read_zeros(act, device):
    """Map entries of -1 (the module's pad rows) read zero token rows in the
    up forward and contribute nothing to grad_w1: same results as a gathered
    x with zero rows there."""
    rows, widths, d, _ = CASES["ragged"]
    m1 = 2 if act == "swiglu" else 1
    eto, tpe, offs1 = _meta(rows, widths, False, m1)
    P = sum(rows)
    gen = torch.Generator().manual_seed(17)
    T = 40
    x_flat = torch.randn(T, d, generator=gen)
    gm = torch.randint(0, T, (P,), generator=gen, dtype=torch.int32)
    gm[::5] = -1
    xg = torch.where((gm >= 0)[:, None], x_flat[gm.clamp(min=0).long()], torch.zeros(()))
    w1 = torch.randn(d, m1 * sum(widths), generator=gen) * 0.1
    args = (_dev(eto, device), _dev(offs1, device), _dev(widths, device), _dev(tpe, device))
    xf, xgd, w1d, gmd = x_flat.to(device), xg.to(device), w1.to(device), gm.to(device)
    h_map, pre_map = grouped_gemm_up(xf, w1d, *args, max(widths), activation=act,
                                     save_pre_act=True, gather_map=gmd)
    h_ref, pre_ref = grouped_gemm_up(xgd, w1d, *args, max(widths), activation=act,
                                     save_pre_act=True)
    assert torch.equal(h_map, h_ref) and torch.equal(pre_map, pre_ref)
    gh = torch.randn(h_ref.shape, generator=gen).to(device)
    _, gw_map = grouped_gemm_up_backward(gh, xf, w1d, pre_ref, *args, d, activation=act,
                                         gather_map=gmd)
    _, gw_ref = grouped_gemm_up_backward(gh, xgd, w1d, pre_ref, *args, d, activation=act)
    assert torch.equal(gw_map, gw_ref)


def test_f32_in_kernel_relu2_rule_matches_formed_ga(device):
    """vmoe_gemm_f32_up_bwd_dx / _dw with VMOE_ACT_RELU_SQUARED (the relu^2
    gradient formed while the operand is loaded) against the path the Python
    layer takes (vmoe_f32_relu2_grad, then VMOE_ACT_NONE): the same products,
    so the same bits. vmoe_f32_relu2_grad itself on strided rows (ld > cols)
    against its formula."""
    from triton_moe import _lib

    rows, widths, d, short = CASES["ragged"]
    eto, tpe, offs = _meta(rows, widths, short)
    P, W, mw = sum(rows), sum(widths), max(widths)
    g = torch.Generator().manual_seed(21)
    x = torch.randn(P, d, generator=g).to(device)
    w1 = (torch.randn(d, W, generator=g) * 0.1).to(device)
    gbuf = torch.randn(P, mw + 24, generator=g).to(device)
    pbuf = torch.relu(torch.randn(P, mw + 24, generator=g)).to(device)
    gh, pre = gbuf[:, :mw], pbuf[:, :mw]  # strided views, ld = mw + 24
    keep = [_dev(eto, device), _dev(offs, device), _dev(widths, device), _dev(tpe, device)]
    meta = tuple(t.data_ptr() for t in keep)
    st = _lib.stream(device)
    gabuf = torch.full((P, mw + 8), float("nan"), device=device)
    ga = gabuf[:, :mw]
    _lib.call("vmoe_f32_relu2_grad", gh.data_ptr(), pre.data_ptr(), gh.stride(0), ga.data_ptr(),
              ga.stride(0), P, mw, st)
    ref = torch.where(pre > 0, gh * 2.0 * pre, torch.zeros_like(pre))
    assert torch.equal(ga, ref)
    assert torch.isnan(gabuf[:, mw:]).all()  # the row padding is not written

    def run(op, act):
        gx = torch.zeros(P, d, device=device)
        gw = torch.zeros(d, W, device=device)
        p_ = pre.data_ptr() if act else None
        _lib.call("vmoe_gemm_f32_up_bwd_dx", op.data_ptr(), p_, None, op.stride(0), act,
                  w1.data_ptr(), w1.stride(0), gx.data_ptr(), gx.stride(0), *meta, len(widths),
                  d, mw, P, st)
        _lib.call("vmoe_gemm_f32_up_bwd_dw", x.data_ptr(), x.stride(0), P, None, op.data_ptr(),
                  p_, None, op.stride(0), act, gw.data_ptr(), gw.stride(0), *meta, len(widths),
                  d, mw, P, st)
        return gx, gw

    gx_a, gw_a = run(ga, _lib.ACT_NONE)
    gx_b, gw_b = run(gh, _lib.ACT_RELU_SQUARED)
    assert torch.equal(gx_a, gx_b) and torch.equal(gw_a, gw_b)
    assert gx_a.abs().sum() > 0 and gw_a.abs().sum() > 0
