"""Grouped GEMMs on the GPU against per-expert fp32 references of the same op
(reference kernels: triton_moe/kernels/grouped_gemm.py:212-1162).

References round to bf16 exactly where the reference kernels store bf16, so
the only difference left is fp32 summation order (tolerance TIGHT, normwise).
Tail columns and uncovered rows must be exactly zero, as the reference's
torch.zeros outputs are.
"""

from __future__ import annotations

import pytest
import torch

from oracle import route as oroute
from oracle.eager import bf, expert_layout
from triton_moe.kernels import (
    grouped_gemm_down,
    grouped_gemm_down_autograd,
    grouped_gemm_down_backward,
    grouped_gemm_up,
    grouped_gemm_up_autograd,
    grouped_gemm_up_backward,
)

from _util import LOOSE, TIGHT, assert_close_norm, bits_equal, expert_rows

pytestmark = pytest.mark.gpu

# (tokens, hidden, expert sizes, top_k, block, skew)
CASES = [
    (128, 128, [(4, 256)], 2, 128, False),            # reference "small" fixture
    (1024, 256, [(8, 512)], 2, 128, False),           # reference "uniform"
    (1024, 256, [(4, 512), (4, 256)], 2, 128, False),  # reference "variable"
    (256, 64, [(2, 64), (2, 128)], 2, 64, False),      # tiles wider than the problem
    (2048, 768, [(4, 512), (8, 256), (4, 128)], 2, 64, False),  # config-2 widths
    (2048, 1024, [(64, 256)], 8, 64, True),            # config-3 shape, skewed, empties
    (1024, 2048, [(2, 1024), (2, 512)], 2, 64, False),  # d x max width >= 2^21: dW lanes of 8
    # hidden and widths multiples of 8 only: every K loop ends in a partial
    # stage (K = 200 or a width of 40 / 24 / 8), top_k 1
    (300, 200, [(3, 40), (2, 24), (1, 8)], 1, 64, False),
]
IDS = ["small", "uniform", "variable", "tiny_tiles", "var3", "skew64", "wide_lanes8", "mult8"]


def _case(T, d, sizes, k, b, skew, seed=0):
    g = torch.Generator().manual_seed(seed)
    widths, offsets = expert_layout(sizes)
    E, W, max_w = len(widths), offsets[-1], max(widths)
    logits = torch.randn(T, E, generator=g)
    if skew:
        logits[:, : E // 8] += 4.0   # hot experts
        logits[:, E - 4:] -= 50.0    # experts that receive nothing
    sel = torch.topk(logits, k, dim=-1).indices
    r = oroute.route(sel.reshape(-1).numpy(), E, b, "up")
    pb = torch.from_numpy(r["padded_bins"]).int()
    eto = torch.cat([torch.zeros(1, dtype=torch.int32), pb])
    tpe = torch.diff(eto)
    P = int(eto[-1])
    xg = torch.randn(P, d, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(d, W, generator=g) * 0.05).to(torch.bfloat16)
    w2 = (torch.randn(W, d, generator=g) * 0.05).to(torch.bfloat16)
    return dict(widths=widths, offsets=offsets, E=E, W=W, max_w=max_w, d=d, P=P, eto=eto,
                tpe=tpe, ewo=torch.tensor(offsets, dtype=torch.int32),
                wid=torch.tensor(widths, dtype=torch.int32), xg=xg, w1=w1, w2=w2,
                rows=expert_rows(r["padded_bins"]), route=r, k=k, T=T)


def _meta_dev(c, device):
    return [c[n].to(device) for n in ("eto", "ewo", "wid", "tpe")]


def _ref_up(c, xg):
    P, max_w = c["P"], c["max_w"]
    pre = torch.zeros(P, max_w)
    h = torch.zeros(P, max_w)
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], c["offsets"][e]
        z = xg[r0:r1].float() @ c["w1"][:, o:o + w].float()
        pre[r0:r1, :w] = bf(torch.relu(z))
        h[r0:r1, :w] = bf(torch.relu(z) ** 2)
    return h, pre


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_up_down_forward(case, device):
    c = _case(*case)
    eto, ewo, wid, tpe = _meta_dev(c, device)
    out, pre = grouped_gemm_up(c["xg"].to(device), c["w1"].to(device), eto, ewo, wid, tpe,
                               c["max_w"], activation="relu_squared", save_pre_act=True)
    h_ref, pre_ref = _ref_up(c, c["xg"])
    assert out.shape == (c["P"], c["max_w"]) and out.dtype == torch.bfloat16
    assert_close_norm(out, h_ref, TIGHT, "H")
    assert_close_norm(pre, pre_ref, TIGHT, "PRE")
    for e, (r0, r1) in enumerate(c["rows"]):
        w = c["widths"][e]
        assert (out[r0:r1, w:] == 0).all() and (pre[r0:r1, w:] == 0).all()
    # down: feed the reference H with NaN in the tails (must never be read)
    h_in = h_ref.clone()
    for e, (r0, r1) in enumerate(c["rows"]):
        h_in[r0:r1, c["widths"][e]:] = float("nan")
    y = grouped_gemm_down(h_in.to(torch.bfloat16).to(device), c["w2"].to(device), eto, ewo,
                          wid, tpe, c["d"])
    y_ref = torch.zeros(c["P"], c["d"])
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], c["offsets"][e]
        y_ref[r0:r1] = bf(h_ref[r0:r1, :w] @ c["w2"][o:o + w].float())
    assert_close_norm(y, y_ref, TIGHT, "Y")


@pytest.mark.parametrize("case", CASES, ids=IDS)
@pytest.mark.parametrize("fused_gather", [False, True])
def test_backward_kernels(case, fused_gather, device):
    c = _case(*case, seed=1)
    eto, ewo, wid, tpe = _meta_dev(c, device)
    P, d, max_w = c["P"], c["d"], c["max_w"]
    g = torch.Generator().manual_seed(2)
    h_ref, pre_ref = _ref_up(c, c["xg"])
    gy = torch.randn(P, d, generator=g).to(torch.bfloat16)
    # down backward
    gh, gw2 = grouped_gemm_down_backward(gy.to(device), h_ref.to(torch.bfloat16).to(device),
                                         c["w2"].to(device), eto, ewo, wid, tpe, d, max_w)
    gh_ref = torch.zeros(P, max_w)
    gw2_ref = torch.zeros(c["W"], d)
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], c["offsets"][e]
        gh_ref[r0:r1, :w] = bf(gy[r0:r1].float() @ c["w2"][o:o + w].float().T)
        gw2_ref[o:o + w] = bf(h_ref[r0:r1, :w].T @ gy[r0:r1].float())
    assert_close_norm(gh, gh_ref, TIGHT, "GH")
    assert_close_norm(gw2, gw2_ref, TIGHT, "GW2")
    for e, (r0, r1) in enumerate(c["rows"]):
        assert (gh[r0:r1, c["widths"][e]:] == 0).all()
    # up backward, from the reference GH and PRE
    ghb = gh_ref.to(torch.bfloat16)
    if fused_gather:
        # x_flat with a gather map: rows of xg come from x_flat[gm]
        T = c["P"] // 2 + 1
        x_flat = torch.randn(T, d, generator=g).to(torch.bfloat16)
        gm = torch.randint(0, T, (P,), generator=g, dtype=torch.int32)
        xs = x_flat[gm.long()]
        x_arg, gm_arg = x_flat.to(device), gm.to(device)
    else:
        xs = c["xg"]
        x_arg, gm_arg = c["xg"].to(device), None
    gx, gw1 = grouped_gemm_up_backward(ghb.to(device), x_arg, c["w1"].to(device),
                                       pre_ref.to(torch.bfloat16).to(device), eto, ewo, wid,
                                       tpe, d, "relu_squared", gather_map=gm_arg)
    ga = bf(torch.where(pre_ref > 0, gh_ref * 2.0 * pre_ref, torch.zeros_like(pre_ref)))
    gx_ref = torch.zeros(P, d)
    gw1_ref = torch.zeros(d, c["W"])
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], c["offsets"][e]
        gx_ref[r0:r1] = bf(ga[r0:r1, :w] @ c["w1"][:, o:o + w].float().T)
        gw1_ref[:, o:o + w] = bf(xs[r0:r1].float().T @ ga[r0:r1, :w])
    assert_close_norm(gx, gx_ref, TIGHT, "GX")
    assert_close_norm(gw1, gw1_ref, TIGHT, "GW1")


def test_empty_experts_get_zero_weight_grads(device):
    c = _case(512, 128, [(8, 128)], 1, 64, False)
    # all tokens to expert 3 -> others empty
    E = c["E"]
    eto = torch.tensor([0, 0, 0, 0, 512, 512, 512, 512, 512], dtype=torch.int32)
    tpe = torch.diff(eto)
    xg = torch.randn(512, 128).to(torch.bfloat16).to(device)
    gy = torch.randn(512, 128).to(torch.bfloat16).to(device)
    h = torch.rand(512, 128).to(torch.bfloat16).to(device)
    d_ = dict(eto=eto.to(device), ewo=c["ewo"].to(device), wid=c["wid"].to(device),
              tpe=tpe.to(device))
    _, gw2 = grouped_gemm_down_backward(gy, h, c["w2"].to(device), d_["eto"], d_["ewo"],
                                        d_["wid"], d_["tpe"], 128, 128)
    _, gw1 = grouped_gemm_up_backward(h, xg, c["w1"].to(device), h, d_["eto"], d_["ewo"],
                                      d_["wid"], d_["tpe"], 128, "relu_squared")
    for e in range(E):
        if e != 3:
            assert (gw2[e * 128:(e + 1) * 128] == 0).all()
            assert (gw1[:, e * 128:(e + 1) * 128] == 0).all()
    assert gw2[384:512].abs().sum() > 0 and gw1[:, 384:512].abs().sum() > 0


def test_uncovered_rows_are_zero(device):
    """tokens_per_expert below the offsets' range leaves rows zero (torch.zeros)."""
    c = _case(256, 128, [(2, 128)], 1, 64, False)
    eto = torch.tensor([0, 128, 256], dtype=torch.int32, device=device)
    tpe = torch.tensor([64, 128], dtype=torch.int32, device=device)
    xg = torch.randn(256, 128).to(torch.bfloat16).to(device)
    out = grouped_gemm_up(xg, c["w1"].to(device), eto, c["ewo"].to(device),
                          c["wid"].to(device), tpe, 128)
    assert (out[64:128] == 0).all() and out[:64].abs().sum() > 0 and out[128:].abs().sum() > 0


def test_activation_none_and_unknown(device):
    c = _case(256, 128, [(2, 128)], 1, 64, False)
    eto, ewo, wid, tpe = _meta_dev(c, device)
    xg = c["xg"].to(device)
    out, pre = grouped_gemm_up(xg, c["w1"].to(device), eto, ewo, wid, tpe, c["max_w"],
                               activation="none", save_pre_act=True)
    ref = torch.zeros(c["P"], c["max_w"])
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], c["offsets"][e]
        ref[r0:r1, :w] = bf(c["xg"][r0:r1].float() @ c["w1"][:, o:o + w].float())
    assert_close_norm(out, ref, TIGHT, "none")
    assert (pre == 0).all()
    out2 = grouped_gemm_up(xg, c["w1"].to(device), eto, ewo, wid, tpe, c["max_w"],
                           activation="gelu")  # unknown -> none, as the reference
    assert torch.equal(out, out2)


def test_up_fwd_gather_map_path(device):
    """grouped_gemm_up(x_flat, gather_map=gm) reads x_flat[gm[row]] (pad rows read row 0)."""
    c = _case(512, 256, [(4, 128)], 2, 64, False)
    eto, ewo, wid, tpe = _meta_dev(c, device)
    T = 300
    x_flat = torch.randn(T, 256).to(torch.bfloat16)
    gm = torch.randint(0, T, (c["P"],), dtype=torch.int32)
    out = grouped_gemm_up(x_flat.to(device), c["w1"].to(device), eto, ewo, wid, tpe,
                          c["max_w"], gather_map=gm.to(device))
    h_ref, _ = _ref_up(c, x_flat[gm.long()])
    assert_close_norm(out, h_ref, TIGHT, "H gm")


@pytest.mark.parametrize("with_workspace", [True, False], ids=["splitk", "no_workspace"])
def test_up_dw_row_map(with_workspace, device):
    """dW1 = x[map]^T @ GA through the row map, called through the C ABI: the
    split-K path (K chunks of 512 rows) and the workspace-free path (whole
    experts of ~1000 rows per item). Map entries outside [0, x_rows), -1 as
    the module's pad rows, read zeros."""
    from triton_moe import _lib
    from triton_moe.kernels.grouped_gemm import _dw_workspace, host_meta

    c = _case(2048, 256, [(2, 256), (2, 128)], 2, 64, False, seed=4)
    eto, ewo, wid, tpe = _meta_dev(c, device)
    P, d, max_w, W = c["P"], c["d"], c["max_w"], c["W"]
    g = torch.Generator().manual_seed(5)
    T = 1500
    x_flat = torch.randn(T, d, generator=g).to(torch.bfloat16)
    gm = torch.randint(0, T, (P,), generator=g, dtype=torch.int32)
    bad = torch.rand(P, generator=g)
    gm[bad < 0.05] = -1
    gm[(bad >= 0.05) & (bad < 0.08)] = T + 7
    ga = (torch.randn(P, max_w, generator=g) * 0.1).to(torch.bfloat16)
    for e, (r0, r1) in enumerate(c["rows"]):
        ga[r0:r1, c["widths"][e]:] = 0
    m = host_meta(eto, ewo, wid, tpe, max_w, d, P, W)
    gw = torch.full((d, W), float("nan"), dtype=torch.bfloat16, device=device)
    ws = _dw_workspace(m, d, device) if with_workspace else None
    xd, gmd, gad = x_flat.to(device), gm.to(device), ga.to(device)
    _lib.call("vmoe_gemm_up_bwd_dw", xd.data_ptr(), xd.stride(0), T, gmd.data_ptr(),
              gad.data_ptr(), gad.stride(0), gw.data_ptr(), gw.stride(0), eto.data_ptr(),
              ewo.data_ptr(), wid.data_ptr(), tpe.data_ptr(), c["E"], d, max_w, P,
              None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
              _lib.stream(xd.device))
    valid = (gm >= 0) & (gm < T)
    xs = torch.where(valid[:, None], x_flat[gm.clamp(0, T - 1).long()], torch.zeros(()))
    ref = torch.zeros(d, W)
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], c["offsets"][e]
        assert r1 - r0 > 8 * 32, "each expert spans more than one map window"
        ref[:, o:o + w] = bf(xs[r0:r1].float().T @ ga[r0:r1, :w].float())
    assert_close_norm(gw, ref, TIGHT, f"GW1 map ws={with_workspace}")


@pytest.mark.parametrize("d,widths,hot", [(512, [256, 128, 256], 30000),
                                          (2048, [1024, 512, 1024], 6000)],
                         ids=["lanes4", "lanes8"])
def test_dw_split_tiles_across_many_lanes(d, widths, hot, device):
    """One expert holds almost every row, so its tiles' K chunks span many
    workgroup lanes (three or more segments per tile): the wave finishing a
    tile's last segment sums the partials in lane order. Checked against the
    per-expert reference, for bitwise determinism over repeated calls (the
    arrival words are left zero for the next call), and against the split-K
    free path within the summation-order tolerance. d x max width >= 2^21
    takes lanes of 8 workgroups, smaller shapes lanes of 4."""
    from triton_moe import _lib
    from triton_moe.kernels.grouped_gemm import _dw_workspace, host_meta

    g = torch.Generator().manual_seed(11)
    E = len(widths)
    offsets = [0]
    for w in widths:
        offsets.append(offsets[-1] + w)
    counts = [hot, 64, 0]            # hot, small, empty
    pad = [(c + 63) // 64 * 64 for c in counts]
    eto = torch.tensor([0] + list(torch.tensor(pad).cumsum(0)), dtype=torch.int32)
    P, W, max_w = int(eto[-1]), offsets[-1], max(widths)
    tpe = torch.diff(eto)
    ewo = torch.tensor(offsets, dtype=torch.int32)
    wid = torch.tensor(widths, dtype=torch.int32)
    xg = torch.randn(P, d, generator=g).to(torch.bfloat16)
    ga = (torch.randn(P, max_w, generator=g) * 0.1).to(torch.bfloat16)
    h = torch.randn(P, max_w, generator=g).abs().to(torch.bfloat16)
    gy = (torch.randn(P, d, generator=g) * 0.1).to(torch.bfloat16)
    for e in range(E):
        r0, r1 = int(eto[e]), int(eto[e + 1])
        ga[r0:r1, widths[e]:] = 0
        h[r0:r1, widths[e]:] = 0
        ga[r0 + counts[e]:r1] = 0
        h[r0 + counts[e]:r1] = 0
    dev = [t.to(device) for t in (eto, ewo, wid, tpe)]
    m = host_meta(*dev, max_w, d, P, W)
    xd, gad, hd, gyd = (t.to(device) for t in (xg, ga, h, gy))
    ws = _dw_workspace(m, d, device)

    def dw1(workspace):
        out = torch.full((d, W), float("nan"), dtype=torch.bfloat16, device=device)
        _lib.call("vmoe_gemm_up_bwd_dw", xd.data_ptr(), xd.stride(0), 0, None, gad.data_ptr(),
                  gad.stride(0), out.data_ptr(), out.stride(0), *(t.data_ptr() for t in dev),
                  E, d, max_w, P, None if workspace is None else workspace.data_ptr(),
                  0 if workspace is None else workspace.numel(), _lib.stream(xd.device))
        return out

    def dw2(workspace):
        out = torch.full((W, d), float("nan"), dtype=torch.bfloat16, device=device)
        _lib.call("vmoe_gemm_down_bwd_dw", hd.data_ptr(), hd.stride(0), gyd.data_ptr(),
                  gyd.stride(0), 0, None, None, out.data_ptr(), out.stride(0),
                  *(t.data_ptr() for t in dev), E, d, max_w, P,
                  None if workspace is None else workspace.data_ptr(),
                  0 if workspace is None else workspace.numel(), _lib.stream(xd.device))
        return out

    ref1 = torch.zeros(d, W)
    ref2 = torch.zeros(W, d)
    for e in range(E):
        r0, r1 = int(eto[e]), int(eto[e + 1])
        w, o = widths[e], offsets[e]
        ref1[:, o:o + w] = bf(xg[r0:r1].float().T @ ga[r0:r1, :w].float())
        ref2[o:o + w] = bf(h[r0:r1, :w].float().T @ gy[r0:r1].float())
    a1, a2 = dw1(ws), dw2(ws)
    assert_close_norm(a1, ref1, TIGHT, "dW1 split across lanes")
    assert_close_norm(a2, ref2, TIGHT, "dW2 split across lanes")
    for _ in range(3):
        assert torch.equal(dw1(ws), a1) and torch.equal(dw2(ws), a2)
    zb = int(_lib.lib().vmoe_gemm_dw_workspace_zero_bytes())
    assert int(ws[:zb].count_nonzero()) == 0, "arrival words left non-zero"
    assert_close_norm(dw1(None), ref1, TIGHT, "dW1 without split-K")
    assert_close_norm(dw2(None), ref2, TIGHT, "dW2 without split-K")


@pytest.mark.parametrize("broadcast", [False, True], ids=["token_rows", "broadcast_row"])
def test_weighted_rows_through_map(broadcast, device):
    """The module's fused path: H' = bf16(w_r relu(z)^2) from x_flat[map]
    (up GEMM with row map and row factor), then from the token gradient G read
    through the map: GA = relu^2 rule of bf16(w_r (G[map] @ W2^T)) (dH GEMM)
    and dW2 = H'^T G[map] (dW GEMM). Map entries -1 (pad rows) read zeros;
    a row-broadcast G (stride 0, the gradient of out.sum()) is one row."""
    from triton_moe.kernels.grouped_gemm import down_bwd, host_meta, up_fwd

    c = _case(2048, 256, [(2, 256), (2, 128), (2, 64)], 2, 64, False, seed=6)
    eto, ewo, wid, tpe = _meta_dev(c, device)
    P, d, max_w, W = c["P"], c["d"], c["max_w"], c["W"]
    g = torch.Generator().manual_seed(7)
    T = 1200
    x_flat = torch.randn(T, d, generator=g).to(torch.bfloat16)
    gm = torch.randint(0, T, (P,), generator=g, dtype=torch.int32)
    gm[torch.rand(P, generator=g) < 0.05] = -1
    w = torch.rand(P, generator=g).to(torch.bfloat16).float()
    w[gm < 0] = 0.0
    m = host_meta(eto, ewo, wid, tpe, max_w, d, P, W)
    h, pre = up_fwd(x_flat.to(device), c["w1"].to(device), m, 1, True, True,
                    gather_map=gm.to(device), row_scale=w.to(device))
    xs = torch.where((gm >= 0)[:, None], x_flat[gm.clamp(min=0).long()], torch.zeros(()))
    h_ref = torch.zeros(P, max_w)
    pre_ref = torch.zeros(P, max_w)
    for e, (r0, r1) in enumerate(c["rows"]):
        wd, o = c["widths"][e], c["offsets"][e]
        z = torch.relu(xs[r0:r1].float() @ c["w1"][:, o:o + wd].float())
        pre_ref[r0:r1, :wd] = bf(z)
        h_ref[r0:r1, :wd] = bf(w[r0:r1, None] * z ** 2)
    assert_close_norm(h, h_ref, TIGHT, "H' (row-scaled)")
    assert_close_norm(pre, pre_ref, TIGHT, "PRE")
    if broadcast:
        G = torch.randn(1, d, generator=g).to(torch.bfloat16).expand(T, d)
    else:
        G = torch.randn(T, d, generator=g).to(torch.bfloat16)
    hb, preb = h_ref.to(torch.bfloat16), pre_ref.to(torch.bfloat16)
    ga, gw2 = down_bwd(G.to(device), hb.to(device), c["w2"].to(device), m, d, True,
                       pre=preb.to(device), gather_map=gm.to(device), row_scale=w.to(device))
    Gs = torch.where((gm >= 0)[:, None], G[gm.clamp(min=0).long()], torch.zeros(())).float()
    ga_ref = torch.zeros(P, max_w)
    gw2_ref = torch.zeros(W, d)
    for e, (r0, r1) in enumerate(c["rows"]):
        wd, o = c["widths"][e], c["offsets"][e]
        gh = bf(w[r0:r1, None] * (Gs[r0:r1] @ c["w2"][o:o + wd].float().T))
        p_ = preb[r0:r1, :wd].float()
        ga_ref[r0:r1, :wd] = bf(torch.where(p_ > 0, 2.0 * gh * p_, torch.zeros(())))
        gw2_ref[o:o + wd] = bf(hb[r0:r1, :wd].float().T @ Gs[r0:r1])
    assert_close_norm(ga, ga_ref, TIGHT, "GA (mapped, row-scaled)")
    assert_close_norm(gw2, gw2_ref, TIGHT, "GW2 (mapped)")


def test_autograd_entry_points(device):
    """grouped_gemm_up_autograd -> grouped_gemm_down_autograd -> sum().backward()
    (the reference's test_grouped_gemm_backward flow, in bf16)."""
    c = _case(1024, 256, [(4, 256), (4, 128)], 2, 64, False, seed=3)
    eto, ewo, wid, tpe = _meta_dev(c, device)
    x = c["xg"].to(device).requires_grad_(True)
    w1 = c["w1"].to(device).requires_grad_(True)
    w2 = c["w2"].to(device).requires_grad_(True)
    h = grouped_gemm_up_autograd(x, w1, eto, ewo, wid, tpe, c["max_w"], c["d"], "relu_squared")
    y = grouped_gemm_down_autograd(h, w2, eto, ewo, wid, tpe, c["d"], c["max_w"])
    # forward equals the raw kernels
    raw = grouped_gemm_down(grouped_gemm_up(x.detach(), w1.detach(), eto, ewo, wid, tpe,
                                            c["max_w"]), w2.detach(), eto, ewo, wid, tpe,
                            c["d"])
    assert torch.equal(y.detach(), raw)
    y.sum().backward()
    for t in (x, w1, w2):
        assert t.grad is not None and torch.isfinite(t.grad.float()).all()
        assert t.grad.abs().sum() > 0
    # against the per-expert fp32 reference with the same bf16 rounding points
    h_ref, pre_ref = _ref_up(c, c["xg"])
    gy = torch.ones(c["P"], c["d"])
    gx_ref = torch.zeros(c["P"], c["d"])
    gw1_ref = torch.zeros_like(c["w1"], dtype=torch.float32)
    gw2_ref = torch.zeros_like(c["w2"], dtype=torch.float32)
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], c["offsets"][e]
        ghe = bf(gy[r0:r1] @ c["w2"][o:o + w].float().T)
        gw2_ref[o:o + w] = bf(h_ref[r0:r1, :w].T @ gy[r0:r1])
        pre = pre_ref[r0:r1, :w]
        ga = bf(torch.where(pre > 0, ghe * 2.0 * pre, torch.zeros_like(pre)))
        gx_ref[r0:r1] = bf(ga @ c["w1"][:, o:o + w].float().T)
        gw1_ref[:, o:o + w] = bf(c["xg"][r0:r1].float().T @ ga)
    assert_close_norm(x.grad, gx_ref, TIGHT, "x.grad")
    assert_close_norm(w1.grad, gw1_ref, TIGHT, "w1.grad")
    assert_close_norm(w2.grad, gw2_ref, TIGHT, "w2.grad")


@pytest.mark.parametrize("activation", ["relu_squared", "swiglu"])
def test_reference_module_chain_autograd(activation, device):
    """The reference module's call chain (moe.py:184-250) through the public API:
    fused_route -> precompute_gather_map -> padded_gather_autograd ->
    grouped_gemm_up_autograd(..., x_flat=x_flat, gather_map=gather_map) ->
    grouped_gemm_down_autograd -> padded_scatter_autograd, forward and
    backward. relu_squared is held to the oracle rounding where the
    reference's kernels do (mode "bf16") at TIGHT; swiglu (whose backward the
    reference leaves unfinished) runs the up stage with x_flat and gather_map
    against float64 autograd at LOOSE."""
    from oracle import eager
    from triton_moe.kernels import (
        fused_route,
        padded_gather_autograd,
        padded_scatter_autograd,
        precompute_gather_map,
    )

    from _util import make_problem

    T, d, sizes, k, b = 768, 256, [(4, 256), (4, 128)], 2, 64
    p = make_problem(T, d, sizes, k, b, seed=21, device=device)
    E = p["E"]
    sel = p["sel"].reshape(-1)
    wts = p["wts"].reshape(-1)
    bin_ids, indices, _tpe, bins, padded_bins = fused_route(sel, E, block_size=b, rounding="up")
    eto = torch.cat([torch.zeros(1, device=device, dtype=torch.int32), padded_bins])
    ptpe = torch.cat([padded_bins[:1], padded_bins[1:] - padded_bins[:-1]])
    gm = precompute_gather_map(indices, bin_ids, bins, padded_bins, k)
    wid = torch.tensor(p["widths"], dtype=torch.int32, device=device)
    max_w = max(p["widths"])
    x_flat = p["x"].to(device).requires_grad_(True)
    G = torch.randn(T, d, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16)
    if activation == "relu_squared":
        ewo = torch.tensor(p["offsets"], dtype=torch.int32, device=device)
        w1 = p["w1"].to(device).requires_grad_(True)
        w2 = p["w2"].to(device).requires_grad_(True)
        xg = padded_gather_autograd(x_flat, indices, bin_ids, bins, padded_bins, k)
        h = grouped_gemm_up_autograd(xg, w1, eto, ewo, wid, ptpe, max_w, d, "relu_squared",
                                     x_flat=x_flat, gather_map=gm)
        y = grouped_gemm_down_autograd(h, w2, eto, ewo, wid, ptpe, d, max_w)
        out = padded_scatter_autograd(y, indices, bin_ids, wts, bins, padded_bins, k)
        out.backward(G.to(device))
        prob = eager.Problem(p["x"].float(), p["w1"].float(), p["w2"].float(), p["widths"],
                             p["offsets"], p["sel"].cpu(), p["wts"].cpu().float(), b)
        fb = eager.forward(prob, "bf16")
        bb = eager.backward(prob, fb, G.float(), "bf16")
        assert_close_norm(out, fb["out"], TIGHT, "chain out")
        for got, key in ((x_flat.grad, "grad_x"), (w1.grad, "grad_w1"), (w2.grad, "grad_w2")):
            assert_close_norm(got, bb[key], TIGHT, f"chain {key}")
        return
    # swiglu: W1 holds gate and up halves per expert
    g = torch.Generator().manual_seed(23)
    offs2 = [0]
    for w in p["widths"]:
        offs2.append(offs2[-1] + 2 * w)
    w1s = (torch.randn(d, offs2[-1], generator=g) * 0.05).to(torch.bfloat16)
    ewo2 = torch.tensor(offs2, dtype=torch.int32, device=device)
    w1 = w1s.to(device).requires_grad_(True)
    xg = padded_gather_autograd(x_flat, indices, bin_ids, bins, padded_bins, k)
    h = grouped_gemm_up_autograd(xg, w1, eto, ewo2, wid, ptpe, max_w, d, "swiglu",
                                 x_flat=x_flat, gather_map=gm)
    Gh = torch.randn(h.shape, generator=g).to(torch.bfloat16)
    h.backward(Gh.to(device))
    # float64 reference: the padded gather (zeros on pad rows), then swiglu
    pb = [0] + padded_bins.cpu().tolist()
    rows = [(pb[e], pb[e + 1]) for e in range(E)]
    gmap = gm.cpu().long()
    r = eager.route(eager.Problem(p["x"].float(), p["w1"].float(), p["w2"].float(),
                                  p["widths"], p["offsets"], p["sel"].cpu(),
                                  p["wts"].cpu().float(), b))
    pad = torch.from_numpy(r["row_src"]) < 0
    x64 = p["x"].double().requires_grad_(True)
    xg64 = torch.where(pad[:, None], torch.zeros((), dtype=torch.float64), x64[gmap])
    w164 = w1s.double().requires_grad_(True)
    h_ref, _ = eager.swiglu_up(xg64, w164, rows, p["widths"], offs2[:-1], max_w)
    h_ref.backward(Gh.double())
    assert_close_norm(h, h_ref, LOOSE, "chain swiglu H")
    assert_close_norm(x_flat.grad, x64.grad, LOOSE, "chain swiglu grad_x")
    assert_close_norm(w1.grad, w164.grad, LOOSE, "chain swiglu grad_w1")


def test_fp16_inputs_not_supported(device):
    """bf16 and fp32 (tests/test_gpu_gemm_f32.py) are taken; fp16 is refused
    loudly rather than cast."""
    eto = torch.tensor([0, 128, 256], dtype=torch.int32, device=device)
    wid = torch.tensor([128, 128], dtype=torch.int32, device=device)
    x = torch.randn(256, 64, device=device).half()
    w1 = torch.randn(64, 256, device=device).half()
    with pytest.raises(NotImplementedError, match="bfloat16"):
        grouped_gemm_up(x, w1, eto, eto, wid, wid, 128)
    with pytest.raises(NotImplementedError, match="float32"):
        grouped_gemm_up(x, w1.float(), eto, eto, wid, wid, 128)


def _swiglu_case(seed=31, skew=False):
    sizes = [(4, 128), (4, 64)] if skew else [(2, 128), (2, 64)]
    c = _case(512, 256, sizes, 2, 64, skew, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    offs2 = [0]
    for w in c["widths"]:
        offs2.append(offs2[-1] + 2 * w)
    c["w1s"] = (torch.randn(c["d"], offs2[-1], generator=g) * 0.05).to(torch.bfloat16)
    c["ewo2"] = torch.tensor(offs2, dtype=torch.int32)
    c["offs2"] = offs2
    return c


@pytest.mark.parametrize("public_backward,skew", [(False, False), (True, False), (False, True)])
def test_swiglu_forward_backward(public_backward, skew, device):
    """activation="swiglu" (gate at ewo_e + c, up at ewo_e + w_e + c, as the
    reference's forward, grouped_gemm.py:295-349) against float64 autograd of
    the oracle; the backward the reference leaves unfinished (:768-790) is
    held to the same LOOSE normwise tolerance (gate, up, dG and dU are
    rounded to bf16). test_swiglu_rounding_order holds both at TIGHT to an
    fp32 reference with the kernels' rounding points."""
    from oracle import eager
    from triton_moe.kernels import grouped_gemm_up_autograd, grouped_gemm_up_backward

    c = _swiglu_case(skew=skew)  # skew: hot experts and four that receive no rows
    eto, _, wid, tpe = _meta_dev(c, device)
    ewo2 = c["ewo2"].to(device)
    xg64 = c["xg"].double().requires_grad_(True)
    w164 = c["w1s"].double().requires_grad_(True)
    h_ref, gate_ref = eager.swiglu_up(xg64, w164, c["rows"], c["widths"], c["offs2"][:-1],
                                      c["max_w"])
    G = (torch.randn(h_ref.shape, generator=torch.Generator().manual_seed(5))).to(torch.bfloat16)
    h_ref.backward(G.double())
    xg, w1 = c["xg"].to(device), c["w1s"].to(device)
    out, pre = grouped_gemm_up(xg, w1, eto, ewo2, wid, tpe, c["max_w"], activation="swiglu",
                               save_pre_act=True)
    assert_close_norm(out, h_ref, LOOSE, "swiglu H")
    assert_close_norm(pre, gate_ref, TIGHT, "swiglu gate")
    if public_backward:
        gx, gw1 = grouped_gemm_up_backward(G.to(device), xg, w1, pre, eto, ewo2, wid, tpe,
                                           c["d"], activation="swiglu")
    else:
        xr = xg.clone().requires_grad_(True)
        w1r = w1.clone().requires_grad_(True)
        o2 = grouped_gemm_up_autograd(xr, w1r, eto, ewo2, wid, tpe, c["max_w"], c["d"],
                                      activation="swiglu")
        assert torch.equal(o2, out)
        o2.backward(G.to(device))
        gx, gw1 = xr.grad, w1r.grad
    assert_close_norm(gx, xg64.grad, LOOSE, "swiglu grad_x")
    assert_close_norm(gw1, w164.grad, LOOSE, "swiglu grad_w1")


def test_swiglu_gather_map_path(device):
    """activation="swiglu" with gather_map: forward reads x_flat[gm[row]] for both
    halves, and the public backward (which recomputes the up half through the
    map) gives grad_w1 of the gathered rows; grad_x stays in gathered rows."""
    from oracle import eager
    from triton_moe.kernels import grouped_gemm_up_backward

    c = _swiglu_case(seed=41)
    eto, _, wid, tpe = _meta_dev(c, device)
    ewo2 = c["ewo2"].to(device)
    T = 300
    x_flat = torch.randn(T, c["d"], generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    gm = torch.randint(0, T, (c["P"],), dtype=torch.int32,
                       generator=torch.Generator().manual_seed(43))
    xg64 = x_flat[gm.long()].double().requires_grad_(True)
    w164 = c["w1s"].double().requires_grad_(True)
    h_ref, gate_ref = eager.swiglu_up(xg64, w164, c["rows"], c["widths"], c["offs2"][:-1],
                                      c["max_w"])
    G = torch.randn(h_ref.shape, generator=torch.Generator().manual_seed(44)).to(torch.bfloat16)
    h_ref.backward(G.double())
    xd, w1, gmd = x_flat.to(device), c["w1s"].to(device), gm.to(device)
    out, pre = grouped_gemm_up(xd, w1, eto, ewo2, wid, tpe, c["max_w"], activation="swiglu",
                               save_pre_act=True, gather_map=gmd)
    assert_close_norm(out, h_ref, LOOSE, "swiglu H gm")
    assert_close_norm(pre, gate_ref, TIGHT, "swiglu gate gm")
    gx, gw1 = grouped_gemm_up_backward(G.to(device), xd, w1, pre, eto, ewo2, wid, tpe, c["d"],
                                       activation="swiglu", gather_map=gmd)
    assert_close_norm(gx, xg64.grad, LOOSE, "swiglu grad_x gm")
    assert_close_norm(gw1, w164.grad, LOOSE, "swiglu grad_w1 gm")


def _glu_ref32(c, xg, w1, offs, G):
    """fp32 swiglu with the fused kernels' rounding points: H = bf16(silu(g) u)
    and gate = bf16(g) from fp32 g, u; the backward from the bf16 gate and up
    (dG, dU rounded to bf16) with grad_x one fp32 sum over both halves and
    grad_w1 per column, each rounded once."""
    P, max_w, d = c["P"], c["max_w"], c["d"]
    h = torch.zeros(P, max_w)
    gate = torch.zeros(P, max_w)
    gx = torch.zeros(P, d)
    gw1 = torch.zeros(w1.shape)
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], offs[e]
        x32 = xg[r0:r1].float()
        wg, wu = w1[:, o:o + w].float(), w1[:, o + w:o + 2 * w].float()
        g, u = x32 @ wg, x32 @ wu
        h[r0:r1, :w] = bf(g * torch.sigmoid(g) * u)
        gate[r0:r1, :w] = bf(g)
        gb, ub = bf(g), bf(u)
        sg = torch.sigmoid(gb)
        gh = G[r0:r1, :w].float()
        dg = bf(gh * ub * sg * (1 + gb * (1 - sg)))
        du = bf(gh * gb * sg)
        gx[r0:r1] = bf(dg @ wg.T + du @ wu.T)
        gw1[:, o:o + w] = bf(x32.T @ dg)
        gw1[:, o + w:o + 2 * w] = bf(x32.T @ du)
    return h, gate, gx, gw1


@pytest.mark.parametrize("gapped,public_backward", [(False, False), (False, True),
                                                    (True, False), (True, True)])
def test_swiglu_rounding_order(gapped, public_backward, device):
    """The fused swiglu (one GEMM whose epilogue forms silu(g) u from the fp32
    accumulators, the reference's order, grouped_gemm.py:347-349; backward
    as [dG | dU] through one dX and one dW GEMM) against an fp32 reference
    with the same rounding points at TIGHT, with W1's expert column ranges
    contiguous (2 w_e apart) or with gaps between them (the backward then
    gathers the ranges into a contiguous copy)."""
    from triton_moe.kernels import grouped_gemm_up_autograd, grouped_gemm_up_backward

    c = _swiglu_case(seed=51, skew=True)
    offs = c["offs2"]
    w1 = c["w1s"]
    if gapped:
        offs = [o + 8 * e for e, o in enumerate(offs)]
        g = torch.Generator().manual_seed(52)
        w1 = (torch.randn(c["d"], offs[-1] + 16, generator=g) * 0.05).to(torch.bfloat16)
    ewo = torch.tensor(offs, dtype=torch.int32).to(device)
    eto, _, wid, tpe = _meta_dev(c, device)
    G = torch.randn(c["P"], c["max_w"], generator=torch.Generator().manual_seed(53))
    G = G.to(torch.bfloat16)
    for e, (r0, r1) in enumerate(c["rows"]):
        G[r0:r1, c["widths"][e]:] = 0
    h_ref, gate_ref, gx_ref, gw1_ref = _glu_ref32(c, c["xg"], w1, offs, G.float())
    xg, w1d = c["xg"].to(device), w1.to(device)
    out, pre = grouped_gemm_up(xg, w1d, eto, ewo, wid, tpe, c["max_w"], activation="swiglu",
                               save_pre_act=True)
    assert_close_norm(out, h_ref, TIGHT, "fused swiglu H")
    assert_close_norm(pre, gate_ref, TIGHT, "fused swiglu gate")
    if public_backward:
        gx, gw1 = grouped_gemm_up_backward(G.to(device), xg, w1d, pre, eto, ewo, wid, tpe,
                                           c["d"], activation="swiglu")
    else:
        xr = xg.clone().requires_grad_(True)
        w1r = w1d.clone().requires_grad_(True)
        o2 = grouped_gemm_up_autograd(xr, w1r, eto, ewo, wid, tpe, c["max_w"], c["d"],
                                      activation="swiglu")
        assert bits_equal(o2, out)
        o2.backward(G.to(device))
        gx, gw1 = xr.grad, w1r.grad
    assert_close_norm(gx, gx_ref, TIGHT, "fused swiglu grad_x")
    assert_close_norm(gw1, gw1_ref, TIGHT, "fused swiglu grad_w1")
    if gapped:
        used = torch.zeros(w1.shape[1], dtype=torch.bool)
        for e, o in enumerate(offs[:-1]):
            used[o:o + 2 * c["widths"][e]] = True
        assert int(gw1.cpu()[:, ~used].abs().sum()) == 0, "columns outside the experts"


def test_glu_row_scale_and_gather_map_capi(device):
    """vmoe_gemm_up_glu through the C ABI with a gather map and row factors:
    out = bf16(row_scale * silu(g) u), gate = bf16(g), up = bf16(u) from the
    fp32 accumulators of x[map[row]] (pad rows, map -1, read zeros)."""
    from triton_moe import _lib
    from triton_moe.kernels.grouped_gemm import _meta_args, glu_meta

    c = _swiglu_case(seed=61, skew=True)
    eto, _, wid, tpe = _meta_dev(c, device)
    ewo = torch.tensor(c["offs2"], dtype=torch.int32, device=device)
    T = 300
    g = torch.Generator().manual_seed(62)
    x_flat = torch.randn(T, c["d"], generator=g).to(torch.bfloat16)
    gm = torch.randint(-1, T, (c["P"],), dtype=torch.int32, generator=g)
    rs = torch.rand(c["P"], generator=g)
    m = glu_meta(eto, ewo, wid, tpe, c["max_w"], c["d"], c["w1s"].shape[1]).fwd
    P, mw = c["P"], c["max_w"]
    outs = [torch.zeros(P, mw, dtype=torch.bfloat16, device=device) for _ in range(3)]
    # device copies held for the whole (asynchronous) launch
    xd, w1d, gmd, rsd = (t.to(device) for t in (x_flat, c["w1s"], gm, rs))
    _lib.call("vmoe_gemm_up_glu", xd.data_ptr(), xd.stride(0), T, gmd.data_ptr(),
              w1d.data_ptr(), w1d.stride(0), *(o.data_ptr() for o in outs), mw,
              rsd.data_ptr(), *_meta_args(m), c["d"], mw, P, _lib.stream(device))
    torch.cuda.synchronize()
    xs = torch.where((gm >= 0)[:, None], x_flat[gm.clamp(min=0).long()], torch.zeros(()))
    h_ref, g_ref, u_ref = (torch.zeros(P, mw) for _ in range(3))
    for e, (r0, r1) in enumerate(c["rows"]):
        w, o = c["widths"][e], c["offs2"][e]
        x32 = xs[r0:r1].float()
        gg_ = x32 @ c["w1s"][:, o:o + w].float()
        uu = x32 @ c["w1s"][:, o + w:o + 2 * w].float()
        h_ref[r0:r1, :w] = bf(rs[r0:r1, None] * (gg_ * torch.sigmoid(gg_) * uu))
        g_ref[r0:r1, :w] = bf(gg_)
        u_ref[r0:r1, :w] = bf(uu)
    assert_close_norm(outs[0], h_ref, TIGHT, "glu H with row factors")
    assert_close_norm(outs[1], g_ref, TIGHT, "glu gate")
    assert_close_norm(outs[2], u_ref, TIGHT, "glu up")


def test_column_slice_operands(device):
    """grouped_gemm_up / _down on column slices of wider tensors (rows 2 bytes
    past a 16-byte boundary) give the bits of contiguous copies."""
    c = _case(1024, 256, [(4, 512), (4, 256)], 2, 128, False)
    eto, ewo, wid, tpe = _meta_dev(c, device)
    P, d, W, max_w = c["P"], c["d"], c["W"], c["max_w"]
    g = torch.Generator().manual_seed(4)
    xw = torch.randn(P, d + 8, generator=g).to(torch.bfloat16).to(device)
    w1w = (torch.randn(d, W + 8, generator=g) * 0.05).to(torch.bfloat16).to(device)
    w2w = (torch.randn(W, d + 8, generator=g) * 0.05).to(torch.bfloat16).to(device)
    res = []
    for sliced in (True, False):
        def view(t, n):
            v = t[:, 1:1 + n]
            return v if sliced else v.contiguous()
        x, w1, w2 = view(xw, d), view(w1w, W), view(w2w, d)
        if sliced:
            assert x.data_ptr() % 16 == 2 and w1.data_ptr() % 16 == 2
        h, pre = grouped_gemm_up(x, w1, eto, ewo, wid, tpe, max_w, activation="relu_squared",
                                 save_pre_act=True)
        y = grouped_gemm_down(h, w2, eto, ewo, wid, tpe, d)
        res.append((h, pre, y))
    torch.cuda.synchronize()
    for a, b in zip(*res):
        assert bits_equal(a, b)
