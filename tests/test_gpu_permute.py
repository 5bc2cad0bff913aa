"""Gather / weighted gather / combine on the GPU are bit-exact with the
oracle (reference gather.py:34-60, 145-174 and scatter.py:35-69, 133)."""

from __future__ import annotations

import pytest
import torch

from oracle import eager
from oracle import route as oroute
from triton_moe.kernels import (
    fused_route,
    padded_gather,
    padded_gather_autograd,
    padded_scatter,
    padded_scatter_autograd,
)
from triton_moe.kernels.gather import combine_rows, gather_rows
from triton_moe.kernels.fused_cumsum import check_route, route_device

from _util import bits_equal

pytestmark = pytest.mark.gpu


def _setup(T, d, E, k, b, device, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    wts, sel = torch.topk(torch.sigmoid(logits), k, dim=-1)
    wts = (wts / wts.sum(-1, keepdim=True)).to(torch.bfloat16)
    r = oroute.route(sel.reshape(-1).numpy(), E, b, "up")
    maps = oroute.row_maps(r["indices"], r["bin_ids"], r["bins"], r["padded_bins"], k,
                           num_assignments=T * k)
    return x, sel, wts, r, maps


def _ref_gather(x, maps, k, w=None):
    rs = torch.from_numpy(maps["row_src"]).long()
    out = torch.zeros(rs.numel(), x.shape[1], dtype=torch.bfloat16)
    ok = rs >= 0
    v = x[rs[ok] // k].float()
    if w is not None:
        v = v * w.reshape(-1)[rs[ok]].float()[:, None]
    out[ok] = v.to(torch.bfloat16)
    return out


@pytest.mark.parametrize("T,d,E,k,b", [(128, 128, 4, 2, 128), (1024, 256, 8, 2, 128),
                                       (2048, 768, 16, 2, 64), (1024, 1024, 64, 8, 64),
                                       (300, 100, 5, 2, 8), (257, 2056, 7, 3, 64)])
def test_gather_and_weighted_gather_exact(T, d, E, k, b, device):
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device)
    dev = lambda a: torch.as_tensor(a).to(device)  # noqa: E731
    P = int(r["padded_bins"][-1])
    got = padded_gather(x.to(device), dev(r["indices"]), dev(r["bin_ids"]), dev(r["bins"]),
                        dev(r["padded_bins"]), k)
    assert got.shape == (P, d)
    assert bits_equal(got, _ref_gather(x, maps, k))
    rs = dev(maps["row_src"])
    gw = gather_rows(x.to(device), rs, k, P, weights=wts.reshape(-1).to(device))
    assert bits_equal(gw, _ref_gather(x, maps, k, wts))


@pytest.mark.parametrize("T,d,E,k,b", [(128, 128, 4, 2, 128), (1024, 256, 8, 2, 128),
                                       (1024, 1024, 64, 8, 64), (300, 100, 5, 2, 8),
                                       (100, 2056, 6, 4, 16)])
def test_combine_exact(T, d, E, k, b, device):
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device, seed=1)
    P = int(r["padded_bins"][-1])
    y = torch.randn(P, d, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    ar = torch.from_numpy(maps["assignment_row"])
    ref_w = eager.combine(y.float(), ar.numpy(), wts.reshape(-1).float(), k, T, "bf16")
    ref_u = eager.combine(y.float(), ar.numpy(), None, k, T, "bf16")
    got_w = combine_rows(y.to(device), ar.to(device), k, T, weights=wts.reshape(-1).to(device))
    got_u = combine_rows(y.to(device), ar.to(device), k, T)
    assert bits_equal(got_w, ref_w.to(torch.bfloat16))
    assert bits_equal(got_u, ref_u.to(torch.bfloat16))
    dev = lambda a: torch.as_tensor(a).to(device)  # noqa: E731
    pub = padded_scatter(y.to(device), dev(r["indices"]), dev(r["bin_ids"]),
                         wts.reshape(-1).to(device), dev(r["bins"]), dev(r["padded_bins"]), k)
    assert bits_equal(pub, ref_w.to(torch.bfloat16))


def test_autograd_gather_scatter(device):
    T, d, E, k, b = 512, 256, 8, 2, 64
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device, seed=3)
    dev = lambda a: torch.as_tensor(a).to(device)  # noqa: E731
    idx, bid, bins, pb = (dev(r["indices"]), dev(r["bin_ids"]), dev(r["bins"]),
                          dev(r["padded_bins"]))
    xg = x.to(device).requires_grad_(True)
    g = padded_gather_autograd(xg, idx, bid, bins, pb, k)
    G = torch.randn(g.shape, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    g.backward(G.to(device))
    ar = maps["assignment_row"]
    ref_gx = eager.combine(G.float(), ar, None, k, T, "bf16").to(torch.bfloat16)
    assert bits_equal(xg.grad, ref_gx)
    # scatter backward = weighted gather (pad rows zero); weights get no grad
    P = int(r["padded_bins"][-1])
    y = torch.randn(P, d, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    yd = y.to(device).requires_grad_(True)
    wd = wts.reshape(-1).to(device).requires_grad_(True)
    out = padded_scatter_autograd(yd, idx, bid, wd, bins, pb, k)
    GO = torch.randn(out.shape, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    out.backward(GO.to(device))
    assert bits_equal(yd.grad, _ref_gather(GO, maps, k, wts))
    assert wd.grad is None


def test_strided_and_broadcast_inputs(device):
    """Row strides other than hidden (views) and stride-0 grads (out.sum())."""
    T, d, E, k, b = 256, 128, 4, 2, 64
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device, seed=7)
    wide = torch.zeros(T, d + 64, dtype=torch.bfloat16)
    wide[:, :d] = x
    dev = lambda a: torch.as_tensor(a).to(device)  # noqa: E731
    got = padded_gather(wide.to(device)[:, :d], dev(r["indices"]), dev(r["bin_ids"]),
                        dev(r["bins"]), dev(r["padded_bins"]), k)
    assert bits_equal(got, _ref_gather(x, maps, k))
    yd = got.clone().requires_grad_(True)
    out = padded_scatter_autograd(yd, dev(r["indices"]), dev(r["bin_ids"]),
                                  wts.reshape(-1).to(device), dev(r["bins"]),
                                  dev(r["padded_bins"]), k)
    out.sum().backward()
    ones = torch.ones(T, d, dtype=torch.bfloat16)
    assert bits_equal(yd.grad, _ref_gather(ones, maps, k, wts))


def test_column_slice_inputs(device):
    """Column slices of wider tensors (rows 2 bytes past a 16-byte boundary)
    as gather source, weighted gather source and scatter input: the bits of
    the contiguous case (the kernels' element-wise paths)."""
    T, d, E, k, b = 256, 128, 4, 2, 64
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device, seed=8)
    dev = lambda a: torch.as_tensor(a).to(device)  # noqa: E731
    idx, bid, bins, pb = (dev(r[n]) for n in ("indices", "bin_ids", "bins", "padded_bins"))
    wide = torch.zeros(T, d + 8, dtype=torch.bfloat16)
    wide[:, 1:1 + d] = x
    xs = wide.to(device)[:, 1:1 + d]
    assert xs.data_ptr() % 16 == 2
    got = padded_gather(xs, idx, bid, bins, pb, k)
    assert bits_equal(got, _ref_gather(x, maps, k))
    wv = wts.reshape(-1).to(device)
    P = got.shape[0]
    ywide = torch.zeros(P, d + 8, dtype=torch.bfloat16, device=device)
    ywide[:, 1:1 + d] = got
    ys = ywide[:, 1:1 + d]
    assert bits_equal(padded_scatter(ys, idx, bid, wv, bins, pb, k),
                      padded_scatter(got, idx, bid, wv, bins, pb, k))


def test_route_maps_feed_permutation(device):
    """route_device's own maps give the same gather as the public API."""
    T, d, E, k = 1000, 256, 16, 4
    x, sel, wts, r, maps = _setup(T, d, E, k, 64, device, seed=8)
    rd = route_device(sel.reshape(-1).to(device), E, k, 64)
    P, _ = check_route(rd)
    got = gather_rows(x.to(device), rd.row_src, k, P)
    assert bits_equal(got, _ref_gather(x, maps, k))
    pub = fused_route(sel.reshape(-1).to(device), E, block_size=64)
    assert torch.equal(pub[1].cpu(), torch.from_numpy(r["indices"]))


@pytest.mark.parametrize("T,d,E,k,b", [(128, 128, 4, 2, 128), (1024, 256, 8, 2, 128),
                                       (2048, 768, 16, 2, 64), (1024, 1024, 64, 8, 64),
                                       (300, 104, 5, 2, 8), (257, 2056, 7, 3, 64),
                                       (300, 100, 5, 2, 8)])
def test_token_major_gather_exact(T, d, E, k, b, device):
    """The token-by-token gather (x read once per token) writes the same rows,
    weighted or not, with zero pad rows (d = 100 takes the row-by-row path)."""
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device, seed=9)
    P = int(r["padded_bins"][-1])
    rs = torch.as_tensor(maps["row_src"]).to(device)
    ar = torch.as_tensor(maps["assignment_row"]).to(device)
    # fill the output allocator with garbage first: every row must be written
    torch.full((P + 64, d), 7.0, dtype=torch.bfloat16, device=device)
    got = gather_rows(x.to(device), rs, k, P, assignment_row=ar)
    assert bits_equal(got, _ref_gather(x, maps, k))
    gw = gather_rows(x.to(device), rs, k, P, weights=wts.reshape(-1).to(device),
                     assignment_row=ar)
    assert bits_equal(gw, _ref_gather(x, maps, k, wts))


def test_token_major_gather_broadcast_and_row_cap(device):
    """A stride-0 input is read from one row; a device row count caps the output."""
    T, d, E, k, b = 512, 256, 8, 4, 64
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device, seed=10)
    rd = route_device(sel.reshape(-1).to(device), E, k, b)
    P, _ = check_route(rd)
    row = torch.randn(1, d, generator=torch.Generator().manual_seed(11)).to(torch.bfloat16)
    full = row.expand(T, d)
    for xin in (row.to(device).expand(T, d), torch.ones((), dtype=torch.bfloat16,
                                                         device=device).expand(T, d)):
        ref_x = full if xin.stride(1) == 1 else torch.ones(T, d, dtype=torch.bfloat16)
        got = gather_rows(xin, rd.row_src, k, rd.rows_bound, weights=wts.reshape(-1).to(device),
                          num_rows_dev=rd.info[0:1], assignment_row=rd.assignment_row)
        assert bits_equal(got[:P], _ref_gather(ref_x, maps, k, wts))


def _abs_dot(G, y, ar, k, T):
    """Per-slot sum |g| |y| (scales the fp32 summation-order tolerance)."""
    return eager.combine_weight_grad(G.float().abs(), y.float().abs(), ar, k, T)


@pytest.mark.parametrize("T,d,E,k,b", [(512, 256, 8, 2, 64), (300, 100, 6, 3, 32),
                                       (1024, 1024, 64, 8, 128), (1, 8, 2, 2, 16)])
def test_combine_weight_grad(T, d, E, k, b, device):
    """Opt-in routing-weight gradient (absent in the reference, scatter.py:176)
    against the float64 oracle, slots without a row included. Tolerance: the
    kernel sums in fp32 in another order, so |got - ref| <= 1e-5 * sum|g||y|."""
    from triton_moe.kernels.gather import combine_weight_grad

    x, sel, wts, r, maps = _setup(T, d, E, k, b, device, seed=11)
    P = int(r["padded_bins"][-1])
    gen = torch.Generator().manual_seed(12)
    y = torch.randn(P, d, generator=gen).to(torch.bfloat16)
    G = torch.randn(T, d, generator=gen).to(torch.bfloat16)
    ar = torch.as_tensor(maps["assignment_row"]).clone()
    ar[::5] = -1  # unplaced slots (dropped tokens) give 0
    ref = eager.combine_weight_grad(G.float(), y.float(), ar.numpy(), k, T)
    got = combine_weight_grad(G.to(device), y.to(device), ar.to(device), k).cpu().double()
    tol = 1e-5 * _abs_dot(G, y, ar.numpy(), k, T) + 1e-30
    assert got.shape == ref.shape
    assert bool(((got - ref).abs() <= tol).all())
    assert bool((got[::5] == 0).all())


def test_combine_weight_grad_empty(device):
    """No tokens: an empty fp32 gradient, no launch."""
    from triton_moe.kernels.gather import combine_weight_grad

    y = torch.zeros(4, 16, dtype=torch.bfloat16, device=device)
    g = torch.zeros(0, 16, dtype=torch.bfloat16, device=device)
    ar = torch.zeros(0, dtype=torch.int32, device=device)
    got = combine_weight_grad(g, y, ar, 2)
    assert got.shape == (0,) and got.dtype == torch.float32


def test_padded_scatter_weight_grad_opt_in(device):
    """padded_scatter_autograd(..., weight_grad=True): the routing weights get the
    gradient (bf16, at most one bf16 rounding step from the oracle); the input
    gradient is unchanged; a broadcast output gradient (out.sum()) works."""
    T, d, E, k, b = 512, 256, 8, 4, 64
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device, seed=13)
    dev = lambda a: torch.as_tensor(a).to(device)  # noqa: E731
    idx, bid, bins, pb = (dev(r["indices"]), dev(r["bin_ids"]), dev(r["bins"]),
                          dev(r["padded_bins"]))
    P = int(r["padded_bins"][-1])
    y = torch.randn(P, d, generator=torch.Generator().manual_seed(14)).to(torch.bfloat16)
    ar = maps["assignment_row"]
    for G in (torch.randn(T, d, generator=torch.Generator().manual_seed(15)).to(torch.bfloat16),
              None):
        yd = y.to(device).requires_grad_(True)
        wd = wts.reshape(-1).to(device).requires_grad_(True)
        out = padded_scatter_autograd(yd, idx, bid, wd, bins, pb, k, weight_grad=True)
        if G is None:
            out.sum().backward()
            G = torch.ones(T, d, dtype=torch.bfloat16)
        else:
            out.backward(G.to(device))
        ref = eager.combine_weight_grad(G.float(), y.float(), ar, k, T)
        tol = ref.abs() * 2.0 ** -8 + 1e-5 * _abs_dot(G, y, ar, k, T) + 1e-30
        assert wd.grad is not None and wd.grad.dtype == torch.bfloat16
        assert bool(((wd.grad.cpu().double() - ref).abs() <= tol).all())
        assert bits_equal(yd.grad, _ref_gather(G, maps, k, wts))


@pytest.mark.parametrize("T,d,E,k,b", [(128, 128, 4, 2, 128), (1024, 256, 8, 2, 128),
                                       (300, 100, 5, 2, 8), (257, 2058, 7, 3, 64)])
def test_f32_gather_combine_and_weight_grad(T, d, E, k, b, device):
    """The fp32 permutation (vmoe_gather_f32, vmoe_combine_f32,
    vmoe_combine_weight_grad_f32) through the public API in float32:
    gathers are exact copies / single fp32 products, the combine is the fp32
    sum in slot order (bit-equal to the same sum on the host), and the
    weight gradient is within fp32 summation order of float64. Odd d takes
    the scalar path."""
    x, sel, wts, r, maps = _setup(T, d, E, k, b, device)
    x32 = x.float() + torch.randn(T, d, generator=torch.Generator().manual_seed(1)) * 1e-3
    w32 = wts.float() * (1 + 1e-3 * torch.rand(T, k, generator=torch.Generator().manual_seed(2)))
    dev = lambda a: torch.as_tensor(a).to(device)  # noqa: E731
    P = int(r["padded_bins"][-1])
    rs = torch.from_numpy(maps["row_src"]).long()
    ok = rs >= 0
    got = padded_gather(x32.to(device), dev(r["indices"]), dev(r["bin_ids"]), dev(r["bins"]),
                        dev(r["padded_bins"]), k)
    ref = torch.zeros(P, d)
    ref[ok] = x32[rs[ok] // k]
    assert got.dtype == torch.float32 and torch.equal(got.cpu(), ref)
    gw = gather_rows(x32.to(device), dev(maps["row_src"]).int(), k, P,
                     weights=w32.reshape(-1).to(device))
    refw = torch.zeros(P, d)
    refw[ok] = x32[rs[ok] // k] * w32.reshape(-1)[rs[ok]][:, None]
    assert torch.equal(gw.cpu(), refw)
    # combine: sum over slots in ascending j, fp32, with and without weights
    y = torch.randn(P, d, generator=torch.Generator().manual_seed(3))
    ar = torch.from_numpy(maps["assignment_row"]).long().view(T, k)
    for w in (None, w32):
        out = combine_rows(y.to(device), dev(maps["assignment_row"]).int(), k, T,
                           weights=None if w is None else w.reshape(-1).to(device))
        ref = torch.zeros(T, d)
        for j in range(k):
            rows = ar[:, j]
            m = rows >= 0
            slot = torch.zeros(T, d)
            slot[m] = y[rows[m]] * (1.0 if w is None else w[m, j][:, None])
            ref = ref + slot
        assert torch.equal(out.cpu(), ref), "fp32 combine"
    # weight gradient of the weighted fp32 scatter (opt-in)
    G = torch.randn(T, d, generator=torch.Generator().manual_seed(4))
    yy = y.to(device).requires_grad_(False)
    ws = w32.reshape(-1).to(device).requires_grad_(True)
    out = padded_scatter_autograd(yy, dev(r["indices"]), dev(r["bin_ids"]), ws, dev(r["bins"]),
                                  dev(r["padded_bins"]), k, weight_grad=True)
    out.backward(G.to(device))
    refg = eager.combine_weight_grad(G, y, maps["assignment_row"], k, T)
    assert ws.grad.dtype == torch.float32
    mag = eager.combine_weight_grad(G.abs(), y.abs(), maps["assignment_row"], k, T)
    assert ((ws.grad.cpu().double() - refg).abs() <= 1e-6 * mag + 1e-30).all()


def test_public_api_empty_inputs(device):
    """No routed tokens through the public operators: the reference returns
    zero tensors early (gather.py:93-94, scatter.py:101-102,
    grouped_gemm.py:430-433, 617-618, 1214-1215, 1333-1334): the padded
    gather is [padded rows, d] of zeros, the scatter [tokens, d] of zeros,
    the grouped GEMMs [0, width] / [0, d], their weight gradients zeros."""
    from triton_moe.kernels import (fused_route, grouped_gemm_down, grouped_gemm_down_backward,
                                    grouped_gemm_up, grouped_gemm_up_backward, padded_gather,
                                    padded_scatter)

    d, E, k, b, max_w = 64, 4, 2, 64, 128
    widths = torch.tensor([128, 64, 128, 64], dtype=torch.int32, device=device)
    ewo = torch.tensor([0, 128, 192, 320, 384], dtype=torch.int32, device=device)
    W = 384
    w1 = torch.randn(d, W, device=device).to(torch.bfloat16)
    w2 = torch.randn(W, d, device=device).to(torch.bfloat16)
    sel = torch.empty(0, dtype=torch.int64, device=device)
    bin_ids, indices, tpe, bins, padded_bins = fused_route(sel, E, block_size=b)
    x = torch.zeros(0, d, dtype=torch.bfloat16, device=device)
    xg = padded_gather(x, indices, bin_ids, bins, padded_bins, k)
    assert xg.shape == (int(padded_bins[-1]), d) and int(xg.count_nonzero()) == 0
    eto = torch.zeros(E + 1, dtype=torch.int32, device=device)
    ptpe = torch.zeros(E, dtype=torch.int32, device=device)
    x0 = torch.zeros(0, d, dtype=torch.bfloat16, device=device)
    h, pre = grouped_gemm_up(x0, w1, eto, ewo, widths, ptpe, max_w, save_pre_act=True)
    assert h.shape == (0, max_w) and pre.shape == (0, max_w)
    y = grouped_gemm_down(h, w2, eto, ewo, widths, ptpe, d)
    assert y.shape == (0, d)
    gy = torch.zeros(0, d, dtype=torch.bfloat16, device=device)
    gh, gw2 = grouped_gemm_down_backward(gy, h, w2, eto, ewo, widths, ptpe, d, max_w)
    assert gh.shape == (0, max_w) and gw2.shape == w2.shape and int(gw2.count_nonzero()) == 0
    gx, gw1 = grouped_gemm_up_backward(gh, x0, w1, pre, eto, ewo, widths, ptpe, d)
    assert gx.shape == (0, d) and gw1.shape == w1.shape and int(gw1.count_nonzero()) == 0
    wts = torch.zeros(0, dtype=torch.bfloat16, device=device)
    out = padded_scatter(xg, indices, bin_ids, wts, bins, padded_bins, k)
    assert out.shape == (0, d)
    torch.cuda.synchronize()
