"""vmoe_route_static (routing without a workspace argument or any allocation:
its workspace is a file-scope device array) gives the same bits as
vmoe_route with a caller-allocated workspace, on two calls in a row, the
second one smaller than the first, through the C ABI."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from triton_moe import _lib
from triton_moe.kernels.fused_cumsum import route_device, rows_upper_bound

pytestmark = pytest.mark.gpu


def _static_route(sel, E, k, b, rounding, map_pad, weights):
    """The outputs of vmoe_route_static in buffers shaped as route_device's."""
    dev = sel.device
    A = sel.numel()
    cap = rows_upper_bound(A, E, b, rounding)
    i32 = dict(dtype=torch.int32, device=dev)
    out = dict(
        bin_ids=torch.full((max(A, 1),), -7, **i32),
        indices=torch.full((max(A, 1),), -7, **i32),
        tokens_per_expert=torch.full((E,), -7, **i32),
        bins=torch.full((E,), -7, **i32),
        padded_bins=torch.full((E,), -7, **i32),
        row_src=torch.full((max(cap, 1),), -7, **i32),
        gather_map=torch.full((max(cap, 1),), -7, **i32),
        assignment_row=torch.full((max(A, 1),), -7, **i32),
        info=torch.full((_lib.INFO_LEN,), -7, **i32),
        expert_offsets=torch.full((E + 1,), -7, **i32),
        padded_counts=torch.full((E,), -7, **i32),
        row_weight=torch.full((max(cap, 1),), -7.0, dtype=torch.float32, device=dev),
    )
    o = out
    st = _lib.lib().vmoe_route_static(
        sel.data_ptr(), int(sel.dtype == torch.int64), A, E, k, b, _lib.ROUNDING[rounding],
        o["bin_ids"].data_ptr(), o["indices"].data_ptr(), o["tokens_per_expert"].data_ptr(),
        o["bins"].data_ptr(), o["padded_bins"].data_ptr(), o["row_src"].data_ptr(),
        o["gather_map"].data_ptr(), map_pad, cap, o["assignment_row"].data_ptr(),
        o["info"].data_ptr(), o["expert_offsets"].data_ptr(), o["padded_counts"].data_ptr(),
        weights.data_ptr(), o["row_weight"].data_ptr(), _lib.stream(dev))
    assert st == _lib.OK, _lib.lib().vmoe_status_string(st)
    return out


def _compare(sel, E, k, b, rounding, weights):
    ref = route_device(sel, E, k, b, rounding, map_pad=-1, weights=weights)
    got = _static_route(sel, E, k, b, rounding, -1, weights)
    torch.cuda.synchronize()
    info = ref.info.cpu().tolist()
    assert got["info"].cpu().tolist() == info
    P, n = info[_lib.INFO_ROWS], info[_lib.INFO_KEPT]
    A = sel.numel()
    pairs = [("bin_ids", ref.bin_ids, n), ("indices", ref.indices, n),
             ("tokens_per_expert", ref.tokens_per_expert, E), ("bins", ref.bins, E),
             ("padded_bins", ref.padded_bins, E), ("row_src", ref.row_src, P),
             ("gather_map", ref.gather_map, P), ("assignment_row", ref.assignment_row, A),
             ("expert_offsets", ref.expert_offsets, E + 1),
             ("padded_counts", ref.padded_counts, E)]
    for name, r, cnt in pairs:
        np.testing.assert_array_equal(got[name][:cnt].cpu().numpy(), r[:cnt].cpu().numpy(),
                                      err_msg=name)
    np.testing.assert_array_equal(got["row_weight"][:P].cpu().view(torch.int32).numpy(),
                                  ref.row_weight[:P].cpu().view(torch.int32).numpy(),
                                  err_msg="row_weight")
    return P


def _inputs(T, E, k, skew, seed, device):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    if skew:
        logits[:, : max(1, E // 8)] += 3.0
        logits[:, E - 2:] -= 50.0
    sel = torch.topk(logits, k, dim=-1).indices.to(torch.int32).reshape(-1)
    w = torch.rand(T * k, generator=g).to(torch.bfloat16)
    return sel.to(device), w.to(device)


def test_route_static_matches_route_twice(device):
    # first call: config-3 shape; second: a smaller one on the same array
    sel, w = _inputs(16384, 64, 8, True, 0, device)
    P1 = _compare(sel, 64, 8, 64, "up", w)
    sel2, w2 = _inputs(1000, 16, 2, False, 1, device)
    P2 = _compare(sel2, 16, 2, 64, "up", w2)
    assert P2 < P1
    # and token dropping on the small shape (rounding on the device)
    _compare(sel2, 16, 2, 64, "down", w2)


def test_route_static_rejects_oversize(device):
    A, E = 1 << 20, 2048
    assert _lib.lib().vmoe_route_workspace_bytes(A, E) > (1 << 20)
    st = _lib.lib().vmoe_route_static(None, 0, A, E, 1, 64, 0, None, None, None, None, None,
                                      None, None, 0, 0, None, None, None, None, None, None,
                                      _lib.stream(device))
    assert st == _lib.ERR_WORKSPACE
