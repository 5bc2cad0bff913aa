"""Routing on the GPU is bit-exact with the oracle (fused_route semantics,
triton_moe/kernels/fused_cumsum.py:85-171 and grouped_gemm.py:104-149)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import route as oroute
from triton_moe.kernels import fused_route, precompute_gather_map
from triton_moe.kernels.fused_cumsum import check_route, route_device

from _util import zipf_bias

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "route_cases.json").read_text())


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("case", GOLDEN, ids=[c["name"] for c in GOLDEN])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_route_golden(case, dtype, device):
    sel = torch.tensor(case["selected"], dtype=dtype, device=device)
    E, k, b, mode = case["num_experts"], case["top_k"], case["block_size"], case["rounding"]
    exp = case["expected"]
    r = route_device(sel, E, k, b, mode)
    P, n = check_route(r)
    assert P == (exp["padded_bins"][-1] if E else 0)
    assert n == len(exp["bin_ids"])
    np.testing.assert_array_equal(_np(r.bin_ids[:n]), exp["bin_ids"])
    np.testing.assert_array_equal(_np(r.indices[:n]), exp["indices"])
    np.testing.assert_array_equal(_np(r.tokens_per_expert), exp["tokens_per_expert"])
    np.testing.assert_array_equal(_np(r.bins), exp["bins"])
    np.testing.assert_array_equal(_np(r.padded_bins), exp["padded_bins"])
    np.testing.assert_array_equal(_np(r.row_src[:P]), exp["row_src"])
    np.testing.assert_array_equal(_np(r.gather_map[:P]), exp["gather_map"])
    np.testing.assert_array_equal(_np(r.assignment_row), exp["assignment_row"])
    # the module's expert_token_offsets and padded counts (moe.py:193-202)
    pb = np.asarray(exp["padded_bins"], dtype=np.int64)
    np.testing.assert_array_equal(_np(r.expert_offsets), np.concatenate([[0], pb]))
    np.testing.assert_array_equal(_np(r.padded_counts), np.diff(np.concatenate([[0], pb])))
    # public entry point
    out = fused_route(sel, E, block_size=b, rounding=mode)
    for t, key in zip(out, ("bin_ids", "indices", "tokens_per_expert", "bins", "padded_bins")):
        assert t.dtype == torch.int32
        np.testing.assert_array_equal(_np(t), exp[key], err_msg=key)
    if mode == "up" and len(case["selected"]):
        gm = precompute_gather_map(out[1], out[0], out[3], out[4], k)
        np.testing.assert_array_equal(_np(gm), exp["gather_map"])


# (tokens, top_k, experts, block): the BASELINE.json shapes and the reference's
# test fixtures (b=128), random top-k routing on the device.
SHAPES = [(2 * 64, 2, 4, 128), (4 * 256, 2, 8, 128), (8 * 512, 2, 8, 64),
          (8 * 1024, 2, 8, 64), (8 * 2048, 2, 16, 64), (16384, 8, 64, 64),
          (32768, 8, 128, 64), (4096, 8, 1000, 16),
          # past the two-launch path's limits (E * tiles > 65536, E > 1024):
          # the three-launch path with the single-workgroup scan
          (65536, 8, 256, 64), (4096, 4, 2048, 16)]


@pytest.mark.parametrize("T,k,E,b", SHAPES)
@pytest.mark.parametrize("mode", ["up", "nearest", "down"])
def test_route_random_topk(T, k, E, b, mode, device):
    g = torch.Generator(device=device).manual_seed(T + E)
    logits = torch.randn(T, E, device=device, generator=g)
    if E == 64:
        logits = logits + zipf_bias(E, alpha=3.0).to(device)
    sel = torch.topk(logits, k, dim=-1).indices.reshape(-1)
    r = route_device(sel, E, k, b, mode)
    P, n = check_route(r)
    ref = oroute.route(_np(sel), E, b, mode)
    maps = oroute.row_maps(ref["indices"], ref["bin_ids"], ref["bins"], ref["padded_bins"], k,
                           num_assignments=sel.numel())
    assert P == int(ref["padded_bins"][-1]) and n == ref["bin_ids"].size
    np.testing.assert_array_equal(_np(r.bin_ids[:n]), ref["bin_ids"])
    np.testing.assert_array_equal(_np(r.indices[:n]), ref["indices"])
    for key in ("tokens_per_expert", "bins", "padded_bins"):
        np.testing.assert_array_equal(_np(getattr(r, key)), ref[key], err_msg=key)
    np.testing.assert_array_equal(_np(r.row_src[:P]), maps["row_src"])
    np.testing.assert_array_equal(_np(r.gather_map[:P]), maps["gather_map"])
    np.testing.assert_array_equal(_np(r.assignment_row), maps["assignment_row"])
    # the module's map: pad rows -1 (read as zeros by the GEMMs' row gather),
    # and each row's routing weight (0 on pad rows)
    wts = torch.rand(sel.numel(), generator=g, device=device).to(torch.bfloat16)
    r2 = route_device(sel, E, k, b, mode, map_pad=-1, weights=wts)
    gm2 = np.where(maps["row_src"] < 0, -1, maps["gather_map"])
    np.testing.assert_array_equal(_np(r2.gather_map[:P]), gm2)
    np.testing.assert_array_equal(_np(r2.row_src[:P]), maps["row_src"])
    rs = torch.from_numpy(maps["row_src"]).long()
    rw_ref = torch.where(rs >= 0, wts.cpu().float()[rs.clamp(min=0)], torch.zeros(()))
    assert torch.equal(r2.row_weight[:P].cpu(), rw_ref)


def test_route_deterministic_and_large(device):
    T, k, E = 65536, 8, 256
    sel = torch.randint(0, E, (T * k,), device=device)
    a = route_device(sel, E, k, 64)
    b = route_device(sel, E, k, 64)
    P, _ = check_route(a)
    assert check_route(b)[0] == P
    # rows past P of the capacity-sized maps are never written, by design
    for x, y in ((a.indices, b.indices), (a.row_src[:P], b.row_src[:P]),
                 (a.gather_map[:P], b.gather_map[:P]), (a.assignment_row, b.assignment_row),
                 (a.padded_bins, b.padded_bins)):
        assert torch.equal(x, y)
    ref = oroute.route(_np(sel), E, 64, "up")
    np.testing.assert_array_equal(_np(a.indices), ref["indices"])


def test_route_bad_ids_raise(device):
    with pytest.raises(RuntimeError, match="outside"):
        fused_route(torch.tensor([0, 7, 1], device=device), 4)
    with pytest.raises(RuntimeError, match="outside"):
        fused_route(torch.tensor([0, -1, 1], device=device), 4)


def test_route_empty(device):
    out = fused_route(torch.empty(0, dtype=torch.int64, device=device), 5, block_size=64)
    assert out[0].numel() == 0 and out[1].numel() == 0
    assert out[2].tolist() == [0] * 5 and out[4].tolist() == [0] * 5
