"""Host-side logic that needs no GPU: config, module construction, metadata
validation, bounds, and that the product path refuses CPU tensors instead of
falling back."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import route as oroute
from triton_moe import TritonMoEConfig, TritonMoEMLP
from triton_moe.kernels import (
    fused_route,
    grouped_gemm_down,
    grouped_gemm_up,
    padded_gather,
    precompute_gather_map,
)
from triton_moe.kernels.fused_cumsum import rows_upper_bound
from triton_moe.kernels.grouped_gemm import host_meta


def test_config_defaults_match_reference():
    c = TritonMoEConfig()
    assert (c.n_embd, c.expert_sizes, c.num_active_experts, c.norm_topk_prob, c.block_size,
            c.use_megablocks_gather_scatter) == (768, [(64, 256)], 8, True, 64, False)


def test_module_layout_and_buffers():
    cfg = TritonMoEConfig(n_embd=64, expert_sizes=[(2, 128), (3, 64)], num_active_experts=2)
    m = TritonMoEMLP(cfg)
    assert m.num_experts == 5 and m.total_expert_width == 448 and m.max_expert_width == 128
    assert m.w1.shape == (64, 448) and m.w2.shape == (448, 64)
    assert m.router.weight.shape == (5, 64) and m.router.bias is None
    assert m.expert_widths_t.tolist() == [128, 128, 64, 64, 64]
    assert m.expert_weight_offsets_t.tolist() == [0, 128, 256, 320, 384, 448]
    assert m.expert_widths_t.dtype == torch.int32
    assert set(m.state_dict()) == {"router.weight", "w1", "w2"}
    assert m.group_sizes.tolist() == [2.0, 3.0]
    assert m.w1.abs().max() <= 0.06 and m.w2.abs().max() <= 0.06


def test_rng_order_router_w1_w2():
    """Identical seeds give the initial weights of the reference's construction
    order: router Linear, then w1, then w2 (triton_moe/moe.py:78-85)."""
    torch.manual_seed(11)
    m = TritonMoEMLP(TritonMoEConfig(n_embd=32, expert_sizes=[(4, 64)], num_active_experts=2))
    torch.manual_seed(11)
    router = nn.Linear(32, 4, bias=False)
    w1 = torch.empty(32, 256)
    w2 = torch.empty(256, 32)
    nn.init.trunc_normal_(w1, mean=0.0, std=0.02, a=-0.06, b=0.06)
    nn.init.trunc_normal_(w2, mean=0.0, std=0.02, a=-0.06, b=0.06)
    assert torch.equal(m.router.weight, router.weight)
    assert torch.equal(m.w1, w1) and torch.equal(m.w2, w2)


def test_width_must_divide_block():
    with pytest.raises(AssertionError):
        TritonMoEMLP(TritonMoEConfig(n_embd=32, expert_sizes=[(2, 96)], block_size=64))


def test_cpu_tensors_are_refused_not_computed():
    m = TritonMoEMLP(TritonMoEConfig(n_embd=32, expert_sizes=[(4, 64)], num_active_experts=2))
    x = torch.randn(1, 8, 32)
    with pytest.raises(AssertionError, match="CUDA"):
        m(x)
    with pytest.raises(AssertionError, match="CUDA"):
        fused_route(torch.tensor([0, 1]), 2)
    with pytest.raises(AssertionError, match="CUDA"):
        padded_gather(x[0], torch.tensor([0]), torch.tensor([0]), torch.tensor([1]),
                      torch.tensor([64]), 1)
    with pytest.raises(AssertionError, match="CUDA"):
        precompute_gather_map(torch.tensor([0]), torch.tensor([0]), torch.tensor([1]),
                              torch.tensor([64]), 1)
    i = torch.tensor([0, 64], dtype=torch.int32)
    with pytest.raises(AssertionError, match="CUDA"):
        grouped_gemm_up(x[0], torch.zeros(32, 64), i, i, i[1:], i[1:], 64)
    with pytest.raises(AssertionError, match="CUDA"):
        grouped_gemm_down(x[0], torch.zeros(64, 32), i, i, i[1:], i[1:], 32)


def test_bad_rounding_mode():
    with pytest.raises(AssertionError):
        fused_route(torch.tensor([0, 1]), 2, rounding="sideways")


def _meta(eto, ewo, widths, tpe, max_w=128, hidden=64, rows=None, total=None):
    t = lambda v: torch.tensor(v, dtype=torch.int32)  # noqa: E731
    return host_meta(t(eto), t(ewo), t(widths), t(tpe), max_w, hidden, rows, total)


def test_host_meta_validation_and_coverage():
    m = _meta([0, 64, 192], [0, 128, 192], [128, 64], [64, 128], total=192)
    assert m.full_rows and m.full_cols and not m.uniform and m.rows == 192
    # tokens_per_expert smaller than the offsets' range leaves rows unwritten
    m = _meta([0, 64, 192], [0, 128, 192], [128, 64], [64, 64], total=192)
    assert not m.full_rows
    # weight columns with a gap are not fully covered
    m = _meta([0, 64, 192], [0, 128, 200], [128, 64], [64, 128], total=200)
    assert not m.full_cols
    with pytest.raises(NotImplementedError):
        _meta([0, 64], [0, 12], [12], [64], max_w=16)
    with pytest.raises(NotImplementedError):
        _meta([0, 64], [0, 16], [16], [64], max_w=16, hidden=20)
    with pytest.raises(ValueError):
        _meta([0, 64, 32], [0, 64, 128], [64, 64], [64, 64])
    with pytest.raises(ValueError):
        _meta([0, 64], [0, 64], [136], [64], max_w=128)
    with pytest.raises(ValueError):
        _meta([0, 64], [0, 64], [64], [64], total=32)
    with pytest.raises(ValueError):
        _meta([0, 64], [0, 64], [64], [-1])


@pytest.mark.parametrize("mode", ["up", "down", "nearest"])
def test_rows_upper_bound_holds(mode):
    rng = np.random.default_rng(0)
    for _ in range(20):
        E = int(rng.integers(1, 70))
        b = int(rng.choice([1, 2, 7, 64, 128]))
        A = int(rng.integers(0, 3000))
        sel = rng.integers(0, E, A)
        r = oroute.route(sel, E, b, mode)
        assert int(r["padded_bins"][-1]) <= rows_upper_bound(A, E, b, mode)


def test_glu_meta_layouts():
    """swiglu metadata: the forward keeps the caller's gate offsets and widths;
    the backward GEMMs get widths 2 w_e over W1's own column ranges when they
    are contiguous (2 w_e apart), else over a gathered contiguous copy whose
    column index lists every expert's gate and up columns in order."""
    from triton_moe.kernels.grouped_gemm import glu_meta

    t = lambda v: torch.tensor(v, dtype=torch.int32)  # noqa: E731
    eto, tpe, widths = t([0, 64, 64, 192]), t([64, 0, 128]), t([16, 8, 16])
    m = glu_meta(eto, t([0, 32, 48, 80]), widths, tpe, 16, 64, 80)
    assert m.cols is None
    assert m.fwd.ewo.tolist() == [0, 32, 48, 80] and m.fwd.widths.tolist() == [16, 8, 16]
    assert m.bwd.widths.tolist() == [32, 16, 32] and m.bwd.max_width == 32
    assert m.bwd.ewo.tolist() == [0, 32, 48, 80] and m.bwd.full_cols
    # gaps of 8 columns between the experts' ranges
    m = glu_meta(eto, t([0, 40, 64, 104]), widths, tpe, 16, 64, 104)
    assert m.bwd.ewo.tolist() == [0, 32, 48, 80]
    want = list(range(0, 32)) + list(range(40, 56)) + list(range(64, 96))
    assert m.cols.tolist() == want
    with pytest.raises(ValueError, match="exceed"):
        glu_meta(eto, t([0, 32, 48, 80]), widths, tpe, 16, 64, 72)
    with pytest.raises(NotImplementedError, match="multiples of 8"):
        glu_meta(eto, t([0, 36, 52, 84]), widths, tpe, 16, 64, 96)


@pytest.mark.parametrize("sizes", [[(8, 256)], [(2, 128), (3, 64)], [(1, 128), (1, 64)],
                                   [(1, 256), (4, 128), (1, 64), (3, 32)],
                                   [(32, 1024), (64, 512), (32, 256)]])
def test_load_balance_coef_from_group_buffers(sizes):
    """The module's load-balance coefficients come from its grouping buffers
    and equal the closed form of router.load_balance_coef; with them the one
    dot product sum_e coef f p reproduces the reference's three formulas
    (moe.py:276-303), restated here from the buffers as the reference uses
    them (uniform: E f.p; no group: f.p; groups: mean_g size_g sum_{e in g} f p)."""
    from triton_moe.kernels.router import load_balance_coef

    m = TritonMoEMLP(TritonMoEConfig(n_embd=32, expert_sizes=sizes, num_active_experts=1,
                                     block_size=32))
    coef = m.load_balance_coef()
    assert coef.tolist() == pytest.approx(load_balance_coef(sizes), rel=0, abs=1e-6)
    g = torch.Generator().manual_seed(len(sizes))
    f = torch.rand(m.num_experts, generator=g, dtype=torch.float64)
    p = torch.rand(m.num_experts, generator=g, dtype=torch.float64)
    if len(set(m.expert_widths)) == 1:
        ref = m.num_experts * (f @ p)
    elif m._num_valid_groups == 0:
        ref = f @ p
    else:
        fp = (f * p).index_select(0, m.valid_expert_indices)
        memb = m.group_membership.double().index_select(0, m.valid_expert_indices)
        ref = (m.group_sizes.double() * (fp @ memb)).mean()
    # coef is fp32 (size / num_groups rounded once)
    assert (coef.double() * f * p).sum().item() == pytest.approx(ref.item(), rel=1e-6)
