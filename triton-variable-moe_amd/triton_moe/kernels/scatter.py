"""Padded scatter (weighted combine) on the gfx950 permutation kernels.

Mirrors triton_moe/kernels/scatter.py of the reference: padded_scatter
(:72-133), PaddedScatterOp (:141-176) and padded_scatter_autograd (:179-189).
The reference writes bf16(y * w) into a zero-filled [T, k, d] intermediate and
sums it with torch; here one kernel reads the k rows of each token through an
assignment -> row map and sums the bf16-rounded products in fp32 registers,
which gives the same value with a third of the HBM traffic. As in the
reference, the routing weights receive no gradient by default;
padded_scatter_autograd(..., weight_grad=True) adds it (the reference returns
None for them, scatter.py:176): gw[t*k+j] = sum_c G[t, c] * x[row(t, j), c].
"""

from __future__ import annotations

import torch
from torch.amp import custom_bwd, custom_fwd
from torch.autograd.function import once_differentiable

from .. import _lib
from .gather import combine_rows, combine_weight_grad, gather_rows, row_maps


@torch.compiler.disable
def padded_scatter(
    x: torch.Tensor,
    indices: torch.Tensor,
    bin_ids: torch.Tensor,
    weights: torch.Tensor,
    bins: torch.Tensor,
    padded_bins: torch.Tensor,
    top_k: int,
) -> torch.Tensor:
    """Scatter with padding (megablocks.ops.padded_scatter interface).

    Args:
        x: Padded gathered tensor [padded_bins[-1], hidden_size].
        weights: Routing weights [num_tokens * top_k], indexed by t * top_k + j.

    Returns:
        [num_tokens, hidden_size]: sum over j of x[row(t, j)] * weights[t*k + j].
    """
    _lib.require_gpu(x)
    total_padded = x.shape[0]
    num_tokens = len(weights) // top_k
    _, _, ar = row_maps(indices, bin_ids, bins, padded_bins, top_k, total_padded,
                        num_tokens * top_k, want_row_src=False, want_assignment_row=True)
    return combine_rows(x, ar, top_k, num_tokens, weights=weights)


class PaddedScatterOp(torch.autograd.Function):
    """Autograd function for padded_scatter; backward is the weighted gather."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x, indices, bin_ids, weights, bins, padded_bins, top_k,
                weight_grad=False):
        _lib.require_gpu(x)
        total_padded = x.shape[0]
        num_tokens = len(weights) // top_k
        rs, _, ar = row_maps(indices, bin_ids, bins, padded_bins, top_k, total_padded,
                             num_tokens * top_k, want_assignment_row=True)
        ctx.weight_grad = bool(weight_grad)
        if ctx.weight_grad:
            ctx.save_for_backward(rs, weights, x, ar)
        else:
            ctx.save_for_backward(rs, weights)
        ctx.top_k = top_k
        ctx.total_padded = total_padded
        return combine_rows(x, ar, top_k, num_tokens, weights=weights)

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, grad_output):
        rs, weights = ctx.saved_tensors[:2]
        grad_x = None
        if ctx.needs_input_grad[0]:
            grad_x = gather_rows(grad_output, rs, ctx.top_k, ctx.total_padded, weights=weights)
        grad_w = None
        if ctx.weight_grad and ctx.needs_input_grad[3]:
            x, ar = ctx.saved_tensors[2:]
            grad_w = combine_weight_grad(grad_output, x, ar, ctx.top_k).to(weights.dtype)
            grad_w = grad_w.reshape(weights.shape)
        return grad_x, None, None, grad_w, None, None, None, None


def padded_scatter_autograd(x, indices, bin_ids, weights, bins, padded_bins, top_k,
                            weight_grad: bool = False):
    """Padded scatter with autograd support.

    weight_grad=True (opt-in, not in the reference) also returns the gradient
    of the routing weights when they require it."""
    return PaddedScatterOp.apply(x, indices, bin_ids, weights, bins, padded_bins, top_k,
                                 weight_grad)
