"""Padded gather on the gfx950 permutation kernels (csrc/permute.hip).

Mirrors triton_moe/kernels/gather.py of the reference: padded_gather
(:63-115), _weighted_padded_gather (:177-218, the scatter backward),
PaddedGatherOp (:226-265) and padded_gather_autograd (:268-277), with the same
arguments, shapes and zero pad rows. The reference zero-fills the whole output
and launches one program per sorted position; here each padded row is written
exactly once (data or zeros) by a row-copy kernel driven by a row -> assignment
map, and the backward is the fused combine instead of a [T, k, d]
intermediate plus torch.sum.
"""

from __future__ import annotations

import torch
from torch.amp import custom_bwd, custom_fwd
from torch.autograd.function import once_differentiable

from .. import _lib


def _require_bf16(t: torch.Tensor, what: str) -> None:
    if t.dtype != torch.bfloat16:
        raise NotImplementedError(f"{what}: only bfloat16 tensors are supported (got {t.dtype})")


def _require_dtype(t: torch.Tensor, what: str) -> bool:
    """True for fp32 rows (the *_f32 entry points), False for bf16."""
    if t.dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError(f"{what}: bfloat16 or float32 tensors only (got {t.dtype})")
    return t.dtype == torch.float32


def _broadcast_rows(t: torch.Tensor):
    """(tensor, leading dimension): a row-broadcast t (row stride 0) as its
    single row with leading dimension 0, else t with unit column stride."""
    if t.shape[0] > 0 and t.stride(0) == 0:
        return (t[:1] if t.stride(1) == 1 else t[:1].contiguous()), 0
    t = _row_major(t)
    return t, t.stride(0)


def _row_major(t: torch.Tensor) -> torch.Tensor:
    """2-D view with unit column stride (the kernels take any row stride)."""
    return t if t.stride(-1) == 1 else t.contiguous()


def row_maps(indices, bin_ids, bins, padded_bins, top_k: int, num_rows: int,
             num_assignments: int, want_row_src=True, want_gather_map=False,
             want_assignment_row=False):
    """row_src / gather_map / assignment_row from caller routing arrays."""
    dev = indices.device
    i32 = dict(dtype=torch.int32, device=dev)
    idx = indices.to(torch.int32).contiguous()
    bid = bin_ids.to(torch.int32).contiguous()
    bns = bins.to(torch.int32).contiguous()
    pbs = padded_bins.to(torch.int32).contiguous()
    rs = torch.empty(max(num_rows, 1), **i32) if want_row_src else None
    gm = torch.empty(max(num_rows, 1), **i32) if want_gather_map else None
    ar = torch.empty(max(num_assignments, 1), **i32) if want_assignment_row else None
    _lib.call("vmoe_row_maps", idx.data_ptr(), bid.data_ptr(), bns.data_ptr(), pbs.data_ptr(),
              idx.numel(), bns.numel(), int(top_k), int(num_rows), int(num_assignments),
              _lib.ptr(rs), _lib.ptr(gm), _lib.ptr(ar), _lib.stream(dev))
    return (rs[:num_rows] if rs is not None else None,
            gm[:num_rows] if gm is not None else None,
            ar[:num_assignments] if ar is not None else None)


def gather_rows(x: torch.Tensor, row_src: torch.Tensor, top_k: int, num_rows: int,
                weights: torch.Tensor | None = None,
                num_rows_dev: torch.Tensor | None = None,
                assignment_row: torch.Tensor | None = None) -> torch.Tensor:
    """out[r] = x[row_src[r] // top_k] (* weights[row_src[r]]), zeros where row_src < 0.

    With assignment_row (the map vmoe_route produces with row_src) the copy
    runs token by token and reads each row of x once; a row-broadcast x (row
    stride 0, such as the gradient of out.sum()) is then read from a single row.
    fp32 x (with fp32 weights) goes to vmoe_gather_f32, row by row.
    """
    hidden = x.shape[1]
    tokens = x.shape[0]
    if _require_dtype(x, "gather"):
        x, ldx = _broadcast_rows(x)
        out = torch.empty(num_rows, hidden, dtype=x.dtype, device=x.device)
        if num_rows == 0 or hidden == 0:
            return out
        w = None if weights is None else weights.to(x.dtype).contiguous()
        _lib.call("vmoe_gather_f32", x.data_ptr(), tokens, ldx, row_src.data_ptr(), int(top_k),
                  _lib.ptr(w), 0 if w is None else w.numel(), out.data_ptr(), out.stride(0),
                  num_rows, _lib.ptr(num_rows_dev), hidden, _lib.stream(x.device))
        return out
    token_major = (assignment_row is not None and hidden % 8 == 0
                   and assignment_row.numel() == tokens * top_k and top_k <= 64)
    if token_major and tokens > 0 and x.stride(0) == 0:
        x, ldx = (x[:1] if x.stride(1) == 1 else x[:1].contiguous()), 0
    else:
        x = _row_major(x)
        ldx = x.stride(0)
    out = torch.empty(num_rows, hidden, dtype=x.dtype, device=x.device)
    if num_rows == 0 or hidden == 0:
        return out
    w = None
    if weights is not None:
        w = weights.to(x.dtype).contiguous()
    if token_major and ldx % 8 == 0 and x.data_ptr() % 16 == 0:
        _lib.call("vmoe_gather_tokens", x.data_ptr(), ldx, assignment_row.data_ptr(), tokens,
                  int(top_k), _lib.ptr(w), row_src.data_ptr(), out.data_ptr(), out.stride(0),
                  num_rows, _lib.ptr(num_rows_dev), hidden, _lib.stream(x.device))
        return out
    _lib.call("vmoe_gather", x.data_ptr(), tokens, ldx, row_src.data_ptr(),
              int(top_k), _lib.ptr(w), 0 if w is None else w.numel(), out.data_ptr(),
              out.stride(0), num_rows, _lib.ptr(num_rows_dev), hidden, _lib.stream(x.device))
    return out


def combine_rows(y: torch.Tensor, assignment_row: torch.Tensor, top_k: int, num_tokens: int,
                 weights: torch.Tensor | None = None) -> torch.Tensor:
    """out[t] = bf16(sum_j f32(bf16(y[row(t,j)] * w[t*k+j]))), unplaced slots add 0
    (fp32 y: the same sum in fp32 with no roundings, vmoe_combine_f32)."""
    sfx = "_f32" if _require_dtype(y, "scatter") else ""
    y = _row_major(y)
    hidden = y.shape[1]
    out = torch.empty(num_tokens, hidden, dtype=y.dtype, device=y.device)
    if num_tokens == 0 or hidden == 0:
        return out
    w = None
    if weights is not None:
        w = weights.to(y.dtype).contiguous()
    _lib.call("vmoe_combine" + sfx, y.data_ptr(), y.shape[0], y.stride(0),
              assignment_row.data_ptr(), _lib.ptr(w), int(top_k), out.data_ptr(), out.stride(0),
              num_tokens, hidden, _lib.stream(y.device))
    return out


def combine_weight_grad(grad: torch.Tensor, y: torch.Tensor, assignment_row: torch.Tensor,
                        top_k: int) -> torch.Tensor:
    """fp32 [T*k]: gw[t*k+j] = sum_c grad[t, c] * y[row(t, j), c], 0 for unplaced slots.

    The routing-weight gradient of combine_rows(y, ..., weights=w), with each
    slot's bf16 rounding taken as identity. A row-broadcast grad (row stride
    0, the gradient of out.sum()) is read from its single row. fp32 y and grad
    go to vmoe_combine_weight_grad_f32."""
    f32 = _require_dtype(y, "combine weight gradient")
    if _require_dtype(grad, "combine weight gradient") != f32:
        raise NotImplementedError("combine weight gradient: grad and y dtypes differ")
    sfx = "_f32" if f32 else ""
    y = _row_major(y)
    tokens, hidden = grad.shape
    grad, ldg = _broadcast_rows(grad)
    gw = torch.empty(tokens * top_k, dtype=torch.float32, device=y.device)
    if gw.numel() == 0:
        return gw
    _lib.call("vmoe_combine_weight_grad" + sfx, grad.data_ptr(), ldg, y.data_ptr(), y.shape[0],
              y.stride(0), assignment_row.data_ptr(), int(top_k), gw.data_ptr(), tokens, hidden,
              _lib.stream(y.device))
    return gw


@torch.compiler.disable
def padded_gather(
    x: torch.Tensor,
    indices: torch.Tensor,
    bin_ids: torch.Tensor,
    bins: torch.Tensor,
    padded_bins: torch.Tensor,
    top_k: int,
) -> torch.Tensor:
    """Gather with padding (megablocks.ops.padded_gather interface).

    Returns [padded_bins[-1], hidden_size] with zeros in padding slots.
    """
    _lib.require_gpu(x)
    total_padded = int(padded_bins[-1].item())
    rs, _, _ = row_maps(indices, bin_ids, bins, padded_bins, top_k, total_padded, 0)
    return gather_rows(x, rs, top_k, total_padded)


@torch.compiler.disable
def _weighted_padded_gather(
    x: torch.Tensor,
    indices: torch.Tensor,
    bin_ids: torch.Tensor,
    weights: torch.Tensor,
    bins: torch.Tensor,
    padded_bins: torch.Tensor,
    top_k: int,
) -> torch.Tensor:
    """Gather with padding and weights: out[row(i)] = x[indices[i] // top_k] * weights[indices[i]]."""
    _lib.require_gpu(x)
    total_padded = int(padded_bins[-1].item())
    rs, _, _ = row_maps(indices, bin_ids, bins, padded_bins, top_k, total_padded, 0)
    return gather_rows(x, rs, top_k, total_padded, weights=weights)


class PaddedGatherOp(torch.autograd.Function):
    """Autograd function for padded_gather; backward is the unweighted combine."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x, indices, bin_ids, bins, padded_bins, top_k):
        _lib.require_gpu(x)
        total_padded = int(padded_bins[-1].item())
        num_tokens = x.shape[0]
        rs, _, ar = row_maps(indices, bin_ids, bins, padded_bins, top_k, total_padded,
                             num_tokens * top_k, want_assignment_row=True)
        ctx.save_for_backward(ar)
        ctx.top_k = top_k
        ctx.num_tokens = num_tokens
        return gather_rows(x, rs, top_k, total_padded)

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, grad_output):
        (ar,) = ctx.saved_tensors
        grad_x = combine_rows(grad_output, ar, ctx.top_k, ctx.num_tokens)
        return grad_x, None, None, None, None, None


def padded_gather_autograd(x, indices, bin_ids, bins, padded_bins, top_k):
    """Padded gather with autograd support."""
    return PaddedGatherOp.apply(x, indices, bin_ids, bins, padded_bins, top_k)
