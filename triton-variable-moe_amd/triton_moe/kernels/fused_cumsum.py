"""Routing on the gfx950 counting-sort kernels (csrc/route.hip).

Mirrors fused_route (triton_moe/kernels/fused_cumsum.py:85-171 of the
reference): same arguments, same five outputs, same errors. The reference runs
torch.sort + torch.bincount + a one-program cumsum kernel and, for token
dropping, a host loop with 2E syncs; here one HIP chain (a per-tile histogram,
then placement; a single-workgroup scan in between for more than 1024 experts
or 65,536 tile counts) produces the sorted arrays, histogram, both cumulative
sums, the padded-row maps and the gather map at once, and only "down"/"nearest"
rounding (whose output length is data dependent) reads anything back to the
host. The module's forward takes the histograms from its top-k launch
(router_topk(route_hist=True)) and runs the placement alone.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib


@dataclass
class Route:
    """Device-side routing state (no host sync needed to build it)."""

    bin_ids: torch.Tensor          # [A] int32, first n_kept valid
    indices: torch.Tensor          # [A] int32
    tokens_per_expert: torch.Tensor  # [E] int32 (raw counts)
    bins: torch.Tensor             # [E] int32
    padded_bins: torch.Tensor      # [E] int32
    row_src: torch.Tensor          # [rows_bound] int32, -1 = pad row
    gather_map: torch.Tensor       # [rows_bound] int32, map_pad (0 or -1) = pad row
    assignment_row: torch.Tensor   # [A] int32, -1 = dropped
    info: torch.Tensor             # [4] int32: rows P, kept, error bits
    expert_offsets: torch.Tensor   # [E+1] int32: [0, padded_bins]
    padded_counts: torch.Tensor    # [E] int32: diff(padded_bins)
    rows_bound: int                # host upper bound of P
    num_assignments: int
    num_experts: int
    top_k: int
    row_weight: torch.Tensor | None = None  # [rows_bound] fp32 routing weight, 0 = pad row


def rows_upper_bound(num_assignments: int, num_experts: int, block_size: int,
                     rounding: str = "up") -> int:
    """Largest possible padded row count P for any routing of A assignments."""
    if rounding == "down":
        return num_assignments
    if rounding == "nearest":
        return num_assignments + num_experts * (block_size // 2)
    return num_assignments + num_experts * (block_size - 1)


def route_device(selected: torch.Tensor, num_experts: int, top_k: int, block_size: int,
                 rounding: str = "up", map_pad: int = 0,
                 weights: torch.Tensor | None = None,
                 workspace: torch.Tensor | None = None) -> Route:
    """Runs the routing chain on the current stream; never syncs.

    map_pad is the gather_map entry of pad rows: 0 as in the reference's
    precompute_gather_map, -1 for the module's fused row gather (the GEMMs
    read zeros for it). With weights (bf16, one per assignment) the route
    also holds row_weight[row] = weights[row_src[row]] (0 on pad rows).
    workspace: the RouterState.route_ws of the router_topk(route_hist=True)
    call that produced `selected`; its per-tile histograms replace the
    routing's own counting launch (vmoe_route_counted)."""
    _lib.require_gpu(selected)
    if rounding not in _lib.ROUNDING:
        raise AssertionError(f"Invalid rounding mode: {rounding}")
    if num_experts > _lib.lib().vmoe_route_max_experts():
        raise NotImplementedError(
            f"num_experts={num_experts} exceeds the routing kernel's limit "
            f"{_lib.lib().vmoe_route_max_experts()}")
    sel = selected.reshape(-1)
    if sel.dtype not in (torch.int32, torch.int64):
        sel = sel.to(torch.int32)
    sel = sel.contiguous()
    dev = sel.device
    A = sel.numel()
    E = int(num_experts)
    cap = rows_upper_bound(A, E, block_size, rounding)
    ws_bytes = int(_lib.lib().vmoe_route_workspace_bytes(A, E))
    # One allocation carved into 16-byte aligned int32 views (one allocator
    # call per routing instead of twelve).
    if weights is not None:
        if weights.dtype != torch.bfloat16 or weights.numel() != A:
            raise ValueError("weights must be bf16 with one entry per assignment")
        weights = weights.reshape(-1).contiguous()
    nrw = max(cap, 1) if weights is not None else 0
    if workspace is not None:
        need = int(_lib.lib().vmoe_route_counted_workspace_bytes(A // int(top_k), E, int(top_k)))
        if (workspace.dtype != torch.int32 or need == 0 or A % int(top_k) or
                workspace.numel() * 4 < need or workspace.device != dev):
            raise ValueError("workspace must be the routing workspace of the "
                             "router_topk(route_hist=True) call that selected these experts")
    sizes = [max(A, 1), max(A, 1), E, E, E, max(cap, 1), max(cap, 1), max(A, 1), _lib.INFO_LEN,
             E + 1, E, nrw, 0 if workspace is not None else (ws_bytes + 3) // 4]
    offs, n = [], 0
    for sz in sizes:
        offs.append(n)
        n += (sz + 3) // 4 * 4
    buf = torch.empty(n, dtype=torch.int32, device=dev)
    (bin_ids, indices, tpe, bins, padded, row_src, gmap, arow, info, eto, ptpe, rw,
     ws) = (buf[o:o + sz] for o, sz in zip(offs, sizes))
    rw = rw.view(torch.float32) if weights is not None else None
    entry = "vmoe_route"
    if workspace is not None:
        entry, ws, ws_bytes = "vmoe_route_counted", workspace, workspace.numel() * 4
    _lib.call(entry, sel.data_ptr(), int(sel.dtype == torch.int64), A, E, int(top_k),
              int(block_size), _lib.ROUNDING[rounding], bin_ids.data_ptr(), indices.data_ptr(),
              tpe.data_ptr(), bins.data_ptr(), padded.data_ptr(), row_src.data_ptr(),
              gmap.data_ptr(), int(map_pad), cap, arow.data_ptr(), info.data_ptr(), eto.data_ptr(),
              ptpe.data_ptr(), _lib.ptr(weights), _lib.ptr(rw), ws.data_ptr(), ws_bytes,
              _lib.stream(dev))
    return Route(bin_ids[:A], indices[:A], tpe, bins, padded, row_src[:cap], gmap[:cap],
                 arow[:A], info, eto, ptpe, cap, A, E, int(top_k),
                 None if rw is None else rw[:cap])


def check_route(r: Route) -> tuple[int, int]:
    """Reads info back (one sync); raises on bad ids. Returns (P, n_kept)."""
    info = r.info.cpu().tolist()
    if info[_lib.INFO_ERRORS] & _lib.ROUTE_BAD_EXPERT_ID:
        raise RuntimeError("selected_experts holds expert ids outside [0, num_experts)")
    if info[_lib.INFO_ERRORS] & _lib.ROUTE_ROW_OVERFLOW:
        raise RuntimeError("padded row count exceeds the routing buffer")
    return info[_lib.INFO_ROWS], info[_lib.INFO_KEPT]


@torch.compiler.disable
def fused_route(
    selected_experts: torch.Tensor,
    num_experts: int,
    block_size: int = 128,
    rounding: str = "up",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Sort + histogram + rounded cumulative sums of expert assignments.

    Args:
        selected_experts: Expert assignments [num_tokens * top_k], int32/int64.
        num_experts: Number of experts.
        block_size: Block size for padding/rounding.
        rounding: "up" (dropless), "down" or "nearest" (token dropping).

    Returns:
        (bin_ids, indices, tokens_per_expert, bins, padded_bins) as in the
        reference: sorted expert ids and the stable permutation (first
        bins[-1] entries kept), the raw histogram, and the inclusive cumsums
        of kept and rounded counts. All int32.
    """
    if not selected_experts.is_cuda:
        raise AssertionError("Input must be on CUDA")
    if rounding not in ("up", "down", "nearest"):
        raise AssertionError(f"Invalid rounding mode: {rounding}")
    r = route_device(selected_experts, num_experts, 1, block_size, rounding)
    _, n_kept = check_route(r)
    return (r.bin_ids[:n_kept], r.indices[:n_kept], r.tokens_per_expert, r.bins,
            r.padded_bins)
