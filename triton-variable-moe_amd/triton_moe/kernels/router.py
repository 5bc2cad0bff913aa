"""Router front end on the gfx950 router kernels (csrc/router.hip).

The reference computes, in TritonMoEMLP.forward (triton_moe/moe.py:166-182,
253-303), sigmoid -> torch.topk -> normalise -> bf16 for the routing, and
logsumexp / mean / matmul chains for the auxiliary losses: about thirty
PyTorch launches per step. Here one kernel does the routing and the
per-token reductions, and one single-workgroup kernel finishes the losses
after the routing counts exist. The losses are differentiable with respect
to the router logits (their gradient is one elementwise kernel); the top-k
weights are not, as in the reference (scatter.py:176), unless a caller opts
in through RouterWeightOp (TritonMoEConfig.routing_weight_grad).

Top-k: the expert ids come out in torch.topk's order on ROCm, ties
included, and the normalised weights carry the bits of the reference's
torch chain (the sum in torch's reduction order); both are held to PyTorch
on the same logits by the GPU tests.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.amp import custom_bwd, custom_fwd
from torch.autograd.function import once_differentiable

from .. import _lib


@dataclass
class RouterState:
    """Outputs of router_topk."""

    weights: torch.Tensor      # [T, k] in the logits' dtype (normalised when requested)
    selected: torch.Tensor     # [T, k] int32 or int64 expert ids
    probs: torch.Tensor | None  # [T, E] fp32 sigmoid(logits), when requested
    lse: torch.Tensor          # [T] fp32 logsumexp of each row (bf16-rounded for bf16 logits)
    partial: torch.Tensor      # per-workgroup sums for the auxiliary losses
    partial_rows: int
    # With route_hist: the routing workspace holding the per-tile expert
    # histograms of `selected` (route_device(..., workspace=) then skips its
    # counting launch); None when the top-k kernel did not count.
    route_ws: torch.Tensor | None = None


def router_topk(logits: torch.Tensor, top_k: int, normalize: bool = True,
                want_probs: bool = False, index_dtype=torch.int32,
                route_hist: bool = False) -> RouterState:
    """sigmoid + top-k + normalisation of bf16 or fp32 router logits [T, E]
    (no host sync); the weights come out in the logits' dtype, as the
    reference's .to(x.dtype) of them (moe.py:176).

    route_hist: where the shape allows it (vmoe_router_topk_hist), the same
    launch also writes the per-tile expert histograms the routing needs, into
    a routing workspace returned as RouterState.route_ws."""
    _lib.require_gpu(logits)
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError(f"router logits must be bfloat16 or float32 "
                                  f"(got {logits.dtype})")
    sfx = "_f32" if logits.dtype == torch.float32 else ""
    if logits.dim() != 2 or logits.stride(-1) != 1:
        logits = logits.reshape(-1, logits.shape[-1]).contiguous()
    T, E = logits.shape
    dev = logits.device
    L = _lib.lib()
    hist_rows = int(L.vmoe_router_topk_hist_blocks(T, E, int(top_k))) if route_hist else 0
    if hist_rows and (logits.stride(0) % 8 or logits.data_ptr() % 16):
        hist_rows = 0
    rows = hist_rows or int(L.vmoe_router_partial_floats(T, E)) // (E + 1)
    nfl = rows * (E + 1)
    f32 = torch.float32
    weights = torch.empty(T, top_k, dtype=logits.dtype, device=dev)
    selected = torch.empty(T, top_k, dtype=index_dtype, device=dev)
    probs = torch.empty(T, E, dtype=f32, device=dev) if want_probs else None
    # lse first, then the partial rows at a 16-byte aligned offset
    off = (T + 3) // 4 * 4
    scratch = torch.empty(off + nfl, dtype=f32, device=dev)
    lse, partial = scratch[:T], scratch[off:]
    is64 = index_dtype == torch.int64
    args = (logits.data_ptr(), logits.stride(0), T, E, int(top_k), int(bool(normalize)),
            weights.data_ptr(), None if is64 else selected.data_ptr(),
            selected.data_ptr() if is64 else None, _lib.ptr(probs), lse.data_ptr(),
            partial.data_ptr(), nfl, None)
    route_ws = None
    if hist_rows:
        ws_bytes = int(L.vmoe_route_counted_workspace_bytes(T, E, int(top_k)))
        route_ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.int32, device=dev)
        _lib.call("vmoe_router_topk_hist" + sfx, *args, route_ws.data_ptr(),
                  route_ws.numel() * 4, _lib.stream(dev))
    else:
        _lib.call("vmoe_router_topk" + sfx, *args, _lib.stream(dev))
    return RouterState(weights, selected, probs, lse, partial, rows, route_ws)


def router_logits_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Shapes and layouts vmoe_router_logits takes (bf16 on the GPU, E % 8 == 0,
    E <= 128, hidden % 256 == 0, contiguous 16-byte aligned rows)."""
    if not (x.is_cuda and weight.is_cuda and x.dtype == torch.bfloat16 and
            weight.dtype == torch.bfloat16 and x.dim() >= 1 and weight.dim() == 2):
        return False
    E, d = weight.shape
    return (x.shape[-1] == d and E % 8 == 0 and E <= 128 and d % 256 == 0 and
            weight.stride(1) == 1 and weight.stride(0) % 8 == 0 and
            weight.data_ptr() % 16 == 0)


class RouterLogitsOp(torch.autograd.Function):
    """logits = bf16(x @ W^T) on the router-logits kernel; the backward is the
    linear layer's (two bf16 matmuls with fp32 accumulation)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x2d, weight):
        T, d = x2d.shape
        E = weight.shape[0]
        if x2d.stride(1) != 1 or x2d.stride(0) % 8 != 0 or x2d.data_ptr() % 16 != 0:
            x2d = x2d.contiguous()
        out = torch.empty(T, E, dtype=torch.bfloat16, device=x2d.device)
        _lib.call("vmoe_router_logits", x2d.data_ptr(), x2d.stride(0), T, d, weight.data_ptr(),
                  weight.stride(0), E, out.data_ptr(), out.stride(0), _lib.stream(x2d.device))
        ctx.save_for_backward(x2d, weight)
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, g):
        x2d, weight = ctx.saved_tensors
        g = g.contiguous()
        gx = g @ weight if ctx.needs_input_grad[0] else None
        gw = g.t().contiguous() @ x2d if ctx.needs_input_grad[1] else None
        return gx, gw


class RouterLinear(nn.Linear):
    """The router of TritonMoEMLP: nn.Linear(n_embd, num_experts, bias=False)
    (moe.py:78 of the reference) -- same parameter, initialisation, state-dict
    key and hooks.

    Its forward is nn.Linear's own (F.linear, hipBLASLt on ROCm), so the
    logits carry the same bits as the reference module's on the same GPU and
    the routing decisions downstream (top-k of their sigmoid, which the
    router kernel reproduces bit for bit) are the reference's. With
    use_logits_kernel = True the inputs vmoe_router_logits supports go to that
    kernel instead: one bf16 rounding of the fp32 product, in its own
    summation order, which can move a logit by one bf16 step (about 0.02 %
    of them at the benchmark shapes) and with it a near-tied routing choice.
    """

    use_logits_kernel: bool = False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if (self.use_logits_kernel and self.bias is None and
                router_logits_supported(x, self.weight)):
            out = RouterLogitsOp.apply(x.reshape(-1, x.shape[-1]), self.weight)
            return out.reshape(*x.shape[:-1], out.shape[-1])
        return F.linear(x, self.weight, self.bias)


class RouterAuxOp(torch.autograd.Function):
    """(z_loss, load_balance_loss, compute_loss, f_i) from the router state and
    the routing counts; backward gives the router-logit gradient. z_loss, f_i
    and the gradient are in the logits' dtype (bf16 or fp32)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, logits, lse, partial, partial_rows, tokens_per_expert, coef, wn):
        T, E = logits.shape
        dev = logits.device
        dt = logits.dtype
        f_i = torch.empty(E, dtype=dt, device=dev)
        f32 = torch.empty(2 * E + 2, dtype=torch.float32, device=dev)
        f_i32, p_i, losses = f32[:E], f32[E:2 * E], f32[2 * E:]
        z = torch.empty((), dtype=dt, device=dev)
        tpe = tokens_per_expert.to(torch.int32).contiguous()
        sfx = "_f32" if dt == torch.float32 else ""
        _lib.call("vmoe_router_aux" + sfx, partial.data_ptr(), int(partial_rows), T, E,
                  tpe.data_ptr(), coef.data_ptr(), wn.data_ptr(), f_i.data_ptr(),
                  f_i32.data_ptr(), p_i.data_ptr(), z.data_ptr(), losses.data_ptr(),
                  _lib.stream(dev))
        ctx.save_for_backward(logits, lse, f_i32, coef, wn)
        ctx.mark_non_differentiable(f_i)
        return z, losses[0], losses[1], f_i

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, g_z, g_lb, g_cl, _g_fi):
        logits, lse, f_i32, coef, wn = ctx.saved_tensors
        T, E = logits.shape

        def scalar(g):
            return None if g is None else g.detach().to(torch.float32).reshape(()).contiguous()

        gz, glb, gcl = scalar(g_z), scalar(g_lb), scalar(g_cl)
        grad = torch.empty_like(logits)
        sfx = "_f32" if logits.dtype == torch.float32 else ""
        _lib.call("vmoe_router_aux_bwd" + sfx, logits.data_ptr(), logits.stride(0), T, E,
                  lse.data_ptr(), f_i32.data_ptr(), coef.data_ptr(), wn.data_ptr(),
                  _lib.ptr(gz), _lib.ptr(glb), _lib.ptr(gcl), grad.data_ptr(), grad.stride(0),
                  _lib.stream(logits.device))
        return grad, None, None, None, None, None, None


class RouterWeightOp(torch.autograd.Function):
    """The routing weights router_topk returned, as a differentiable function
    of the router logits (opt-in; the reference's weights get no gradient,
    scatter.py:176): backward is the chain of the reference's
    sigmoid -> topk -> normalise (moe.py:168-176) for the selected experts,
    0 for the others (vmoe_router_weight_bwd)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, logits, weights, selected, normalize):
        ctx.save_for_backward(logits, selected)
        ctx.normalize = bool(normalize)
        return weights.clone()

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, g_w):
        logits, selected = ctx.saved_tensors
        T, E = logits.shape
        k = selected.shape[-1]
        dt = logits.dtype
        g = g_w.reshape(T, k).to(dt).contiguous()
        sel = selected.reshape(T, k).contiguous()
        is64 = sel.dtype == torch.int64
        grad = torch.empty(T, E, dtype=dt, device=logits.device)
        sfx = "_f32" if dt == torch.float32 else ""
        _lib.call("vmoe_router_weight_bwd" + sfx, logits.data_ptr(), logits.stride(0), T, E, k,
                  int(ctx.normalize), None if is64 else sel.data_ptr(),
                  sel.data_ptr() if is64 else None, g.data_ptr(), g.stride(0), grad.data_ptr(),
                  grad.stride(0), _lib.stream(logits.device))
        return grad, None, None, None


def load_balance_coef(expert_sizes) -> list[float]:
    """Per-expert weights that turn the reference's three load-balance formulas
    (moe.py:276-303) into one dot product sum_e coef[e] f_i[e] p_i[e]:
    uniform widths -> E; no group with more than one expert -> 1; otherwise
    group_size / num_groups for experts of a group, 0 for lone experts."""
    widths = [w for c, w in expert_sizes for _ in range(c)]
    E = len(widths)
    if len(set(widths)) == 1:
        return [float(E)] * E
    groups = [c for c, _ in expert_sizes if c > 1]
    if not groups:
        return [1.0] * E
    coef = []
    for c, _w in expert_sizes:
        coef += [float(c) / len(groups) if c > 1 else 0.0] * c
    return coef
