"""Eager per-expert-loop restatement of TritonMoEMLP (test infrastructure only).

Runs on the CPU in float32 (or float64 for pinning tests). Two numerics modes:

* mode="fp32": no intermediate rounding. This is the tolerance oracle the
  HIP path is held to with a normwise bf16 tolerance.
* mode="bf16": rounds to bf16 exactly at the points where the reference's
  kernels store bf16 (Appendix-A semantics of the reference):
    PRE = bf16(relu(z)), H = bf16(relu(z)^2) from the fp32 accumulator
        (triton_moe/kernels/grouped_gemm.py:336-346)
    Y = bf16(H @ W2)                       (grouped_gemm.py:575-583)
    combine slot = bf16(Y * w), fp32 sum over j, bf16 result
        (triton_moe/kernels/scatter.py:61-69, 133)
    GY = bf16(G * w)                       (triton_moe/kernels/gather.py:170-174)
    GH = bf16(GY @ W2^T), GW2 = bf16(H^T @ GY)   (grouped_gemm.py:1054-1063, 1153-1162)
    GA = bf16(PRE > 0 ? 2 * GH * PRE : 0)  (grouped_gemm.py:751-766, 914-928)
    GXg = bf16(GA @ W1^T), GW1 = bf16(Xg^T @ GA) (grouped_gemm.py:793-802, 947-967)
    Gx = bf16(sum_j GXg[row(t, j)])        (gather.py:256-263 via padded_scatter)
  The only remaining difference to a GPU run is fp32 summation order.
* mode="bf16w": the same products with the routing weight w of each row
  applied to H instead of to Y, the order the HIP module path rounds in
  (its up GEMM scales H, so the combine and the backward need no weighted
  copies of Y or of the output gradient G):
    H' = bf16(w * relu(z)^2), Y' = bf16(H' @ W2), out = bf16(sum_j Y'[row(t, j)])
    GH = bf16(w * (G[t] @ W2^T)), GW2 = bf16(H'^T @ G[t]); GA, GXg, GW1, Gx as above.
  In exact arithmetic all three modes agree: w (H @ W2) = (w H) @ W2 and
  H^T (w G) = (w H)^T G.

Routing weights get no gradient, as in the reference (scatter.py:176); the
opt-in routing-weight gradient of the weighted combine, which the reference
lacks, is combine_weight_grad below (pinned against torch autograd of combine),
and its chain into the router logits router_weight_logit_grad (float64
autograd of the reference's sigmoid / normalise, pinned by gradcheck).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import route as _route


def bf(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (torch's round-to-nearest-even) and back to t's dtype."""
    return t.to(torch.bfloat16).to(t.dtype)


def expert_layout(expert_sizes) -> tuple[list[int], list[int]]:
    """Per-expert widths and column offsets (triton_moe/moe.py:64-75)."""
    widths, offsets = [], [0]
    for count, size in expert_sizes:
        for _ in range(count):
            widths.append(int(size))
            offsets.append(offsets[-1] + int(size))
    return widths, offsets


@dataclass
class Problem:
    """One MoE-MLP invocation: flat tokens, weights, and the routing decision."""

    x: torch.Tensor          # [T, d]
    w1: torch.Tensor         # [d, W]
    w2: torch.Tensor         # [W, d]
    widths: list
    offsets: list
    selected: torch.Tensor   # [T, k] int64
    weights: torch.Tensor    # [T, k] (bf16 values, any float dtype)
    block_size: int = 64
    rounding: str = "up"

    @property
    def top_k(self) -> int:
        return self.selected.shape[1]

    @property
    def num_experts(self) -> int:
        return len(self.widths)


def route(prob: Problem) -> dict:
    """fused_route + row maps of a problem (numpy int32 arrays)."""
    r = _route.route(prob.selected.reshape(-1).numpy(), prob.num_experts, prob.block_size,
                     prob.rounding)
    maps = _route.row_maps(r["indices"], r["bin_ids"], r["bins"], r["padded_bins"], prob.top_k,
                           num_assignments=prob.selected.numel())
    r.update(maps)
    r["P"] = int(r["padded_bins"][-1]) if prob.num_experts else 0
    return r


def _rows(r: dict, e: int) -> tuple[int, int]:
    pb = r["padded_bins"]
    r0 = int(pb[e - 1]) if e > 0 else 0
    return r0, int(pb[e])


def _row_weights(prob: Problem, row_src: torch.Tensor, dt) -> torch.Tensor:
    """w[row] = weights[row_src[row]], 0 on pad rows (column vector)."""
    w_flat = prob.weights.to(dt).reshape(-1)
    valid = row_src >= 0
    rw = torch.zeros(row_src.numel(), dtype=dt)
    rw[valid] = w_flat[row_src[valid]]
    return rw[:, None]


def forward(prob: Problem, mode: str = "fp32", r: dict | None = None) -> dict:
    """Forward of the MoE MLP. Returns out [T, d] and the padded intermediates
    (in mode "bf16w", h and y are the row-weighted H' and Y')."""
    assert mode in ("fp32", "bf16", "bf16w")
    rb = bf if mode != "fp32" else (lambda t: t)
    dt = prob.x.dtype
    r = route(prob) if r is None else r
    T, d = prob.x.shape
    k = prob.top_k
    P = r["P"]
    max_w = max(prob.widths)
    row_src = torch.from_numpy(r["row_src"].astype(np.int64))
    valid = row_src >= 0
    xg = torch.zeros(P, d, dtype=dt)
    xg[valid] = prob.x[row_src[valid] // k]
    rw = _row_weights(prob, row_src, dt) if mode == "bf16w" else None
    z = torch.zeros(P, max_w, dtype=dt)
    pre = torch.zeros(P, max_w, dtype=dt)
    h = torch.zeros(P, max_w, dtype=dt)
    y = torch.zeros(P, d, dtype=dt)
    for e, (w, o) in enumerate(zip(prob.widths, prob.offsets)):
        r0, r1 = _rows(r, e)
        if r1 == r0:
            continue
        ze = xg[r0:r1] @ prob.w1[:, o:o + w]
        z[r0:r1, :w] = ze
        relu = torch.clamp_min(ze, 0)
        pre[r0:r1, :w] = rb(relu)
        h[r0:r1, :w] = rb(relu * relu if rw is None else rw[r0:r1] * (relu * relu))
        y[r0:r1] = rb(h[r0:r1, :w] @ prob.w2[o:o + w])
    wc = None if mode == "bf16w" else prob.weights.to(dt).reshape(-1)
    out = combine(y, r["assignment_row"], wc, k, T, mode)
    return {"out": out, "x_gathered": xg, "z": z, "pre_act": pre, "h": h, "y": y, "route": r}


def combine(y: torch.Tensor, assignment_row, weights_flat, k: int, T: int,
            mode: str) -> torch.Tensor:
    """out[t] = sum_j slot(t, j), slot = y[row] * w (rounded to bf16 in bf16 mode),
    summed in fp32 in ascending j (scatter.py:61-69, 133)."""
    rb = bf if mode != "fp32" else (lambda t: t)
    ar = torch.as_tensor(np.asarray(assignment_row, np.int64)).view(T, k)
    out = torch.zeros(T, y.shape[1], dtype=y.dtype)
    for j in range(k):
        rows = ar[:, j]
        ok = rows >= 0
        slot = torch.zeros_like(out)
        if weights_flat is None:
            slot[ok] = y[rows[ok]]
        else:
            wj = weights_flat.view(T, k)[:, j]
            slot[ok] = rb(y[rows[ok]] * wj[ok, None])
        out = out + slot
    return rb(out)


def swiglu_up(xg: torch.Tensor, w1: torch.Tensor, rows, widths, offsets,
              max_w: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(H, gate) of the grouped up projection with swiglu, unrounded, per-expert
    loop: gate = X_e W1[:, o_e : o_e + w_e], up = X_e W1[:, o_e + w_e : o_e + 2 w_e],
    H = silu(gate) * up (reference grouped_gemm.py:295-297, 323-330, 347-349).
    Differentiable (torch autograd gives the backward the reference leaves
    unfinished, grouped_gemm.py:768-790)."""
    P = xg.shape[0]
    h = torch.zeros(P, max_w, dtype=xg.dtype)
    gate = torch.zeros(P, max_w, dtype=xg.dtype)
    hs, gs = [], []
    for e, (r0, r1) in enumerate(rows):
        w, o = widths[e], offsets[e]
        g = xg[r0:r1] @ w1[:, o:o + w]
        u = xg[r0:r1] @ w1[:, o + w:o + 2 * w]
        hs.append((e, r0, r1, w, g * torch.sigmoid(g) * u))
        gs.append(g)
    for (e, r0, r1, w, he), g in zip(hs, gs):
        h = h.index_put((torch.arange(r0, r1)[:, None], torch.arange(w)[None, :]), he)
        gate = gate.index_put((torch.arange(r0, r1)[:, None], torch.arange(w)[None, :]), g)
    return h, gate


def combine_weight_grad(grad: torch.Tensor, y: torch.Tensor, assignment_row, k: int,
                        T: int) -> torch.Tensor:
    """d(sum out * grad)/dw of combine in fp32 mode: gw[t*k+j] = sum_c grad[t, c] *
    y[row(t, j), c], 0 for slots with row < 0; float64 accumulation.
    The reference has no such gradient (scatter.py:176 returns None)."""
    ar = torch.as_tensor(np.asarray(assignment_row, np.int64)).view(T, k)
    g64, y64 = grad.double(), y.double()
    gw = torch.zeros(T, k, dtype=torch.float64)
    for j in range(k):
        rows = ar[:, j]
        ok = rows >= 0
        gw[ok, j] = (g64[ok] * y64[rows[ok]]).sum(dim=1)
    return gw.reshape(-1)


def backward(prob: Problem, fwd: dict, grad_out: torch.Tensor, mode: str = "fp32") -> dict:
    """Gradients of the forward above for upstream grad_out [T, d] (fwd from
    forward() in the same mode)."""
    assert mode in ("fp32", "bf16", "bf16w")
    rb = bf if mode != "fp32" else (lambda t: t)
    r = fwd["route"]
    dt = prob.x.dtype
    T, d = prob.x.shape
    k = prob.top_k
    P = r["P"]
    max_w = max(prob.widths)
    g = grad_out.to(dt)
    w_flat = prob.weights.to(dt).reshape(-1)
    row_src = torch.from_numpy(r["row_src"].astype(np.int64))
    valid = row_src >= 0
    gy = torch.zeros(P, d, dtype=dt)
    rw = None
    if mode == "bf16w":
        gy[valid] = g[row_src[valid] // k]  # G[t], the weight goes on GH
        rw = _row_weights(prob, row_src, dt)
    else:
        gy[valid] = rb(g[row_src[valid] // k] * w_flat[row_src[valid], None])
    gh = torch.zeros(P, max_w, dtype=dt)
    ga = torch.zeros(P, max_w, dtype=dt)
    gxg = torch.zeros(P, d, dtype=dt)
    gw1 = torch.zeros_like(prob.w1, dtype=dt)
    gw2 = torch.zeros_like(prob.w2, dtype=dt)
    for e, (w, o) in enumerate(zip(prob.widths, prob.offsets)):
        r0, r1 = _rows(r, e)
        if r1 == r0:
            continue
        ghe = gy[r0:r1] @ prob.w2[o:o + w].T
        ghe = rb(ghe if rw is None else rw[r0:r1] * ghe)
        gh[r0:r1, :w] = ghe
        gw2[o:o + w] = rb(fwd["h"][r0:r1, :w].T @ gy[r0:r1])
        pre = fwd["pre_act"][r0:r1, :w]
        gae = rb(torch.where(pre > 0, ghe * 2.0 * pre, torch.zeros_like(pre)))
        ga[r0:r1, :w] = gae
        gxg[r0:r1] = rb(gae @ prob.w1[:, o:o + w].T)
        gw1[:, o:o + w] = rb(fwd["x_gathered"][r0:r1].T @ gae)
    gx = combine(gxg, r["assignment_row"], None, k, T, mode)
    return {"grad_x": gx, "grad_w1": gw1, "grad_w2": gw2, "grad_y": gy, "grad_h": gh,
            "grad_a": ga, "grad_xg": gxg}


def router_weights(logits: torch.Tensor, selected: torch.Tensor,
                   normalize: bool = True) -> torch.Tensor:
    """The reference's routing weights for a given selection (moe.py:168-176):
    v = sigmoid(L)[selected], normalised by (sum v + 1e-20); unrounded and
    differentiable in L (the selection itself is piecewise constant)."""
    v = torch.sigmoid(logits).gather(1, selected.long())
    if normalize:
        v = v / (v.sum(dim=-1, keepdim=True) + 1e-20)
    return v


def router_weight_logit_grad(logits: torch.Tensor, selected: torch.Tensor,
                             grad_weights: torch.Tensor, normalize: bool = True) -> torch.Tensor:
    """dL/dlogits of sum(router_weights(logits) * grad_weights), float64 torch
    autograd. The reference computes no such gradient (scatter.py:176); this
    is the opt-in routing-weight gradient's chain into the router."""
    L = logits.detach().to(torch.float64).requires_grad_(True)
    v = router_weights(L, selected, normalize)
    (v * grad_weights.detach().to(torch.float64).reshape(v.shape)).sum().backward()
    return L.grad


def aux_losses(router_logits: torch.Tensor, tokens_per_expert, widths, expert_sizes,
               dtype=torch.bfloat16) -> dict:
    """Auxiliary losses of TritonMoEMLP.forward (triton_moe/moe.py:253-303), in float64."""
    L = router_logits.to(torch.float64)
    probs = torch.sigmoid(L)
    E = len(widths)
    z_loss = torch.logsumexp(L, dim=-1).pow(2).mean()
    tpe = torch.as_tensor(np.asarray(tokens_per_expert), dtype=torch.float64)
    f_i = (tpe / tpe.sum()).to(dtype)
    p_i = probs.mean(dim=0)
    fi = f_i.to(torch.float64)
    if len(set(widths)) == 1:
        lb = E * (fi @ p_i)
    else:
        groups = []
        e = 0
        for count, _ in expert_sizes:
            if count > 1:
                groups.append(list(range(e, e + count)))
            e += count
        if not groups:
            lb = fi @ p_i
        else:
            fp = fi * p_i
            lb = torch.stack([len(gr) * fp[gr].sum() for gr in groups]).mean()
    mean_w = sum(widths) / E
    wn = torch.tensor([w / mean_w for w in widths], dtype=torch.float32).to(dtype)
    compute = (probs @ wn.to(torch.float64)).mean()
    return {"router_z_loss": z_loss, "load_balance_loss": lb, "compute_loss": compute, "f_i": f_i}
