#!/usr/bin/env python
"""Benchmark of the MoE MLP hot path on one MI355X.

Workload: BASELINE.json config 3 -- TritonMoEMLP with n_embd=1024,
expert_sizes=[(64, 256)], top_k=8, 16384 tokens, block_size 64, bf16, router
logits biased by a Zipf(s=1.2) rank profile (alpha = smallest integer giving an
empty expert and a hottest expert above 4x the mean). Synthetic data: one CPU
torch.Generator(0) draws x ~ N(0,1), then router, w1, w2 ~ N(0, 0.02).

A step is one forward + out.sum().backward() of the layer (router, routing,
token gather (fused into the up GEMM's operand staging), grouped GEMM up +
relu^2, grouped GEMM down, weighted combine and the full backward including
both dW GEMMs).

Prints one JSON line: value = grouped-GEMM TFLOP/s of the whole step
(12 * d * sum_e n_e * w_e over the step's wall time), plus ms_per_step, the
per-kernel breakdown (HIP events around each launch inside real steps, on the
launch stream), the roofline of the
dominant kernel and the CPU baseline (the fp32 eager per-expert-loop oracle on
the host cores).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "triton-variable-moe_amd"))

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
# The box's measured device copy rate (read + write, 1 GiB, torch copy_;
# bench.py --ceiling, profiles/practical_ceiling.md): the practical ceiling of
# a row-copy kernel such as the combine.
COPY_GBS = 5260.0

CONFIGS = {
    # name: (n_embd, expert_sizes, top_k, tokens, zipf)
    "cfg1": (768, [(8, 512)], 2, 8 * 1024, False),
    "cfg2": (768, [(4, 512), (8, 256), (4, 128)], 2, 8 * 2048, False),
    "cfg3": (1024, [(64, 256)], 8, 16384, True),
    "cfg4": (2048, [(32, 1024), (64, 512), (32, 256)], 8, 32768, False),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="cfg3", choices=sorted(CONFIGS))
    ap.add_argument("--kernel-steps", type=int, default=10,
                    help="steps run with a HIP event pair around every launch (per-kernel times)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-iters", type=int, default=3)
    ap.add_argument("--profile-steps", type=int, default=0,
                    help="only run this many steps (for rocprofv3), print nothing else")
    ap.add_argument("--ceiling", action="store_true",
                    help="only measure the box's practical ceilings: dense bf16 torch.matmul "
                         "(hipBLASLt) at square and MoE-like shapes, and device copy / fill "
                         "bandwidth")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip timing the step replayed from a HIP graph (graph_ms_per_step)")
    ap.add_argument("--other-configs", default="cfg1,cfg2,cfg4",
                    help="comma-separated configurations also measured (fewer steps) and "
                         "reported under other_configs; empty to skip")
    ap.add_argument("--fp32-gemm", action="store_true",
                    help="only time the fp32 grouped GEMMs (float32 weights on the public API) "
                         "at cfg3's shapes with balanced routing")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy a 1 GiB device buffer 5 times: the known-size kernel that "
                         "scales the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--host-profile", action="store_true",
                    help="only measure where the host time of an eager step of --config goes: "
                         "issue and completion rates, the library calls' host time, and "
                         "torch.profiler's CPU table over the steps")
    return ap.parse_args()


# Kernel symbol of each GEMM op (grouped_gemm_kernel<Variant>).
GEMM_SYMBOL = {
    "gemm_up_fwd": "grouped_gemm_kernel<0>",
    "gemm_down_fwd": "grouped_gemm_kernel<1>",
    "gemm_up_bwd_dx": "grouped_gemm_kernel<2>",
    "gemm_up_bwd_dw": "grouped_gemm_kernel<3>",
    "gemm_down_bwd_dh_ga": "grouped_gemm_kernel<4>",
    "gemm_down_bwd_dw": "grouped_gemm_kernel<5>",
}


def gemm_bytes(op, A, T, d, nw, W):
    """Minimal unique HBM bytes of one GEMM launch (bf16): its operands read
    once and its outputs written once. A = routed rows, T = tokens (the up
    GEMM and its dW read the token rows x, the dH and dW2 GEMMs the token
    gradient G, through the row map), nw = sum_e n_e w_e, W = total expert
    width. G counts as T rows (a real upstream gradient; the bench's
    out.sum() gradient is one broadcast row)."""
    rows_d, tok_d, inter, weights = 2 * A * d, 2 * T * d, 2 * nw, 2 * d * W
    return {
        "gemm_up_fwd": tok_d + weights + 2 * inter,           # x[gm], W1 -> H', PRE
        "gemm_down_fwd": inter + weights + rows_d,            # H', W2 -> Y'
        "gemm_down_bwd_dh_ga": tok_d + weights + 2 * inter,   # G[gm], W2, PRE -> GA
        "gemm_up_bwd_dx": inter + weights + rows_d,           # GA, W1 -> GXg
        "gemm_up_bwd_dw": tok_d + inter + weights,            # x[gm], GA -> GW1
        "gemm_down_bwd_dw": inter + tok_d + weights,          # H', G[gm] -> GW2
    }[op]


def measured_traffic(config, symbol):
    """HBM bytes per launch of `symbol` from the committed rocprofv3 counter
    summary (profiles/hbm_traffic_<config>.json), or None."""
    path = REPO / "profiles" / f"hbm_traffic_{config}.json"
    try:
        data = json.loads(path.read_text())
        k = data["kernels"][symbol]
        return int(k["fetch_bytes"] + k["write_bytes"])
    except (OSError, KeyError, ValueError, TypeError):
        return None


def ceiling():
    """Practical ceilings of this GPU: dense bf16 GEMMs through torch.matmul
    (hipBLASLt) on random and on all-zero operands (the power draw of random
    data lowers the clock), at square sizes and at the dense equivalents of
    cfg3's GEMMs (rows = T k, the expert dimension folded), and copy / fill
    bandwidth of a 1 GiB buffer."""
    import torch

    dev = torch.device("cuda:0")

    def timed(fn, iters):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters * 1e-3

    out = {"gemm_tflops": {}, "bandwidth_tbs": {}}
    g = torch.Generator(device=dev).manual_seed(0)
    for M, N, K, zero, ta in [(8192, 8192, 8192, False, False), (8192, 8192, 8192, True, False),
                              (16384, 16384, 16384, False, False),
                              (131072, 256, 1024, False, False), (131072, 1024, 256, False, False),
                              (1024, 256, 131072, False, True)]:
        a = (torch.randn(K, M, device=dev, dtype=torch.bfloat16, generator=g).t() if ta else
             torch.randn(M, K, device=dev, dtype=torch.bfloat16, generator=g))
        b = torch.randn(K, N, device=dev, dtype=torch.bfloat16, generator=g)
        if zero:
            a.zero_()
            b.zero_()
        sec = timed(lambda: a @ b, 20 if M * N * K < 2 ** 40 else 5)
        key = f"{M}x{N}x{K}" + ("_zeros" if zero else "") + ("_At" if ta else "")
        out["gemm_tflops"][key] = round(2.0 * M * N * K / sec / 1e12, 1)
        del a, b
    n = 1 << 30
    x = torch.empty(n, dtype=torch.uint8, device=dev)
    y = torch.empty_like(x)
    out["bandwidth_tbs"]["copy_read_plus_write"] = round(2 * n / timed(lambda: y.copy_(x), 20) / 1e12, 2)
    out["bandwidth_tbs"]["fill_write"] = round(n / timed(lambda: y.fill_(1), 20) / 1e12, 2)
    print(json.dumps({"ceiling": out, "device": torch.cuda.get_device_name(0)}))


def fp32_gemm():
    """The fp32 grouped GEMMs (csrc/gemm_f32.hip) at cfg3's shapes: 64 experts
    of width 256, n_embd 1024, 16384 tokens x top-8 routed evenly (2048 rows
    per expert), through the public functions (each call includes its output's
    zero fill). Rates are against the 157.3 TFLOP/s dense fp32 peak."""
    import torch

    from triton_moe.kernels import (grouped_gemm_down, grouped_gemm_down_backward,
                                    grouped_gemm_up, grouped_gemm_up_backward)

    dev = torch.device("cuda:0")
    d, sizes, k, T, _ = CONFIGS["cfg3"]
    E, w = sizes[0]
    rows = T * k // E
    P = rows * E
    g = torch.Generator(device=dev).manual_seed(0)
    eto = torch.arange(0, P + 1, rows, dtype=torch.int32, device=dev)
    ewo = torch.arange(0, E * w + 1, w, dtype=torch.int32, device=dev)
    wid = torch.full((E,), w, dtype=torch.int32, device=dev)
    tpe = torch.full((E,), rows, dtype=torch.int32, device=dev)
    x = torch.randn(P, d, device=dev, generator=g)
    w1 = torch.randn(d, E * w, device=dev, generator=g) * 0.03
    w2 = torch.randn(E * w, d, device=dev, generator=g) * 0.03
    gy = torch.randn(P, d, device=dev, generator=g)
    h, pre = grouped_gemm_up(x, w1, eto, ewo, wid, tpe, w, save_pre_act=True)
    gh, _ = grouped_gemm_down_backward(gy, h, w2, eto, ewo, wid, tpe, d, w)
    calls = {
        "up_fwd": (1, lambda: grouped_gemm_up(x, w1, eto, ewo, wid, tpe, w, save_pre_act=True)),
        "down_fwd": (1, lambda: grouped_gemm_down(h, w2, eto, ewo, wid, tpe, d)),
        "down_bwd_dh_dw": (2, lambda: grouped_gemm_down_backward(gy, h, w2, eto, ewo, wid, tpe,
                                                                  d, w)),
        "up_bwd_dx_dw": (2, lambda: grouped_gemm_up_backward(gh, x, w1, pre, eto, ewo, wid, tpe,
                                                              d)),
    }
    flops = 2.0 * P * d * w
    out = {}
    for name, (n, fn) in calls.items():
        fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / 5 * 1e3
        out[name] = {"us": round(us, 1), "tflops": round(n * flops / (us * 1e-6) / 1e12, 2)}
    total_us = sum(v["us"] for v in out.values())
    print(json.dumps({"fp32_gemm": out, "gemm_flops_each": flops,
                      "step_tflops": round(6 * flops / (total_us * 1e-6) / 1e12, 2),
                      "peak_tflops_fp32": 157.3,
                      "shape": f"cfg3 balanced: P={P}, d={d}, E={E}, w={w}"}))


def copy_calibration():
    import torch

    n = 1 << 30
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 5}))


def build_workload(name, device):
    import numpy as np
    import torch

    from triton_moe import TritonMoEConfig, TritonMoEMLP

    d, sizes, k, T, zipf = CONFIGS[name]
    E = sum(c for c, _ in sizes)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, T, d, generator=g)
    wr = torch.randn(E, d, generator=g) * 0.02
    cfg = TritonMoEConfig(n_embd=d, expert_sizes=sizes, num_active_experts=k, block_size=64)
    m = TritonMoEMLP(cfg)
    W = m.total_expert_width
    w1 = torch.randn(d, W, generator=g) * 0.02
    w2 = torch.randn(W, d, generator=g) * 0.02
    with torch.no_grad():
        m.router.weight.copy_(wr)
        m.w1.copy_(w1)
        m.w2.copy_(w2)
    m = m.to(device).to(torch.bfloat16)
    xb = x.to(torch.bfloat16).to(device)
    info = {"alpha": None}
    if zipf:
        ranks = np.random.default_rng(0).permutation(E) + 1
        base = torch.tensor(-1.2 * np.log(ranks), dtype=torch.float32, device=device)
        state = {"bias": None}
        # the bias is held in the logits' dtype (bf16), converted once per alpha
        m.router.register_forward_hook(
            lambda mod, inp, out: out if state["bias"] is None else out + state["bias"])
        with torch.no_grad():
            for alpha in range(1, 20):
                state["bias"] = (alpha * base).to(torch.bfloat16)
                _, _, f_i = m(xb)
                logits = m.router(xb.reshape(-1, d))
                sel = torch.topk(torch.sigmoid(logits.float()), k, dim=-1).indices
                hist = torch.bincount(sel.reshape(-1), minlength=E)
                if hist.min().item() == 0 and hist.max().item() > 4 * hist.float().mean().item():
                    info["alpha"] = alpha
                    break
        info["histogram"] = hist.tolist()
    xb.requires_grad_(True)
    return m, xb, info


def gemm_flops(m, xb):
    import torch

    with torch.no_grad():
        d = xb.shape[-1]
        logits = m.router(xb.reshape(-1, d))
        sel = torch.topk(torch.sigmoid(logits.float()), m.num_active_experts, dim=-1).indices
        counts = torch.bincount(sel.reshape(-1), minlength=m.num_experts).cpu().tolist()
    snw = sum(n * w for n, w in zip(counts, m.expert_widths))
    return 12.0 * d * snw, counts, sel


def make_step(m, xb):
    """One training step of the layer: forward, loss out.sum(), backward."""

    def step():
        m.zero_grad(set_to_none=True)
        xb.grad = None
        out, _, _ = m(xb)
        out.sum().backward()

    return step


def time_graph_steps(m, xb, steps, warmup):
    """The same step captured once into a HIP graph (torch.cuda.graph) and
    replayed: forward and backward of out.sum()'s gradient (a broadcast row
    of ones, passed directly, so that no reduction kernel with a memset node
    sits in the graph); gradients are re-created inside the capture
    (zero_grad(set_to_none=True)), as the eager step does. Every launch of the
    eager step except the loss reduction and its fills is replayed; the host's
    per-launch work is gone."""
    import torch

    T, d = xb.shape[1], xb.shape[2]
    gout = torch.ones(1, 1, d, dtype=xb.dtype, device=xb.device).expand(xb.shape)

    def step():
        m.zero_grad(set_to_none=True)
        xb.grad = None
        out, _, _ = m(xb)
        out.backward(gout)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    del g
    return ms


def time_steps(m, xb, steps, warmup):
    import torch

    step = make_step(m, xb)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


# Entry point -> op name of the per-kernel breakdown; the combine runs twice
# per step (forward, then the backward gather of dX).
OP_OF = {
    "vmoe_router_logits": ("router_logits",),
    "vmoe_router_topk": ("router_topk",),
    "vmoe_router_topk_hist": ("router_topk",),
    "vmoe_route": ("route",),
    "vmoe_route_counted": ("route",),
    "vmoe_gemm_up_fwd": ("gemm_up_fwd",),
    "vmoe_gemm_down_fwd": ("gemm_down_fwd",),
    "vmoe_combine": ("combine", "gather_bwd_combine"),
    "vmoe_router_aux": ("router_aux",),
    "vmoe_gemm_down_bwd_dh": ("gemm_down_bwd_dh_ga",),
    "vmoe_gemm_up_bwd_dw": ("gemm_up_bwd_dw",),
    "vmoe_gemm_up_bwd_dx": ("gemm_up_bwd_dx",),
    "vmoe_gemm_down_bwd_dw": ("gemm_down_bwd_dw",),
}


class LaunchTimer:
    """A HIP event pair around every C-ABI launch of a step, bound to the
    launched kernels' own dispatches (vmoe_set_launch_timing), so each kernel
    is timed where it runs in the real step (after the kernels that precede
    it, with their caches and write-backs), not in a loop of its own, and
    without the gaps that event records between the kernels would add."""

    def __init__(self):
        import torch

        self.torch = torch
        self.marks = []
        self.seen = {}
        self.open = None

    def new_step(self):
        self.seen = {}

    def begin(self, name):
        from triton_moe import _lib

        e0 = self.torch.cuda.Event(enable_timing=True)
        e1 = self.torch.cuda.Event(enable_timing=True)
        # recorded once so that the events exist; the entry point's kernels
        # then record them again on their own dispatch (vmoe_set_launch_timing:
        # start of the first kernel, end of the last), so the pair times the
        # kernels and not the event records around them
        e0.record()
        e1.record()
        _lib.lib().vmoe_set_launch_timing(e0.cuda_event, e1.cuda_event)
        self.open = (e0, e1)

    def end(self, name):
        from triton_moe import _lib

        _lib.lib().vmoe_set_launch_timing(None, None)
        e0, e1 = self.open
        n = self.seen.get(name, 0)
        self.seen[name] = n + 1
        ops = OP_OF.get(name, (name,))
        self.marks.append((ops[min(n, len(ops) - 1)], e0, e1))


def kernel_breakdown(m, xb, steps):
    """Average duration (us) of each launch of the step, from HIP events
    around the launches of `steps` real steps (the timed steps run without
    the events)."""
    import torch

    from triton_moe import _lib

    from triton_moe.kernels import grouped_gemm as gg

    step = make_step(m, xb)
    step()
    timer = LaunchTimer()
    _lib.set_launch_timer(timer)
    # one stream, so that no two timed launches overlap (the timed steps
    # run the weight-gradient GEMMs beside the others on a second stream)
    side = gg.BACKWARD_SIDE_STREAM
    gg.BACKWARD_SIDE_STREAM = False
    try:
        # A bounded spin kernel (torch.cuda._sleep) holds the GPU while the
        # host queues every timed step, so the launches then run back to
        # back: an event pair around a launch the host has not yet queued
        # would also time the host's launch latency (small configurations
        # are host-bound otherwise).
        torch.cuda.synchronize()
        torch.cuda._sleep(int(3e6) * steps)
        for _ in range(steps):
            timer.new_step()
            step()
    finally:
        _lib.set_launch_timer(None)
        gg.BACKWARD_SIDE_STREAM = side
    torch.cuda.synchronize()
    tot, cnt = {}, {}
    for op, e0, e1 in timer.marks:
        tot[op] = tot.get(op, 0.0) + e0.elapsed_time(e1) * 1e3
        cnt[op] = cnt.get(op, 0) + 1
    return {op: tot[op] / cnt[op] for op in tot}


def cpu_baseline(m, xb, sel, iters):
    """fp32 eager per-expert-loop oracle (forward + backward) on the host."""
    import torch

    from oracle import eager

    d = xb.shape[-1]
    x = xb.detach().reshape(-1, d).float().cpu()
    k = m.num_active_experts
    with torch.no_grad():
        logits = m.router(xb.detach().reshape(-1, d))
        wts, sel2 = torch.topk(torch.sigmoid(logits.float()), k, dim=-1)
        wts = (wts / (wts.sum(-1, keepdim=True) + 1e-20)).to(torch.bfloat16)
    prob = eager.Problem(x, m.w1.detach().float().cpu(), m.w2.detach().float().cpu(),
                         m.expert_widths, m.expert_offsets, sel2.cpu(), wts.cpu().float(),
                         m.block_size)
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    G = torch.ones(x.shape[0], d)

    def run():
        f = eager.forward(prob, "fp32")
        eager.backward(prob, f, G, "fp32")

    run()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], torch.get_num_threads()


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def measure(name, device, steps, warmup, kernel_steps, graph):
    """Times one configuration: eager steps (and HIP-graph replays when
    `graph`), then the per-launch breakdown. Returns the figures and the
    workload (model, input, routing) for the CPU baseline."""
    import torch

    torch.manual_seed(0)
    m, xb, info = build_workload(name, device)
    flops, counts, sel = gemm_flops(m, xb)
    ms = time_steps(m, xb, steps, warmup)
    graph_ms = time_graph_steps(m, xb, steps, warmup) if graph else None
    kern = kernel_breakdown(m, xb, kernel_steps)
    gemm_names = [n for n in kern if n.startswith("gemm_")]
    gemm_us = sum(kern[n] for n in gemm_names)
    gemm_tflops = flops / (gemm_us * 1e-6) / 1e12
    dom = max(gemm_names, key=lambda n: kern[n])
    achieved = flops / 6.0 / (kern[dom] * 1e-6) / 1e12

    d, sizes, k, T, _ = CONFIGS[name]
    A = T * k
    E = m.num_experts
    widths = [w for c, w in sizes for _ in range(c)]
    nw = sum(int(n) * w for n, w in zip(counts, widths))
    # Permutation and routing bytes: each combine reads the k rows of every
    # token and the row of each assignment and writes the token rows; the
    # routing reads the ids (int32) and bf16 weights and writes bin_ids,
    # indices and assignment_row per assignment and row_src, gather_map and
    # the fp32 row weight per padded row (+ five E-long arrays).
    P = sum(-(-int(n) // 64) * 64 for n in counts)
    perm_bytes = {
        "combine": 2 * A * d + 2 * T * d + 4 * A,
        "gather_bwd_combine": 2 * A * d + 2 * T * d + 4 * A,
        "route": 6 * A + 12 * A + 12 * P + 20 * E,
    }
    perm_us = sum(kern[n] for n in perm_bytes)
    perm_gbs = sum(perm_bytes.values()) / (perm_us * 1e-6) / 1e9
    return {
        "m": m, "xb": xb, "sel": sel, "info": info, "counts": counts, "flops": flops,
        "ms": ms, "graph_ms": graph_ms, "kern": kern, "gemm_tflops": gemm_tflops,
        "dom": dom, "achieved": achieved, "A": A, "T": T, "d": d, "nw": nw,
        "W": sum(widths), "perm_gbs": perm_gbs, "perm_us": perm_us,
    }


def summary(name, r):
    """The compact record of a configuration in `other_configs`."""
    d, sizes, k, T, _ = CONFIGS[name]
    return {
        "workload": f"n_embd={d}, expert_sizes={sizes}, top_k={k}, tokens={T}, block_size=64",
        "ms_per_step": round(r["ms"], 4),
        "graph_ms_per_step": None if r["graph_ms"] is None else round(r["graph_ms"], 4),
        "eager_over_graph": None if r["graph_ms"] is None else round(r["ms"] / r["graph_ms"], 3),
        "value_tflops": round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 2),
        "gemm_tflops_kernel_time": round(r["gemm_tflops"], 2),
        "gemm_pct_mfma_peak": round(100 * r["gemm_tflops"] / PEAK_BF16_TFLOPS, 2),
        "permutation_pct_hbm_peak": round(100 * r["perm_gbs"] / PEAK_HBM_GBS, 2),
        "tokens_per_expert_min_max": [min(r["counts"]), max(r["counts"])],
        "kernel_us": {n: round(v, 2) for n, v in r["kern"].items()},
    }


def host_profile(name, device, steps):
    """Host side of the eager step of `name`: how fast the host issues steps
    (timed before the final synchronize) against how fast they complete, the
    host time inside the two library calls of the layer (vmoe_moe_forward /
    vmoe_moe_backward, bound ctypes functions timed around the call), and
    torch.profiler's CPU-only table over the same steps (self time per op, the
    autograd device thread included). Prints text, not a bench line."""
    import torch
    from torch.profiler import ProfilerActivity, profile

    from triton_moe.kernels import grouped_gemm as gg

    torch.manual_seed(0)
    m, xb, _info = build_workload(name, device)
    step = make_step(m, xb)
    for _ in range(20):
        step()
    torch.cuda.synchronize()
    print(f"# host profile, {name}, {steps} eager steps per measurement")
    for n in (20, steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            step()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        print(f"steps {n}: host issue {1e6 * (t1 - t0) / n:.1f} us/step, completion "
              f"{1e6 * (t2 - t0) / n:.1f} us/step")
    # host time inside the layer's two library calls
    acc = {}

    def timed(fn, what):
        def call(*a):
            t = time.perf_counter()
            r = fn(*a)
            acc.setdefault(what, []).append(time.perf_counter() - t)
            return r
        return call

    plans = dict(gg._MOE_PLANS)
    for key, plan in plans.items():
        gg._MOE_PLANS[key] = plan[:7] + (timed(plan[7], "vmoe_moe_forward"),
                                         timed(plan[8], "vmoe_moe_backward"))
    try:
        for _ in range(steps):
            torch.cuda.synchronize()
            step()
        torch.cuda.synchronize()
    finally:
        gg._MOE_PLANS.update(plans)
    for what, v in acc.items():
        v = sorted(v)
        print(f"{what}: median {1e6 * v[len(v) // 2]:.1f} us host time per call "
              f"(min {1e6 * v[0]:.1f}), {len(v)} calls")
    with profile(activities=[ProfilerActivity.CPU]) as prof:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    print(f"torch.profiler, CPU only, {steps} steps (times are totals over the steps):")
    print(prof.key_averages().table(sort_by="self_cpu_time_total", row_limit=25))


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only (--gpus 1); the expert/data "
                          "parallel sharding of the layer is designed, not built or measured",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        sys.exit(1)
    device = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration()
        return
    if args.ceiling:
        ceiling()
        return
    if args.fp32_gemm:
        fp32_gemm()
        return
    if args.host_profile:
        host_profile(args.config, device, args.steps)
        return

    if args.profile_steps:
        torch.manual_seed(0)
        m, xb, _info = build_workload(args.config, device)
        time_steps(m, xb, args.profile_steps, 1)
        print(json.dumps({"profile_steps": args.profile_steps, "config": args.config}))
        return

    r = measure(args.config, device, args.steps, args.warmup, args.kernel_steps, not args.no_graph)
    m, xb, sel, info, counts, flops = r["m"], r["xb"], r["sel"], r["info"], r["counts"], r["flops"]
    ms, kern, dom = r["ms"], r["kern"], r["dom"]
    value = flops / (ms * 1e-3) / 1e12
    d, sizes, k, T, _ = CONFIGS[args.config]
    dom_bytes = gemm_bytes(dom, r["A"], T, d, r["nw"], r["W"])
    ai = flops / 6.0 / dom_bytes
    ai_bound = min(PEAK_BF16_TFLOPS, ai * PEAK_HBM_GBS / 1e3)
    achieved = r["achieved"]

    result = {
        "metric": "MoE fwd+bwd ms + grouped-GEMM TFLOP/s (% MFMA peak), 64 experts k=8 bf16",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) tokens, N(0,0.02) weights, Zipf-biased router)",
        "config": {"workload": f"{args.config}: TritonMoEMLP fwd+bwd, n_embd={d}, "
                               f"expert_sizes={sizes}, top_k={k}, tokens={T}, block_size=64",
                   "global_batch": T, "seq_len": T, "parallelism": "none (1 GPU)",
                   "zipf_alpha": info.get("alpha"),
                   "tokens_per_expert_min_max": [min(counts), max(counts)]},
        "gemm_flops_per_step": flops,
        "gemm_tflops_kernel_time": round(r["gemm_tflops"], 2),
        "gemm_pct_mfma_peak": round(100 * r["gemm_tflops"] / PEAK_BF16_TFLOPS, 2),
        "permutation_gbs": round(r["perm_gbs"], 1),
        "permutation_pct_hbm_peak": round(100 * r["perm_gbs"] / PEAK_HBM_GBS, 2),
        "permutation_pct_copy_rate": round(100 * r["perm_gbs"] / COPY_GBS, 2),
        "permutation_us": round(r["perm_us"], 2),
        "permutation_scope": "both combines + routing (vmoe_route_counted; the per-tile "
                             "expert counts come out of the top-k launch, router_topk_us), "
                             "bytes and time",
        "routing_us": round(kern["route"], 2),
        "router_topk_us": round(kern.get("router_topk", 0.0), 2),
        "kernel_us": {n: round(v, 2) for n, v in kern.items()},
        "graph_ms_per_step": None if r["graph_ms"] is None else round(r["graph_ms"], 4),
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic(args.config, GEMM_SYMBOL[dom]),
                     "algorithmic_bytes": dom_bytes,
                     "ai_flop_per_byte": round(ai, 1),
                     "ai_bound_tflops": round(ai_bound, 1),
                     "frac_of_ai_bound": round(achieved / ai_bound, 4)},
    }
    if not args.no_cpu_baseline:
        sec, threads = cpu_baseline(m, xb, sel, args.cpu_iters)
        result["cpu_baseline"] = {
            "value": round(flops / sec / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "ms_per_step": round(sec * 1e3, 1),
            "sample": f"full {args.config} step (fp32 eager per-expert-loop oracle, fwd+bwd), "
                      f"median of {args.cpu_iters} after 1 warmup, {cpu_model()}"}
    del m, xb, sel, r
    others = [c for c in args.other_configs.split(",") if c and c != args.config]
    if others:
        result["other_configs"] = {}
        for name in others:
            torch.cuda.empty_cache()
            o = measure(name, device, min(args.steps, 20), min(args.warmup, 5),
                        min(args.kernel_steps, 5), not args.no_graph)
            result["other_configs"][name] = summary(name, o)
            del o
            print(f"# {name} done", file=sys.stderr, flush=True)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
