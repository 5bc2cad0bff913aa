"""Helpers shared by the GPU parity tests."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import eager

# Normwise tolerances (max|d| / max|ref|, mean|d| / mean|ref|).
# Against the bf16-faithful oracle, only fp32 summation order differs.
TIGHT = (1e-2, 2e-3)
# Against the unrounded fp32 oracle: bf16 storage of H, Y, GY, GH, GA adds
# rounding (measured on the CPU by comparing the two oracle modes).
LOOSE = (2e-2, 6e-3)


def normwise(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    g = got.detach().float().cpu()
    r = ref.detach().float().cpu()
    d = (g - r).abs()
    mx = r.abs().max().item()
    mn = r.abs().mean().item()
    return (d.max().item() / mx if mx > 0 else d.max().item(),
            d.mean().item() / mn if mn > 0 else d.mean().item())


def assert_close_norm(got, ref, tol=TIGHT, what=""):
    assert got.shape == ref.shape, (what, tuple(got.shape), tuple(ref.shape))
    g = got.detach().float().cpu()
    assert torch.isfinite(g).all(), f"{what}: non-finite values"
    mx, mn = normwise(got, ref)
    assert mx <= tol[0] and mn <= tol[1], f"{what}: normwise max {mx:.3e} mean {mn:.3e} > {tol}"


def bf16_ulps(got: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 units in the last place between two bf16 tensors
    (int64, elementwise): the bit patterns mapped to a monotone integer
    line (sign-magnitude to two's complement), so +0 and -0 are 0 apart and
    neighbouring values across zero 1 apart."""
    def line(t):
        i = t.detach().cpu().to(torch.bfloat16).contiguous().view(torch.int16).to(torch.int64)
        mag = i & 0x7FFF
        return torch.where(i < 0, -mag, mag)
    return (line(got) - line(ref)).abs()


def parity_stats(got: torch.Tensor, ref: torch.Tensor, mag: torch.Tensor) -> dict:
    """ulp-level agreement of a bf16 result with an oracle that rounds at the
    same points (ref, rounded to bf16 here): shares of elements bit-equal and
    within 1 and 2 ulps, the largest ulp distance, and the largest
    conditioned error (|d| - ulp(ref)) / (2^-8 * mag), mag the sum of the
    magnitudes of the terms each element sums: an element whose terms agree
    to one rounding each stays at or below 1 however much its sum cancels."""
    r = ref.detach().cpu().float().to(torch.bfloat16)
    g = got.detach().cpu().to(torch.bfloat16)
    u = bf16_ulps(g, r)
    n = max(u.numel(), 1)
    rf = r.float()
    # one bf16 ulp of |ref|: 2^(e - 7) for normal values, 2^-133 below
    e = torch.frexp(rf.abs().clamp_min(2.0 ** -126))[1].to(torch.float32)
    ulp = torch.pow(2.0, e - 8)
    d = (g.float() - rf).abs()
    cond = ((d - ulp).clamp_min(0) / (2.0 ** -8 * mag.detach().cpu().float()).clamp_min(1e-30))
    return {"eq": float((u == 0).sum()) / n, "ulp1": float((u <= 1).sum()) / n,
            "ulp2": float((u <= 2).sum()) / n, "max_ulp": int(u.max()) if u.numel() else 0,
            "cond": float(cond.max()) if cond.numel() else 0.0}


def bits_equal(got: torch.Tensor, ref: torch.Tensor) -> bool:
    g = got.detach().cpu().contiguous()
    r = ref.detach().cpu().to(g.dtype).contiguous()
    if g.dtype == torch.bfloat16:
        return torch.equal(g.view(torch.int16), r.view(torch.int16))
    return torch.equal(g, r)


def make_problem(T, d, sizes, k, block_size=64, seed=0, skew=None, device="cuda"):
    """Seeded bf16 inputs on the CPU (so the oracle sees identical bits), routing
    decided on the device by the reference's own chain (moe.py:166-176):
    nn.Linear logits (+ skew, as a forward hook on the router adds it),
    sigmoid, torch.topk, normalisation, bf16."""
    g = torch.Generator().manual_seed(seed)
    widths, offsets = eager.expert_layout(sizes)
    E, W = len(widths), offsets[-1]
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    wr = (torch.randn(E, d, generator=g) * 0.02).to(torch.bfloat16)
    w1 = (torch.randn(d, W, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(W, d, generator=g) * 0.02).to(torch.bfloat16)
    logits = torch.nn.functional.linear(x.to(device), wr.to(device))
    if skew is not None:
        logits = logits + skew.to(device=device, dtype=logits.dtype)
    probs = torch.sigmoid(logits.float())
    wts, sel = torch.topk(probs, k, dim=-1)
    wts = (wts / (wts.sum(-1, keepdim=True) + 1e-20)).to(torch.bfloat16)
    return {"x": x, "wr": wr, "w1": w1, "w2": w2, "sel": sel, "wts": wts, "widths": widths,
            "offsets": offsets, "k": k, "E": E, "block_size": block_size, "logits": logits}


def oracle_problem(p, dtype=torch.float32) -> eager.Problem:
    return eager.Problem(p["x"].to(dtype), p["w1"].to(dtype), p["w2"].to(dtype), p["widths"],
                         p["offsets"], p["sel"].cpu(), p["wts"].cpu().to(dtype),
                         p["block_size"])


def zipf_bias(E: int, s: float = 1.2, alpha: float = 1.0, seed: int = 0) -> torch.Tensor:
    """Additive router bias -alpha * s * ln(rank), ranks a seeded permutation of 1..E."""
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(E) + 1
    return torch.tensor(-alpha * s * np.log(ranks), dtype=torch.float32)


def expert_rows(padded_bins) -> list[tuple[int, int]]:
    pb = [0] + [int(v) for v in padded_bins]
    return [(pb[i], pb[i + 1]) for i in range(len(pb) - 1)]


def cdiv(a, b):
    return -(-a // b)


def isclose_int(a, b):
    return math.isclose(a, b)
