"""Writes tests/golden/route_cases.json: routing known answers.

Expected values come from an independent pure-Python brute force (Python's
stable `sorted`, plain counting, exact rational rounding), not from the C
oracle or the HIP kernels, so the fixtures check both. Semantics are those of
fused_route (triton_moe/kernels/fused_cumsum.py:85-171) and
precompute_gather_map (triton_moe/kernels/grouped_gemm.py:104-149).

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import math
import random
from fractions import Fraction
from pathlib import Path

OUT = Path(__file__).resolve().parent / "route_cases.json"


def rounded(c: int, b: int, mode: str) -> int:
    if mode == "up":
        return b * math.ceil(Fraction(c, b))
    if mode == "down":
        return b * math.floor(Fraction(c, b))
    return b * math.floor(Fraction(c, b) + Fraction(1, 2))  # nearest, ties up


def brute(sel, E, k, b, mode):
    A = len(sel)
    order = sorted(range(A), key=lambda i: sel[i])  # stable
    tpe = [sum(1 for s in sel if s == e) for e in range(E)]
    kept = [min(c, rounded(c, b, mode)) for c in tpe]
    rnd = [rounded(c, b, mode) for c in tpe]
    bin_ids, indices = [], []
    for e in range(E):
        members = [i for i in order if sel[i] == e][: kept[e]]
        bin_ids += [e] * len(members)
        indices += members
    bins = [sum(kept[: e + 1]) for e in range(E)]
    padded = [sum(rnd[: e + 1]) for e in range(E)]
    P = padded[-1]
    gm = [0] * P
    row_src = [-1] * P
    arow = [-1] * A
    for i, (e, a) in enumerate(zip(bin_ids, indices)):
        row = (padded[e - 1] if e else 0) + i - (bins[e - 1] if e else 0)
        gm[row] = a // k
        row_src[row] = a
        arow[a] = row
    return {"bin_ids": bin_ids, "indices": indices, "tokens_per_expert": tpe, "bins": bins,
            "padded_bins": padded, "gather_map": gm, "row_src": row_src,
            "assignment_row": arow}


def topk_like(rng, T, E, k):
    """Per-token distinct experts in random order, like torch.topk rows."""
    out = []
    for _ in range(T):
        out += rng.sample(range(E), k)
    return out


def cases():
    rng = random.Random(20260101)
    yield "tiny", [2, 0, 2, 1, 0, 2], 3, 1, 2
    yield "empty", [], 4, 2, 64
    yield "all_one_expert", [1] * 10, 4, 1, 4
    yield "exact_multiples", [0] * 8 + [1] * 4 + [3] * 12, 4, 1, 4
    yield "single_expert", [0] * 7, 1, 1, 4
    yield "k_equals_E", topk_like(rng, 5, 4, 4), 4, 4, 4
    yield "odd_block", topk_like(rng, 40, 6, 2), 6, 2, 3
    yield "uniform_b64", topk_like(rng, 300, 8, 3), 8, 3, 64
    yield "uniform_b128", topk_like(rng, 300, 8, 3), 8, 3, 128
    skew = [min(int(rng.paretovariate(1.2)) - 1, 15) for _ in range(400)]
    yield "skew_empty_experts", skew, 16, 1, 8
    yield "many_experts", topk_like(rng, 200, 64, 8), 64, 8, 16


def main():
    data = []
    for name, sel, E, k, b in cases():
        for mode in ("up", "down", "nearest"):
            data.append({"name": f"{name}-{mode}", "selected": sel, "num_experts": E,
                         "top_k": k, "block_size": b, "rounding": mode,
                         "expected": brute(sel, E, k, b, mode)})
    OUT.write_text(json.dumps(data, separators=(",", ":")))
    print(f"wrote {len(data)} cases to {OUT}")


if __name__ == "__main__":
    main()
