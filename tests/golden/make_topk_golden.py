"""Writes tests/golden/topk_cases.json: outputs of the reference router's
top-k chain (torch.sigmoid -> torch.topk -> normalise -> bf16, reference
triton_moe/moe.py:168-176) and of torch.sum over short fp32 rows, computed
by PyTorch on a ROCm GPU. They pin oracle/topk.py, which restates the order
PyTorch's GPU kernels give to equal values and to the sum.

Run on a GPU box from the repository root:
    python tests/golden/make_topk_golden.py
Inputs are seeded; logits are drawn from a few bf16 levels per case so that
ties (inside the top k and at its boundary) are common.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

OUT = Path(__file__).resolve().parent / "topk_cases.json"

# (name, E, k, norm, levels, rows)
CASES = [
    ("e64_k8_l16", 64, 8, True, 16, 64),
    ("e64_k8_l4", 64, 8, True, 4, 64),
    ("e64_k8_l16_nonorm", 64, 8, False, 16, 32),
    ("e8_k2_l4", 8, 2, True, 4, 64),
    ("e16_k2_l6", 16, 2, True, 6, 64),
    ("e128_k8_l24", 128, 8, True, 24, 32),
    ("e64_k1_l8", 64, 1, True, 8, 32),
    ("e64_k3_l8", 64, 3, True, 8, 32),
    ("e64_k5_l8", 64, 5, True, 8, 32),
    ("e64_k6_l8", 64, 6, True, 8, 32),
    ("e64_k7_l8", 64, 7, True, 8, 32),
    ("e40_k12_l8", 40, 12, True, 8, 32),
    ("e256_k16_l16", 256, 16, True, 16, 16),
    ("e64_k32_l8", 64, 32, True, 8, 16),
    ("e256_k48_l16", 256, 48, True, 16, 8),
    ("e2048_k8_l64", 2048, 8, True, 64, 8),
]


def bits16(t: torch.Tensor) -> list[int]:
    return [int(v) & 0xFFFF for v in t.contiguous().view(torch.int16).reshape(-1).tolist()]


def bits32(t: torch.Tensor) -> list[int]:
    return [int(v) & 0xFFFFFFFF for v in t.contiguous().view(torch.int32).reshape(-1).tolist()]


def main() -> None:
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1234)
    cases = []
    for name, E, k, norm, nlev, T in CASES:
        levels = (torch.randn(nlev, generator=g) * 2.0).to(torch.bfloat16)
        idx = torch.randint(0, nlev, (T, E), generator=g)
        L = levels[idx].to(dev)
        probs = torch.sigmoid(L.float())
        w, sel = torch.topk(probs, k, dim=-1)
        if norm:
            w = w / (w.sum(dim=-1, keepdim=True) + 1e-20)
        w = w.to(torch.bfloat16)
        cases.append({
            "name": name, "E": E, "k": k, "norm": norm,
            "levels_bf16": bits16(levels),
            "levels_prob": bits32(torch.sigmoid(levels.to(dev).float()).cpu()),
            "idx": idx.tolist(),
            "selected": sel.cpu().tolist(),
            "weights_bf16": [bits16(row) for row in w.cpu()],
        })
    sums = []
    for k in list(range(1, 17)) + [24, 31, 32, 33, 48, 63, 64]:
        v = torch.rand(8, k, generator=g) * torch.exp2(torch.randint(-8, 8, (8, k), generator=g).float())
        s = v.to(dev).sum(dim=-1).cpu()
        sums.append({"k": k, "rows": [bits32(r) for r in v], "sum": bits32(s)})
    OUT.write_text(json.dumps({"torch": torch.__version__, "device": torch.cuda.get_device_name(0),
                               "cases": cases, "sums": sums}, separators=(",", ":")))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
