#!/usr/bin/env python
"""Parity report of TritonMoEMLP against the eager oracle, per configuration
(the configurations of tests/test_gpu_module.py): for out, x.grad, w1.grad
and w2.grad, the share of elements bit-equal to / within 1 and 2 bf16 ulps of
the oracle rounding in the module's order ("bf16w"), the largest ulp
distance, the largest error measured against the element's own conditioning
(|d| - ulp(ref)) / (2^-8 * M), M the sum of the magnitudes of the terms the
element sums (so that a result that cancels to near zero is judged by its
terms, not by its own size), and the normwise errors (max|d| / max|ref|,
mean|d| / mean|ref|) against the bf16w and the unrounded fp32 oracles.

Run on a GPU box: python tests/parity_report.py [config ...] > report.md
(not collected by pytest; tests/test_gpu_module.py asserts the bounds).
"""

from __future__ import annotations

import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
for p in (str(HERE), str(HERE.parent), str(HERE.parent / "triton-variable-moe_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

from _util import normwise, parity_stats  # noqa: E402
from oracle import eager  # noqa: E402
from test_gpu_module import CONFIGS, _run, term_magnitudes  # noqa: E402


def main(names):
    device = torch.device("cuda:0")
    print("| config | tensor | bit-equal % | ≤ 1 ulp % | ≤ 2 ulp % | max ulp | max conditioned "
          "error | normwise vs bf16w (max / mean) | normwise vs fp32 (max / mean) |")
    print("|---|---|---|---|---|---|---|---|---|")
    for name in names:
        m, x, out, _aux, _f_i, prob = _run(name, device)
        T, d = prob.x.shape
        if T <= 4096:
            G = torch.randn(T, d, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
            out.backward(G.to(device).view_as(out))
        else:
            G = torch.ones(T, d, dtype=torch.bfloat16)
            out.sum().backward()
        fb, ff = eager.forward(prob, "bf16w"), eager.forward(prob, "fp32")
        bb = eager.backward(prob, fb, G.float(), "bf16w")
        bf_ = eager.backward(prob, ff, G.float(), "fp32")
        mags = term_magnitudes(prob, fb, bb)
        got = {"out": out.detach().reshape(T, d), "grad_x": x.grad.reshape(T, d),
               "grad_w1": m.w1.grad, "grad_w2": m.w2.grad}
        refb = {"out": fb["out"], "grad_x": bb["grad_x"], "grad_w1": bb["grad_w1"],
                "grad_w2": bb["grad_w2"]}
        reff = {"out": ff["out"], "grad_x": bf_["grad_x"], "grad_w1": bf_["grad_w1"],
                "grad_w2": bf_["grad_w2"]}
        for key in got:
            s = parity_stats(got[key], refb[key], mags[key])
            nb, nf = normwise(got[key], refb[key]), normwise(got[key], reff[key])
            print(f"| {name} | {key} | {100 * s['eq']:.3f} | {100 * s['ulp1']:.3f} | "
                  f"{100 * s['ulp2']:.3f} | {s['max_ulp']} | {s['cond']:.3f} | "
                  f"{nb[0]:.2e} / {nb[1]:.2e} | {nf[0]:.2e} / {nf[1]:.2e} |", flush=True)
        del m, x, out


if __name__ == "__main__":
    main(sys.argv[1:] or list(CONFIGS))
