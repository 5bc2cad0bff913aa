"""CPU oracle of the MoE MLP hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker or the timed CPU baseline. The product
(triton-variable-moe_amd/triton_moe) never imports it and has no CPU fallback.

Contents:
  route.py  -- ctypes wrapper of route_oracle.c: fused_route and the row maps
               (bit-exact integer restatement).
  eager.py  -- fp32 eager per-expert-loop restatement of TritonMoEMLP's
               forward and backward, in two modes: "fp32" (no intermediate
               rounding; the tolerance oracle) and "bf16" (rounds to bf16
               exactly where the reference's kernels do; the tight oracle).
  topk.py   -- the reference router's top-k chain (torch.topk order of equal
               values and torch.sum order on the GPU, normalisation, bf16).

Pinning (what checks each function against something other than itself):
  route / row maps: numpy stable argsort + bincount + cumsum (library
      routines), a pure-Python brute force on small inputs, hand-computed
      known answers and invariants (tests/test_oracle_route.py).
  eager forward/backward: a dense all-experts formulation with a routing
      weight matrix and torch autograd for the gradients, float64 on small
      inputs (tests/test_oracle_eager.py).
  topk chain: torch.topk / torch.sum outputs recorded on a ROCm GPU
      (tests/golden/topk_cases.json) and a lexicographic sort for the
      selected set (tests/test_oracle_topk.py).
"""
