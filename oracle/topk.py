"""CPU restatement of the reference router's top-k step (test infrastructure only).

The reference module routes with (triton_moe/moe.py:168-176)

    router_probs = F.sigmoid(router_logits.float())
    top_k_weights, selected_experts = torch.topk(router_probs, k, dim=-1)
    if norm_topk_prob:
        top_k_weights = top_k_weights / (top_k_weights.sum(dim=-1, keepdim=True) + 1e-20)
    top_k_weights = top_k_weights.to(bf16)

The selected set is fixed by the values (the k largest; at the boundary the
lowest indices). The ORDER of equal values and the fp32 rounding of the sum
are fixed by PyTorch's GPU kernels, which this file restates for rows of up
to a few thousand values (PyTorch 2.x on ROCm; the reference's dependency,
not vendored in the reference):

* selection (aten/src/ATen/native/cuda/TensorTopK.cu, single-block path):
  the values strictly above the k-th largest, in ascending index order, then
  the values equal to it in ascending index order until k are written;
* sort of the k results (aten/src/ATen/native/cuda/Sort.cu,
  sortKeyValueInplace): nothing for k == 1; for k <= 32 the in-place bitonic
  sort of SortUtils.cuh (bitonicSortKVInPlace, 32 slots, 16 comparators per
  pass, descending, unused slots sorted to the end); for larger k a stable
  sort, descending;
* sum over the k values (aten/src/ATen/native/cuda/Reduce.cuh): block width
  bw = the largest power of two <= k (at most the wave size, 64), thread x
  adds elements x, x + bw, x + 2 bw ... starting from 0, then the threads are
  combined by shfl_down with offsets 1, 2, ..., bw / 2.

Pinned by tests/test_oracle_topk.py against torch.topk / torch.sum outputs
recorded on the GPU (tests/golden/topk_cases.json, made by
tests/golden/make_topk_golden.py), and by properties that fix the selected
set independently of the order (a lexicographic sort).
"""

from __future__ import annotations

import numpy as np
import torch

f32 = np.float32


def _selection(p: np.ndarray, k: int) -> list[int]:
    """TensorTopK.cu's selection order: > kth by index, then == kth by index."""
    E = len(p)
    kth = sorted((float(v) for v in p), reverse=True)[k - 1]
    gt = [e for e in range(E) if p[e] > kth]
    eq = [e for e in range(E) if p[e] == kth][: k - len(gt)]
    return gt + eq


def _bitonic32(keys: list[float], vals: list[int], n: int) -> list[int]:
    """bitonicSortKVInPlace with 32 slots (2 per thread, 16 threads), descending;
    slot i is valid for i < n. Returns the first n values."""
    size_all = 32
    keys = list(keys) + [0.0] * (size_all - n)
    vals = list(vals) + [0] * (size_all - n)
    valid = [True] * n + [False] * (size_all - n)

    def swap(i: int, j: int, direction: bool) -> None:
        # invalid entries always sort to the end
        s = (keys[i] > keys[j] and valid[i]) or not valid[j]
        if s == direction:
            keys[i], keys[j] = keys[j], keys[i]
            vals[i], vals[j] = vals[j], vals[i]
            valid[i], valid[j] = valid[j], valid[i]

    size = 2
    while size < size_all:
        stride = size // 2
        while stride > 0:
            for tid in range(size_all // 2):
                flag = (tid & (size // 2)) != 0
                pos = 2 * tid - (tid & (stride - 1))
                swap(pos, pos + stride, flag)
            stride //= 2
        size *= 2
    stride = size_all // 2
    while stride > 0:
        for tid in range(size_all // 2):
            pos = 2 * tid - (tid & (stride - 1))
            swap(pos, pos + stride, False)
        stride //= 2
    return vals[:n]


def topk_indices(p: np.ndarray, k: int) -> list[int]:
    """Indices of torch.topk(p, k) on the GPU, in its output order (p: fp32 row)."""
    p = np.asarray(p, dtype=f32)
    if not 1 <= k <= len(p):
        raise ValueError("need 1 <= k <= len(p)")
    sel = _selection(p, k)
    if k == 1:
        return sel
    if k <= 32:
        return _bitonic32([float(p[e]) for e in sel], sel, k)
    return sorted(sel, key=lambda e: -float(p[e]))  # stable: ties keep selection order


def row_sum(v: np.ndarray) -> np.float32:
    """torch.sum(v) of a contiguous fp32 row of k values, in the GPU kernel's order."""
    v = np.asarray(v, dtype=f32)
    k = len(v)
    bw = 1
    while bw * 2 <= min(k, 64):
        bw *= 2
    acc = []
    for x in range(bw):
        a = f32(0.0)
        for j in range(x, k, bw):
            a = f32(a + v[j])
        acc.append(a)
    off = 1
    while off < bw:
        for x in range(0, bw, 2 * off):
            acc[x] = f32(acc[x] + acc[x + off])
        off *= 2
    return acc[0]


def route_weights(probs: np.ndarray, k: int, norm: bool) -> tuple[np.ndarray, np.ndarray]:
    """(bf16 weights as uint16 bits [T, k], selected experts [T, k]) of the
    reference's routing chain, given router_probs [T, E] (fp32)."""
    probs = np.asarray(probs, dtype=f32)
    T = probs.shape[0]
    sel = np.zeros((T, k), dtype=np.int64)
    w = np.zeros((T, k), dtype=f32)
    eps = f32(1e-20)
    for t in range(T):
        idx = topk_indices(probs[t], k)
        v = probs[t][idx]
        sel[t] = idx
        if norm:
            s = f32(row_sum(v) + eps)
            w[t] = np.array([f32(x / s) for x in v], dtype=f32)
        else:
            w[t] = v
    wb = torch.from_numpy(w).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return wb, sel
