"""oracle/topk.py (the reference router's top-k chain on CPU) against the
outputs PyTorch's GPU kernels recorded in tests/golden/topk_cases.json, and
against properties that fix the selected set without any tie order."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import topk

GOLDEN = Path(__file__).resolve().parent / "golden" / "topk_cases.json"


def _golden():
    return json.loads(GOLDEN.read_text())


def _f32(bits):
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


@pytest.mark.parametrize("case", [c["name"] for c in json.loads(GOLDEN.read_text())["cases"]])
def test_topk_chain_matches_recorded_torch(case):
    c = next(c for c in _golden()["cases"] if c["name"] == case)
    probs = _f32(c["levels_prob"])[np.asarray(c["idx"])]
    wb, sel = topk.route_weights(probs, c["k"], c["norm"])
    assert sel.tolist() == c["selected"]
    assert wb.astype(np.int64).tolist() == c["weights_bf16"]


def test_row_sum_matches_recorded_torch():
    for s in _golden()["sums"]:
        got = [topk.row_sum(_f32(r)) for r in s["rows"]]
        assert np.asarray(got, dtype=np.float32).view(np.uint32).tolist() == s["sum"], s["k"]


def test_row_sum_order_is_not_sequential():
    """The recorded sums pin an order: some rows differ from a left-to-right sum
    (otherwise the fixture would not tell the orders apart)."""
    differ = 0
    for s in _golden()["sums"]:
        for r, want in zip(s["rows"], s["sum"]):
            acc = np.float32(0)
            for v in _f32(r):
                acc = np.float32(acc + v)
            differ += int(np.float32(acc).view(np.uint32)) != want
    assert differ > 0


def test_golden_has_boundary_and_inner_ties():
    """The recorded rows exercise both kinds of ties the order depends on."""
    inner = boundary = 0
    for c in _golden()["cases"]:
        probs = _f32(c["levels_prob"])[np.asarray(c["idx"])]
        k = c["k"]
        for p, sel in zip(probs, c["selected"]):
            v = p[sel]
            inner += len(set(v.tolist())) < k
            kth = v[-1]
            boundary += int((p == kth).sum()) > int((v == kth).sum())
    assert inner > 100 and boundary > 100


@pytest.mark.parametrize("seed", range(5))
def test_selected_set_is_the_lexicographic_top_k(seed):
    """Whatever the order, the set is the k largest values with the lowest
    indices at the boundary: the first k of a sort by (-value, index)."""
    rng = np.random.default_rng(seed)
    for _ in range(50):
        E = int(rng.integers(1, 80))
        k = int(rng.integers(1, E + 1))
        p = rng.integers(0, 5, E).astype(np.float32) / 4
        got = topk.topk_indices(p, k)
        want = sorted(range(E), key=lambda e: (-p[e], e))[:k]
        assert sorted(got) == sorted(want)
        vals = p[got]
        assert all(vals[i] >= vals[i + 1] for i in range(k - 1)), "descending"


def test_distinct_values_sort_descending():
    rng = np.random.default_rng(7)
    for k in (1, 2, 5, 8, 16, 32, 40):
        p = rng.permutation(64).astype(np.float32)
        assert topk.topk_indices(p, k) == list(np.argsort(-p, kind="stable")[:k])


def test_small_known_answers():
    # equal values at the boundary: the lowest indices enter; bitonic order
    # of the selection [1, 4, 0, 2] (0.7, 0.9, 0.5, 0.5) is 4, 1, 0, 2
    p = np.array([0.5, 0.7, 0.5, 0.5, 0.9, 0.5], dtype=np.float32)
    assert topk.topk_indices(p, 4) == [4, 1, 0, 2]
    assert topk.topk_indices(p, 1) == [4]
    # k = 4 pairs (v0 + v1) + (v2 + v3): the two small terms meet first and
    # survive, where a left-to-right sum loses each of them to rounding
    v = np.array([1.0, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24], dtype=np.float32)
    assert topk.row_sum(v) == np.float32(1.0 + 2.0 ** -23)
    # k = 6: bw = 4, thread 0 adds v0 + v4, thread 1 adds v1 + v5
    v = np.array([1.0, 0.0, 2.0 ** -24, 0.0, 2.0 ** -24, 0.0], dtype=np.float32)
    assert topk.row_sum(v) == np.float32(1.0)
