"""Pins the routing oracle (oracle/route_oracle.c) on the CPU.

Checks, each independent of the oracle's own code:
  * the golden fixtures (pure-Python brute force, tests/golden/make_golden.py);
  * numpy's stable argsort / bincount / cumsum on random inputs;
  * hand-computed known answers;
  * invariants (sortedness, permutation, stability, block alignment).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import route as oroute

GOLDEN = json.loads((Path(__file__).parent / "golden" / "route_cases.json").read_text())


@pytest.mark.parametrize("case", GOLDEN, ids=[c["name"] for c in GOLDEN])
def test_oracle_matches_golden(case):
    sel = np.asarray(case["selected"], np.int64)
    E, k, b, mode = case["num_experts"], case["top_k"], case["block_size"], case["rounding"]
    r = oroute.route(sel, E, b, mode)
    exp = case["expected"]
    for key in ("bin_ids", "indices", "tokens_per_expert", "bins", "padded_bins"):
        np.testing.assert_array_equal(r[key], np.asarray(exp[key], np.int32), err_msg=key)
    m = oroute.row_maps(r["indices"], r["bin_ids"], r["bins"], r["padded_bins"], k,
                        num_assignments=sel.size)
    for key in ("gather_map", "row_src", "assignment_row"):
        np.testing.assert_array_equal(m[key], np.asarray(exp[key], np.int32), err_msg=key)


def test_known_answer_by_hand():
    # sel = [2, 0, 2, 1, 0, 2], E = 3, block 2, top_k 1
    r = oroute.route([2, 0, 2, 1, 0, 2], 3, 2, "up")
    assert r["bin_ids"].tolist() == [0, 0, 1, 2, 2, 2]
    assert r["indices"].tolist() == [1, 4, 3, 0, 2, 5]
    assert r["tokens_per_expert"].tolist() == [2, 1, 3]
    assert r["bins"].tolist() == [2, 3, 6]
    assert r["padded_bins"].tolist() == [2, 4, 8]
    m = oroute.row_maps(r["indices"], r["bin_ids"], r["bins"], r["padded_bins"], 1,
                        num_assignments=6)
    # expert 0 -> rows 0,1; expert 1 -> row 2 (row 3 pad); expert 2 -> rows 4,5,6 (7 pad)
    assert m["row_src"].tolist() == [1, 4, 3, -1, 0, 2, 5, -1]
    assert m["gather_map"].tolist() == [1, 4, 3, 0, 0, 2, 5, 0]
    assert m["assignment_row"].tolist() == [4, 0, 5, 2, 1, 6]
    # rounding down drops the third token of expert 2 and all of expert 1
    d = oroute.route([2, 0, 2, 1, 0, 2], 3, 2, "down")
    assert d["bin_ids"].tolist() == [0, 0, 2, 2]
    assert d["indices"].tolist() == [1, 4, 0, 2]
    assert d["bins"].tolist() == [2, 2, 4]
    assert d["padded_bins"].tolist() == [2, 2, 4]
    # nearest: counts 2,1,3 with b=2 -> 2,2,4 (1 and 3 round half up)
    n = oroute.route([2, 0, 2, 1, 0, 2], 3, 2, "nearest")
    assert n["padded_bins"].tolist() == [2, 4, 8]
    assert n["bins"].tolist() == [2, 3, 6]


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("mode", ["up", "down", "nearest"])
def test_oracle_matches_numpy(seed, mode):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 200))
    A = int(rng.integers(0, 5000))
    b = int(rng.choice([1, 3, 16, 64, 128]))
    # skewed ids so some experts are empty
    sel = np.minimum((rng.pareto(1.0, A) * E / 8).astype(np.int64), E - 1)
    r = oroute.route(sel, E, b, mode)
    order = np.argsort(sel, kind="stable")
    tpe = np.bincount(sel, minlength=E)
    if mode == "up":
        rnd = -(-tpe // b) * b
    elif mode == "down":
        rnd = tpe // b * b
    else:
        rnd = (tpe + b // 2) // b * b
    kept = np.minimum(tpe, rnd)
    np.testing.assert_array_equal(r["tokens_per_expert"], tpe)
    np.testing.assert_array_equal(r["bins"], np.cumsum(kept))
    np.testing.assert_array_equal(r["padded_bins"], np.cumsum(rnd))
    starts = np.concatenate([[0], np.cumsum(tpe)[:-1]])
    keep = np.concatenate([order[s:s + kk] for s, kk in zip(starts, kept)]) if A else order
    np.testing.assert_array_equal(r["indices"], keep)
    np.testing.assert_array_equal(r["bin_ids"], sel[keep])


def test_invariants_large():
    rng = np.random.default_rng(7)
    T, k, E, b = 4096, 8, 64, 64
    sel = np.stack([rng.permutation(E)[:k] for _ in range(T)]).reshape(-1)
    r = oroute.route(sel, E, b, "up")
    A = sel.size
    assert r["bins"][-1] == A
    assert np.all(r["padded_bins"] % b == 0)
    assert np.all(np.diff(r["bin_ids"]) >= 0)
    assert sorted(r["indices"].tolist()) == list(range(A))
    # stable: indices ascend inside each expert
    for e in range(E):
        seg = r["indices"][r["bin_ids"] == e]
        assert np.all(np.diff(seg) > 0)
    m = oroute.row_maps(r["indices"], r["bin_ids"], r["bins"], r["padded_bins"], k,
                        num_assignments=A)
    valid = m["row_src"] >= 0
    assert valid.sum() == A
    np.testing.assert_array_equal(m["gather_map"][valid], m["row_src"][valid] // k)
    np.testing.assert_array_equal(m["assignment_row"][m["row_src"][valid]],
                                  np.nonzero(valid)[0])


def test_bad_expert_id_raises():
    with pytest.raises(ValueError):
        oroute.route([0, 5], 3, 4, "up")
    with pytest.raises(ValueError):
        oroute.route([0, -1], 3, 4, "up")
