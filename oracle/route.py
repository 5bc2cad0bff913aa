"""ctypes wrapper of oracle/route_oracle.c (test infrastructure only).

route()    restates fused_route       (triton_moe/kernels/fused_cumsum.py:85-171)
row_maps() restates precompute_gather_map (triton_moe/kernels/grouped_gemm.py:104-149)
           and the padded-row placement of gather.py:34-60 / scatter.py:35-69.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "_build" / "liboracle.so"
_lib = None

ROUNDING = {"up": 0, "down": 1, "nearest": 2}


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            from . import build as _b  # noqa: PLC0415

            _b.build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.POINTER
        lib.oracle_route.restype = ctypes.c_int
        lib.oracle_route.argtypes = [
            P(ctypes.c_int64), ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            P(ctypes.c_int32), P(ctypes.c_int32), P(ctypes.c_int32), P(ctypes.c_int32),
            P(ctypes.c_int32), P(ctypes.c_int64),
        ]
        lib.oracle_row_maps.restype = None
        lib.oracle_row_maps.argtypes = [
            P(ctypes.c_int32), P(ctypes.c_int32), P(ctypes.c_int32), P(ctypes.c_int32),
            ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ]
        _lib = lib
    return _lib


def _i32p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def route(selected, num_experts: int, block_size: int = 128, rounding: str = "up") -> dict:
    """Returns bin_ids, indices, tokens_per_expert, bins, padded_bins (int32 numpy)."""
    if rounding not in ROUNDING:
        raise ValueError(f"Invalid rounding mode: {rounding}")
    sel = np.ascontiguousarray(np.asarray(selected).reshape(-1), dtype=np.int64)
    A = sel.size
    bin_ids = np.zeros(max(A, 1), np.int32)
    indices = np.zeros(max(A, 1), np.int32)
    tpe = np.zeros(num_experts, np.int32)
    bins = np.zeros(num_experts, np.int32)
    padded = np.zeros(num_experts, np.int32)
    n_kept = ctypes.c_int64(0)
    rc = _load().oracle_route(
        sel.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), A, num_experts, block_size,
        ROUNDING[rounding], _i32p(bin_ids), _i32p(indices), _i32p(tpe), _i32p(bins),
        _i32p(padded), ctypes.byref(n_kept))
    if rc == 1:
        raise ValueError("selected_experts holds ids outside [0, num_experts)")
    if rc != 0:
        raise RuntimeError(f"oracle_route failed ({rc})")
    n = n_kept.value
    return {
        "bin_ids": bin_ids[:n].copy(),
        "indices": indices[:n].copy(),
        "tokens_per_expert": tpe,
        "bins": bins,
        "padded_bins": padded,
    }


def row_maps(indices, bin_ids, bins, padded_bins, top_k: int, num_rows: int | None = None,
             num_assignments: int = 0) -> dict:
    """gather_map [P], row_src [P] and assignment_row [num_assignments] (int32)."""
    indices = np.ascontiguousarray(indices, np.int32)
    bin_ids = np.ascontiguousarray(bin_ids, np.int32)
    bins = np.ascontiguousarray(bins, np.int32)
    padded_bins = np.ascontiguousarray(padded_bins, np.int32)
    P = int(padded_bins[-1]) if num_rows is None else int(num_rows)
    gm = np.zeros(max(P, 1), np.int32)
    rs = np.zeros(max(P, 1), np.int32)
    ar = np.zeros(max(num_assignments, 1), np.int32)
    _load().oracle_row_maps(
        _i32p(indices), _i32p(bin_ids), _i32p(bins), _i32p(padded_bins), indices.size,
        bins.size, top_k, P, num_assignments, gm.ctypes.data, rs.ctypes.data, ar.ctypes.data)
    return {"gather_map": gm[:P], "row_src": rs[:P], "assignment_row": ar[:num_assignments]}
