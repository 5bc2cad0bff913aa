"""ctypes binding of libvmoe.so (the C ABI in include/vmoe.h).

The library is loaded on first use. If it is missing or fails to load, every
kernel entry point raises RuntimeError: there is no CPU or eager fallback.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("VMOE_LIB", _HERE / "libvmoe.so"))

_c_i32p = ctypes.c_void_p
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# name -> argtypes (all return int status unless listed in _RESTYPES)
_SIGNATURES = {
    "vmoe_status_string": [ctypes.c_int],
    "vmoe_version": [],
    "vmoe_set_launch_timing": [_vp, _vp],
    "vmoe_route_max_experts": [],
    "vmoe_route_workspace_bytes": [_i64, _i32],
    "vmoe_route": [_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                   _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp],
    "vmoe_route_counted": [_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                           _vp, _vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                           ctypes.c_size_t, _vp],
    "vmoe_route_static": [_vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                          _vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "vmoe_row_maps": [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i64, _i64, _vp, _vp, _vp, _vp],
    "vmoe_gather": [_vp, _i64, _i64, _vp, _i32, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp],
    "vmoe_gather_tokens": [_vp, _i64, _vp, _i64, _i32, _vp, _vp, _vp, _i64, _i64, _vp, _i64,
                           _vp],
    "vmoe_combine": [_vp, _i64, _i64, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp],
    "vmoe_combine_weight_grad": [_vp, _i64, _vp, _i64, _i64, _vp, _i32, _vp, _i64, _i64, _vp],
    "vmoe_routing_weight_grad": [_vp, _i64, _i32, _i64, _vp, _vp, _i64, _vp, _vp],
    "vmoe_expert_layout": [_i64, _i32, _i32, _i32, _i64, _i64, _i32, _vp],
    "vmoe_moe_layout": [_i64, _i32, _i32, _i32, _i64, _i64, _vp],
    "vmoe_moe_forward": [_vp, _i64, _i32, _i32, _i32, _i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp,
                         _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp],
    "vmoe_moe_backward": [_vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp, _i64, _vp, _i64, _vp,
                          _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp,
                          _i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, ctypes.c_size_t,
                          _vp, _vp],
    "vmoe_expert_forward": [_vp, _i32, _vp, _i64, _i32, _i32, _i32, _vp, ctypes.c_size_t, _vp,
                            _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp,
                            _i64, _vp],
    "vmoe_expert_backward": [_vp, _i64, _i32, _i32, _i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp,
                             _vp, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _i64,
                             _vp, _vp, _vp, ctypes.c_size_t, _vp, _vp],
    "vmoe_routing_weight_grad_direct": [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _i64,
                                        _i32, _vp, _vp, _vp, _i32, _i64, _i64, _vp, _vp],
    "vmoe_gemm_up_fwd": [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _i32, _vp, _vp, _vp,
                         _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "vmoe_gemm_down_fwd": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i64,
                           _i64, _i64, _vp],
    "vmoe_relu2_grad": [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp],
    "vmoe_gemm_up_glu": [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                         _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "vmoe_glu_grad": [_vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i32, _i64, _i64,
                      _vp],
    "vmoe_gemm_up_bwd_dx": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i64,
                            _i64, _i64, _vp],
    "vmoe_gemm_dw_workspace_bytes": [_i32, _i64, _i64, _i64],
    "vmoe_gemm_dw_workspace_zero_bytes": [],
    "vmoe_gemm_up_bwd_dw": [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp,
                            _i32, _i64, _i64, _i64, _vp, ctypes.c_size_t, _vp],
    "vmoe_gemm_down_bwd_dh": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp,
                              _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp],
    "vmoe_gemm_down_bwd_dw": [_vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                              _vp, _i32, _i64, _i64, _i64, _vp, ctypes.c_size_t, _vp],
    "vmoe_zero_tail_cols": [_vp, _i64, _vp, _vp, _i32, _i64, _i64, _vp],
    "vmoe_gemm_f32_up_fwd": [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i32, _vp,
                             _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "vmoe_gemm_f32_down_fwd": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i64,
                               _i64, _i64, _vp],
    "vmoe_gemm_f32_up_bwd_dx": [_vp, _vp, _vp, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp,
                                _vp, _i32, _i64, _i64, _i64, _vp],
    "vmoe_gemm_f32_up_bwd_dw": [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i32, _vp, _i64, _vp,
                                _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "vmoe_f32_relu2_grad": [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp],
    "vmoe_gemm_f32_down_bwd_dh": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32,
                                  _i64, _i64, _i64, _vp],
    "vmoe_gemm_f32_down_bwd_dw": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32,
                                  _i64, _i64, _i64, _vp],
    "vmoe_router_logits": [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _vp, _i64, _vp],
    "vmoe_router_partial_floats": [_i64, _i32],
    "vmoe_router_topk": [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                         ctypes.c_size_t, _vp, _vp],
    "vmoe_router_topk_hist_blocks": [_i64, _i32, _i32],
    "vmoe_router_topk_f32": [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                             ctypes.c_size_t, _vp, _vp],
    "vmoe_router_topk_hist_f32": [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                  _vp, ctypes.c_size_t, _vp, _vp, ctypes.c_size_t, _vp],
    "vmoe_router_aux_f32": [_vp, _i32, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "vmoe_router_aux_bwd_f32": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                _i64, _vp],
    "vmoe_router_weight_bwd_f32": [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _vp,
                                   _i64, _vp],
    "vmoe_combine_f32": [_vp, _i64, _i64, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp],
    "vmoe_gather_f32": [_vp, _i64, _i64, _vp, _i32, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp],
    "vmoe_combine_weight_grad_f32": [_vp, _i64, _vp, _i64, _i64, _vp, _i32, _vp, _i64, _i64,
                                     _vp],
    "vmoe_route_counted_workspace_bytes": [_i64, _i32, _i32],
    "vmoe_router_topk_hist": [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                              ctypes.c_size_t, _vp, _vp, ctypes.c_size_t, _vp],
    "vmoe_router_aux": [_vp, _i32, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "vmoe_router_aux_bwd": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                            _vp],
    "vmoe_router_weight_bwd": [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _vp, _i64,
                               _vp],
}
_RESTYPES = {
    "vmoe_status_string": ctypes.c_char_p,
    "vmoe_route_workspace_bytes": ctypes.c_size_t,
    "vmoe_route_counted_workspace_bytes": ctypes.c_size_t,
    "vmoe_gemm_dw_workspace_bytes": ctypes.c_size_t,
    "vmoe_gemm_dw_workspace_zero_bytes": ctypes.c_size_t,
    "vmoe_router_partial_floats": ctypes.c_size_t,
}

# Status codes (include/vmoe.h).
OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_LAUNCH, ERR_WORKSPACE = 0, 1, 2, 3, 4
ROUNDING = {"up": 0, "down": 1, "nearest": 2}
ACT_NONE, ACT_RELU_SQUARED, ACT_SWIGLU = 0, 1, 2
INFO_ROWS, INFO_KEPT, INFO_ERRORS, INFO_LEN = 0, 1, 2, 4
# Slots of vmoe_expert_layout's saved buffer (enum vmoe_expert_slot).
(X_BIN_IDS, X_INDICES, X_TPE, X_BINS, X_PADDED_BINS, X_ROW_SRC, X_GATHER_MAP, X_ASSIGNMENT_ROW,
 X_INFO, X_EXPERT_OFFSETS, X_PADDED_COUNTS, X_ROW_WEIGHT, X_H, X_PRE, X_NSLOTS) = range(15)
# Slots of vmoe_moe_layout's saved buffer after the expert ones (enum vmoe_moe_slot).
M_SELECTED, M_WEIGHTS, M_LSE, M_F_I32, M_NSLOTS = range(5)
ROUTE_BAD_EXPERT_ID, ROUTE_ROW_OVERFLOW = 1, 2

_lib = None
_load_error: Exception | None = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it cannot be loaded."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise RuntimeError(f"libvmoe.so unavailable: {_load_error}") from _load_error
    try:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} not found; build it with `python triton-variable-moe_amd/build.py`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = handle
        return _lib
    except Exception as exc:  # noqa: BLE001 - re-raised with context
        _load_error = exc
        raise RuntimeError(f"libvmoe.so unavailable: {exc}") from exc


def check(status: int, what: str) -> None:
    if status != OK:
        msg = lib().vmoe_status_string(status).decode()
        if status == ERR_UNSUPPORTED:
            raise NotImplementedError(f"{what}: {msg}")
        if status == ERR_INVALID_ARG:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what}: {msg} (status {status})")


# Optional observer of every launch (bench.py's per-kernel timing): an object
# with begin(name) and end(name), called around each entry point on the
# calling thread; None in normal use.
_launch_timer = None


def set_launch_timer(timer) -> None:
    global _launch_timer
    _launch_timer = timer


_FNS: dict = {}


def call(name: str, *args) -> None:
    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(lib(), name)
    timer = _launch_timer
    if timer is None:
        status = fn(*args)
        if status != OK:
            check(status, name)
        return
    timer.begin(name)
    status = fn(*args)
    timer.end(name)
    check(status, name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    """The raw hipStream_t of the device's current stream (what
    torch.cuda.current_stream(device).cuda_stream returns, without building
    a Stream object)."""
    if not isinstance(device, (torch.device, int)):
        device = torch.device(device)
    idx = device.index if isinstance(device, torch.device) else device
    if idx is None:
        idx = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def require_gpu(t: torch.Tensor, what: str = "Input") -> None:
    if not t.is_cuda:
        raise AssertionError(f"{what} must be on CUDA")
