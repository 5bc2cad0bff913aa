"""The C-ABI library loads and exports every symbol include/vmoe.h declares,
and its argument checks fire on the host (no GPU needed: none of these calls
reach a kernel launch)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from triton_moe import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "vmoe.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(vmoe_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("vmoe_route", "vmoe_row_maps", "vmoe_gather", "vmoe_combine",
                 "vmoe_gemm_up_fwd", "vmoe_gemm_down_fwd", "vmoe_gemm_up_bwd_dx",
                 "vmoe_gemm_up_bwd_dw", "vmoe_gemm_down_bwd_dh", "vmoe_gemm_down_bwd_dw",
                 "vmoe_zero_tail_cols", "vmoe_status_string", "vmoe_gather_tokens",
                 "vmoe_gemm_f32_up_fwd", "vmoe_gemm_f32_down_fwd", "vmoe_gemm_f32_up_bwd_dx",
                 "vmoe_gemm_f32_up_bwd_dw", "vmoe_gemm_f32_down_bwd_dh",
                 "vmoe_gemm_f32_down_bwd_dw", "vmoe_f32_relu2_grad"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers them all
    assert set(declared_functions()) == set(_lib._SIGNATURES)


def test_status_strings_and_queries():
    lib = _lib.lib()
    assert lib.vmoe_status_string(0) == b"ok"
    assert b"multiple" in lib.vmoe_status_string(2)
    assert lib.vmoe_version() >= 1
    assert lib.vmoe_route_max_experts() >= 1024
    ws = lib.vmoe_route_workspace_bytes(262144, 128)
    assert ws >= 4 * 128 * (262144 // 1024)
    assert lib.vmoe_route_workspace_bytes(-1, 4) == 0
    # the dW workspace's arrival words: a 256-byte multiple, at most 8 KiB,
    # a prefix of the whole workspace
    z = lib.vmoe_gemm_dw_workspace_zero_bytes()
    assert 0 < z <= 8192 and z % 256 == 0
    assert lib.vmoe_gemm_dw_workspace_bytes(64, 1024, 256, 140000) > z


def test_argument_checks_return_invalid_arg():
    lib = _lib.lib()
    # negative sizes / bad enums are rejected before any launch
    assert lib.vmoe_route(None, 0, -1, 4, 1, 64, 0, None, None, None, None, None, None, None,
                          0, 0, None, None, None, None, None, None, None, 0,
                          None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_route(None, 0, 0, 4, 1, 64, 7, None, None, None, None, None, None, None,
                          0, 0, None, None, None, None, None, None, None, 0,
                          None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gather(None, 0, 0, None, 1, None, 0, None, 8, -1, None, 8,
                           None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_combine(None, 0, 0, None, None, 0, None, 8, 1, 8, None) == _lib.ERR_INVALID_ARG
    # routing-weight gradient: bad top_k, negative stride, missing output
    assert lib.vmoe_combine_weight_grad(1, 8, 1, 4, 8, 1, 0, 1, 4, 8,
                                        None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_combine_weight_grad(1, -8, 1, 4, 8, 1, 2, 1, 4, 8,
                                        None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_combine_weight_grad(1, 8, 1, 4, 8, 1, 2, None, 4, 8,
                                        None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_combine_weight_grad(None, 0, None, 0, 0, None, 2, None, 0, 8,
                                        None) == _lib.OK
    # module-path routing-weight gradient: ld below the block count, missing inputs
    assert lib.vmoe_routing_weight_grad(1, 2, 4, 8, 1, 1, 16, 1, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_routing_weight_grad(1, 4, 4, 8, None, 1, 16, 1, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_routing_weight_grad(None, 4, 4, 8, 1, None, 0, None, None) == _lib.OK
    # its direct form for tiny weights: ldw2 below hidden, top_k 0, missing pre_act
    f = lib.vmoe_routing_weight_grad_direct
    args = [1, 64, 8, None, 1, 64, 1, 256, 1, 1, 16, 2, 1, 1, 1, 4, 64, 32, 1, None]
    assert f(*args[:4], 1, 32, *args[6:]) == _lib.ERR_INVALID_ARG
    assert f(*args[:11], 0, *args[12:]) == _lib.ERR_INVALID_ARG
    assert f(*args[:6], None, *args[7:]) == _lib.ERR_INVALID_ARG
    assert f(*args[:10], 0, *args[11:]) == _lib.OK  # no assignments: nothing to do
    # fp32 permutation: bad top_k, short ldo, missing output
    assert lib.vmoe_combine_f32(1, 8, 16, 1, None, 0, 1, 16, 4, 16,
                                None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_combine_f32(1, 8, 16, 1, None, 2, 1, 8, 4, 16, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gather_f32(1, 8, 16, 1, 2, None, 0, None, 16, 4, None, 16,
                               None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_combine_weight_grad_f32(1, 16, 1, 8, 8, 1, 2, 1, 4, 16,
                                            None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_combine_f32(None, 0, 16, None, None, 2, None, 16, 0, 16, None) == _lib.OK
    # fp32 router: k > E invalid, more than 2048 experts unsupported; aux needs outputs
    assert lib.vmoe_router_topk_f32(1, 8, 4, 8, 9, 1, 1, 1, None, None, 1, 1, 1 << 20, None,
                                    None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_router_topk_f32(1, 4096, 4, 4096, 8, 1, 1, 1, None, None, 1, 1, 1 << 20,
                                    None, None) == _lib.ERR_UNSUPPORTED
    assert lib.vmoe_router_aux_f32(1, 1, 4, 8, 1, 1, 1, None, 1, 1, 1, 1,
                                   None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_router_weight_bwd_f32(1, 8, 4, 8, 2, 1, 1, 1, 1, 2, 1, 8,
                                          None) == _lib.ERR_INVALID_ARG
    # layer / expert path: layouts, and calls with missing buffers
    lay = (ctypes.c_int64 * (5 + _lib.X_NSLOTS + _lib.M_NSLOTS))()
    assert lib.vmoe_moe_layout(16384, 64, 8, 64, 1024, 256, lay) == _lib.OK
    assert lay[3] == 16384 * 8 + 64 * 63                 # rows bound of a dropless routing
    assert lay[4 + _lib.X_NSLOTS + _lib.M_NSLOTS] == 1   # the counted top-k applies
    offs = list(lay[4:4 + _lib.X_NSLOTS + _lib.M_NSLOTS])
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs) and offs[-1] < lay[0]
    assert lay[4 + _lib.X_H] + 2 * lay[3] * 256 <= lay[4 + _lib.X_PRE]
    assert lib.vmoe_moe_layout(100, 6, 3, 64, 96, 128, lay) == _lib.OK
    assert lay[4 + _lib.X_NSLOTS + _lib.M_NSLOTS] == 0   # E % 8 != 0: plain top-k
    assert lib.vmoe_moe_layout(100, 0, 2, 64, 96, 128, lay) == _lib.ERR_INVALID_ARG
    xl = (ctypes.c_int64 * (4 + _lib.X_NSLOTS))()
    assert lib.vmoe_expert_layout(128, 4, 2, 128, 64, 256, 1, xl) == _lib.OK
    assert lib.vmoe_expert_layout(128, 4, 2, 128, 64, 256, 0, xl) == _lib.OK
    assert lib.vmoe_expert_layout(-1, 4, 2, 128, 64, 256, 0, xl) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_moe_forward(1, 128, 4, 2, 1, 128, 1, 64, 1, 256, 1, 64, 1, 1, 64, 256,
                                1, 1, None, 1, 1, 64, 1, 1, 1, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_moe_forward(None, 0, 4, 2, 1, 128, None, 64, None, 256, None, 64, None,
                                None, 64, 256, None, None, None, None, None, 64, None, None,
                                None, None) == _lib.OK                    # no tokens
    # its logit gradient: both or neither index arrays, k above one wave
    assert lib.vmoe_router_weight_bwd(1, 8, 4, 8, 2, 1, 1, 1, 1, 2, 1, 8,
                                      None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_router_weight_bwd(1, 8, 4, 8, 2, 1, None, None, 1, 2, 1, 8,
                                      None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_router_weight_bwd(1, 128, 4, 128, 65, 1, 1, None, 1, 65, 1, 128,
                                      None) == _lib.ERR_UNSUPPORTED
    # token-major gather: top_k above one wave is rejected, unaligned widths unsupported
    assert lib.vmoe_gather_tokens(1, 8, 1, 4, 65, None, 1, 1, 8, 4, None, 8,
                                  None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gather_tokens(1, 12, 1, 4, 2, None, 1, 1, 12, 4, None, 12,
                                  None) == _lib.ERR_UNSUPPORTED
    # router: k > E is invalid, more than 2048 experts unsupported
    assert lib.vmoe_router_topk(1, 8, 4, 8, 9, 1, 1, 1, None, None, 1, 1, 1 << 20, None,
                                None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_router_topk(1, 4096, 4, 4096, 8, 1, 1, 1, None, None, 1, 1, 1 << 20, None,
                                None) == _lib.ERR_UNSUPPORTED
    assert lib.vmoe_router_topk(1, 8, 4, 8, 2, 1, 1, 1, None, None, 1, 1, 0, None,
                                None) == _lib.ERR_WORKSPACE
    assert lib.vmoe_router_partial_floats(16384, 64) % 65 == 0
    # top-k with the routing histograms: one workgroup per 1024-assignment
    # tile where the grouped kernel applies and k divides 1024, else 0
    assert lib.vmoe_router_topk_hist_blocks(16384, 64, 8) == 256    # 2 per tile
    assert lib.vmoe_router_topk_hist_blocks(32768, 128, 8) == 256   # 1 per tile
    assert lib.vmoe_router_topk_hist_blocks(8192, 8, 2) == 128      # 8 per tile
    assert lib.vmoe_router_topk_hist_blocks(1000, 64, 8) == 64
    assert lib.vmoe_router_topk_hist_blocks(262144, 128, 8) == 0   # over 65536 counts
    assert lib.vmoe_route_counted_workspace_bytes(16384, 64, 8) > \
        lib.vmoe_route_workspace_bytes(131072, 64)
    assert lib.vmoe_route_counted_workspace_bytes(16384, 64, 3) == 0
    assert lib.vmoe_router_topk_hist_blocks(16384, 64, 3) == 0
    assert lib.vmoe_router_topk_hist_blocks(16384, 12, 2) == 0
    assert lib.vmoe_router_topk_hist_blocks(16384, 256, 8) == 0
    assert lib.vmoe_router_topk_hist_blocks(0, 64, 8) == 0
    # (logits at 16, ld 64, 1000 tokens, 64 experts, k 8); unsupported shapes
    # launch nothing; short partial rows or routing workspace are refused
    hist = (16, 64, 1000, 64, 8, 1, 16, 16, None, None, 16, 16)
    assert lib.vmoe_router_topk_hist(16, 64, 1000, 64, 3, 1, 16, 16, None, None, 16, 16,
                                     1 << 20, None, 16, 1 << 20, None) == _lib.ERR_UNSUPPORTED
    assert lib.vmoe_router_topk_hist(*hist, 63 * 65, None, 16, 1 << 20,
                                     None) == _lib.ERR_WORKSPACE
    assert lib.vmoe_router_topk_hist(*hist, 64 * 65, None, 16, 64, None) == _lib.ERR_WORKSPACE
    assert lib.vmoe_router_topk_hist(*hist, 64 * 65, None, None, 1 << 20,
                                     None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_route_counted(None, 0, -1, 4, 1, 64, 0, None, None, None, None, None,
                                  None, None, 0, 0, None, None, None, None, None, None, None,
                                  0, None) == _lib.ERR_INVALID_ARG
    # counts the top-k launch cannot have written (k = 3) are unsupported
    assert lib.vmoe_route_counted(1, 0, 6, 64, 3, 64, 0, 1, 1, 1, 1, 1, 1, 1, 0, 512, 1, 1,
                                  None, None, None, None, 1, 1 << 20,
                                  None) == _lib.ERR_UNSUPPORTED
    # router logits: ld below the row is invalid; E % 8 != 0 is unsupported
    assert lib.vmoe_router_logits(1, 32, 4, 64, 1, 64, 8, 1, 8, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_router_logits(16, 256, 4, 256, 16, 256, 7, 8, 8, None) == _lib.ERR_UNSUPPORTED
    assert lib.vmoe_router_aux(None, 1, 4, 8, None, None, None, None, None, None, None, None,
                               None) == _lib.ERR_INVALID_ARG
    # unaligned hidden size is unsupported, not silently wrong
    assert lib.vmoe_gemm_up_fwd(None, 8, 0, None, None, 8, None, None, 8, 1, None, 1, 1, 1, 1,
                                4, 12, 16, 64, None) == _lib.ERR_UNSUPPORTED
    assert lib.vmoe_gemm_down_fwd(None, 8, None, 8, None, 8, None, None, None, None, 4, 16, 16,
                                  64, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_up_fwd(1, 8, 0, None, 1, 8, 1, None, 8, 5, None, 1, 1, 1, 1, 4, 16,
                                16, 64, None) == _lib.ERR_INVALID_ARG
    # dH row sums need pre_act and a row stride of at least ceil(max_width / 64)
    assert lib.vmoe_gemm_down_bwd_dh(1, 16, 4, None, None, 1, 16, None, None, 1, 128, 1, 1, 1,
                                     1, 4, 16, 128, 64, 1, 2, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_down_bwd_dh(1, 16, 4, None, None, 1, 16, 1, None, 1, 128, 1, 1, 1,
                                     1, 4, 16, 128, 64, 1, 1, None) == _lib.ERR_INVALID_ARG
    # a row-weight output without the weights it is read from
    assert lib.vmoe_route(1, 0, 4, 4, 1, 64, 0, 1, 1, 1, 1, 1, 1, 1, 0, 8, 1, 1, None, None,
                          None, 1, 1, 4096, None) == _lib.ERR_INVALID_ARG
    # fp32 GEMMs: bad activation, missing pre/up for the activation's rule,
    # leading dimensions below the row, no output at all
    assert lib.vmoe_gemm_f32_up_fwd(1, 16, 4, None, 1, 16, 1, None, None, 16, 3, 1, 1, 1, 1, 2,
                                    16, 16, 64, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_f32_up_fwd(1, 8, 4, None, 1, 16, 1, None, None, 16, 1, 1, 1, 1, 1, 2,
                                    16, 16, 64, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_f32_up_fwd(1, 16, 4, None, 1, 16, None, None, None, 16, 1, 1, 1, 1, 1,
                                    2, 16, 16, 64, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_f32_up_bwd_dx(1, None, None, 16, 1, 1, 16, 1, 16, 1, 1, 1, 1, 2, 16,
                                       16, 64, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_f32_up_bwd_dw(1, 16, 4, None, 1, 1, None, 16, 2, 1, 16, 1, 1, 1, 1, 2,
                                       16, 16, 64, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_f32_down_fwd(1, 16, 1, 8, 1, 16, 1, 1, 1, 1, 2, 16, 16, 64,
                                      None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_f32_down_bwd_dh(1, 16, 1, 16, 1, 8, 1, 1, 1, 1, 2, 16, 16, 64,
                                         None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_gemm_f32_down_bwd_dw(1, 16, 1, 16, 1, 16, None, 1, 1, 1, 2, 16, 16, 64,
                                         None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_f32_relu2_grad(1, 1, 8, 1, 16, 4, 16, None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_f32_relu2_grad(None, None, 16, None, 16, 0, 16, None) == _lib.OK
    # no rows: nothing to launch
    assert lib.vmoe_gemm_f32_down_fwd(1, 16, 1, 16, 1, 16, 1, 1, 1, 1, 2, 16, 16, 0,
                                      None) == _lib.OK


def test_check_maps_status_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_INVALID_ARG, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ERR_LAUNCH, "x")
    _lib.check(_lib.OK, "x")


def test_launch_timing_hook_arguments():
    """vmoe_set_launch_timing: a start event needs a stop event; NULL, NULL
    switches it off (no GPU call is made)."""
    lib = _lib.lib()
    assert lib.vmoe_set_launch_timing(ctypes.c_void_p(8), None) == _lib.ERR_INVALID_ARG
    assert lib.vmoe_set_launch_timing(None, None) == _lib.OK


def test_launch_timer_sees_every_call():
    """The observer hook (bench.py's per-launch timing) is called around each
    entry point, also when the call fails its argument checks."""

    class Rec:
        def __init__(self):
            self.log = []

        def begin(self, name):
            self.log.append(("begin", name))

        def end(self, name):
            self.log.append(("end", name))

    rec = Rec()
    _lib.set_launch_timer(rec)
    try:
        with pytest.raises(ValueError):
            _lib.call("vmoe_combine", None, 0, 0, None, None, 0, None, 8, 1, 8, None)
    finally:
        _lib.set_launch_timer(None)
    assert rec.log == [("begin", "vmoe_combine"), ("end", "vmoe_combine")]
