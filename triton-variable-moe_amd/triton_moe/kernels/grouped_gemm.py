"""Variable-width grouped GEMMs on gfx950 bf16 MFMA (csrc/gemm.hip).

Mirrors triton_moe/kernels/grouped_gemm.py of the reference:
precompute_gather_map (:104-149), grouped_gemm_up (:379-477),
grouped_gemm_down (:587-651), grouped_gemm_up_backward (:1166-1290),
grouped_gemm_down_backward (:1294-1390), GroupedGemmUp (:1393-1525),
GroupedGemmDown (:1528-1601), grouped_gemm_up_autograd (:1604-1639) and
grouped_gemm_down_autograd (:1642-1665): same signatures, output shapes,
zero-filled padding, saved tensors and gradient tuples.

Layouts are the reference's: W1 [hidden, total_width] with experts side by
side in columns, W2 [total_width, hidden] stacked in rows, intermediates
[total_tokens, max_expert_width] with expert e in columns [0, width_e).

The public functions read the small metadata arrays back once (the
reference does several .item() syncs) to size outputs and validate; the
RoutedMoEOp node used by the module takes a prebuilt GemmMeta and never
syncs: the kernels find their tiles on the device.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch
from torch.amp import custom_bwd, custom_fwd
from torch.autograd.function import once_differentiable

from .. import _lib
from .gather import row_maps

_ACTIVATIONS = {"none": _lib.ACT_NONE, "relu_squared": _lib.ACT_RELU_SQUARED}


ACT_SWIGLU = _lib.ACT_SWIGLU  # activation="swiglu" (vmoe_gemm_up_glu; fp32: VMOE_ACT_SWIGLU)


def _activation_code(activation: str) -> int:
    if activation == "swiglu":
        return ACT_SWIGLU
    return _ACTIVATIONS.get(activation, _lib.ACT_NONE)


@dataclass
class GemmMeta:
    """Expert metadata for one grouped GEMM call.

    eto/ewo [E+1], widths/tpe [E]: device int32. rows: row count of the
    padded buffers (sizes outputs and bounds row indices). full_rows: every
    row < rows is written by the row tiles. full_cols: the expert column
    ranges tile the weight matrix. uniform: every width equals max_width.
    """

    eto: torch.Tensor
    ewo: torch.Tensor
    widths: torch.Tensor
    tpe: torch.Tensor
    num_experts: int
    max_width: int
    rows: int
    full_rows: bool = True
    full_cols: bool = True
    uniform: bool = True


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.int32).contiguous()


def host_meta(eto, ewo, widths, tpe, max_width: int, hidden: int, rows: int | None,
              total_width: int | None, align8: bool = True) -> GemmMeta:
    """Validates caller metadata on the host (one device->host copy).
    align8: the bf16 kernels' rule that hidden, widths and offsets are
    multiples of 8 (the fp32 kernels have none, so their callers pass False)."""
    eto_d, ewo_d, w_d, tpe_d = _i32(eto), _i32(ewo), _i32(widths), _i32(tpe)
    E = w_d.numel()
    if E == 0:
        raise ValueError("expert_widths is empty")
    if eto_d.numel() < E + 1 or ewo_d.numel() < E + 1 or tpe_d.numel() < E:
        raise ValueError("expert metadata shorter than num_experts (+1)")
    host = torch.cat([eto_d[:E + 1], ewo_d[:E + 1], w_d, tpe_d[:E]]).cpu().tolist()
    h_eto, h_ewo = host[:E + 1], host[E + 1:2 * E + 2]
    h_w, h_tpe = host[2 * E + 2:3 * E + 2], host[3 * E + 2:]
    if rows is None:
        rows = h_eto[E]
    if align8 and (any(v % 8 for v in h_w) or any(v % 8 for v in h_ewo) or hidden % 8 or
                   max_width % 8):
        raise NotImplementedError(
            "hidden size, expert widths and weight offsets must be multiples of 8")
    if any(w < 0 or w > max_width for w in h_w):
        raise ValueError("expert width outside [0, max_expert_width]")
    if any(b < a for a, b in zip(h_eto, h_eto[1:])) or h_eto[0] < 0 or h_eto[E] > rows:
        raise ValueError("expert_token_offsets must be non-decreasing within [0, total_tokens]")
    if any(t < 0 for t in h_tpe):
        raise ValueError("tokens_per_expert must be non-negative")
    if any(o < 0 for o in h_ewo) or (total_width is not None and any(
            h_ewo[e] + h_w[e] > total_width or h_ewo[e + 1] > total_width for e in range(E))):
        raise ValueError("expert weight ranges exceed the weight matrix")
    if any(h_ewo[e + 1] - h_ewo[e] > max_width for e in range(E)):
        raise ValueError("expert weight range wider than max_expert_width")
    full_rows = h_eto[0] == 0 and h_eto[E] == rows and all(
        h_tpe[e] >= h_eto[e + 1] - h_eto[e] for e in range(E))
    full_cols = total_width is not None and h_ewo[0] == 0 and h_ewo[E] == total_width and all(
        h_ewo[e + 1] == h_ewo[e] + h_w[e] for e in range(E))
    uniform = all(w == max_width for w in h_w)
    return GemmMeta(eto_d, ewo_d, w_d, tpe_d, E, int(max_width), int(rows), full_rows,
                    full_cols, uniform)


def _bf16(t: torch.Tensor, what: str) -> torch.Tensor:
    """t as the bf16 GEMMs read it: unit column stride, rows 16-byte aligned
    (row stride a multiple of 8 elements, 16-byte aligned start). Any other
    view, such as a column slice, is copied into a fresh tensor."""
    if t.dtype != torch.bfloat16:
        raise NotImplementedError(f"{what}: only bfloat16 is supported (got {t.dtype})")
    if t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _token_source(g: torch.Tensor):
    """(tensor, leading dimension) of a bf16 [T, d] source read through a row
    map; a row-broadcast source (row stride 0, such as the gradient of
    out.sum()) is passed as its first row with leading dimension 0."""
    g = _bf16_any(g, "token source")
    if g.shape[0] > 0 and g.stride(0) == 0:
        row = g[:1] if g.stride(1) == 1 and g.data_ptr() % 16 == 0 else g[:1].contiguous()
        return row, 0
    g = _bf16(g, "token source")
    return g, g.stride(0)


def _bf16_any(t: torch.Tensor, what: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise NotImplementedError(f"{what}: only bfloat16 is supported (got {t.dtype})")
    return t


def _f32_rows(t: torch.Tensor | None, rows: int, what: str) -> torch.Tensor | None:
    if t is None:
        return None
    _need(t.dtype == torch.float32 and t.is_contiguous() and t.numel() >= rows,
          f"{what} must be contiguous fp32 with one entry per row")
    return t


def _alloc(rows, cols, like, zero):
    f = torch.zeros if zero else torch.empty
    return f(rows, cols, dtype=like.dtype, device=like.device)


def _meta_args(m: GemmMeta):
    return (m.eto.data_ptr(), m.ewo.data_ptr(), m.widths.data_ptr(), m.tpe.data_ptr(),
            m.num_experts)


_DW_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _dw_workspace(m: GemmMeta, hidden: int, device) -> torch.Tensor:
    """Split-K workspace of the dW GEMMs. Its arrival words must be zero when
    a launch starts, and every launch leaves them zero, so one zero-filled
    buffer per (device, stream) is kept and reused: calls on one stream run
    in order, and calls on different streams get different buffers."""
    return _dw_workspace_bytes(m.num_experts, hidden, m.max_width, m.rows, device,
                               _lib.stream(device))


def _dw_workspace_bytes(E: int, hidden: int, max_width: int, rows: int, device,
                        stream: int) -> torch.Tensor:
    """_dw_workspace for the dW GEMMs launched on the raw stream handle `stream`."""
    n = max(int(_lib.lib().vmoe_gemm_dw_workspace_bytes(E, hidden, max_width,
                                                        max(rows, 1))), 16)
    device = torch.device(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _DW_WORKSPACES.get(key)
    if ws is None or ws.numel() < n:
        # Only the arrival words at the start must be zero (the partial tiles
        # need no initial value); zero_() is a fill kernel, so this also holds
        # under graph capture, where a workspace made during the capture is
        # cleared again at every replay (8 KiB, not the whole 64 MiB).
        ws = torch.empty(n, dtype=torch.uint8, device=device)
        ws[:min(n, int(_lib.lib().vmoe_gemm_dw_workspace_zero_bytes()))].zero_()
        _DW_WORKSPACES[key] = ws
    return ws


def _zero_tails(buf: torch.Tensor, m: GemmMeta):
    if m.uniform or buf.shape[0] == 0:
        return
    _lib.call("vmoe_zero_tail_cols", buf.data_ptr(), buf.stride(0), m.eto.data_ptr(),
              m.widths.data_ptr(), m.num_experts, m.max_width, buf.shape[0],
              _lib.stream(buf.device))


# ---------------------------------------------------------------------------
# Launchers (no host sync; shapes come from GemmMeta)
# ---------------------------------------------------------------------------


def up_fwd(x, w1, m: GemmMeta, act: int, save_pre: bool, zero_tails: bool,
           gather_map: torch.Tensor | None = None, row_scale: torch.Tensor | None = None):
    """out = act(x_e @ W1_e) and pre_act = relu(z) (or zeros for act none).
    With row_scale (fp32 per row) out[row] = bf16(row_scale[row] * act(z))."""
    x = _bf16(x, "grouped_gemm_up x")
    w1 = _bf16(w1, "grouped_gemm_up w1")
    hidden = x.shape[1]
    _need(w1.shape[0] == hidden, "w1 rows must equal the hidden size of x")
    if gather_map is None:
        _need(x.shape[0] >= m.rows, "x has fewer rows than expert_token_offsets[-1]")
    else:
        _need(gather_map.numel() >= m.rows, "gather_map shorter than the padded row count")
    out = _alloc(m.rows, m.max_width, x, not m.full_rows)
    pre = None
    if save_pre:
        pre = _alloc(m.rows, m.max_width, x, not m.full_rows or act == _lib.ACT_NONE)
    gm = None if gather_map is None else _i32(gather_map)
    if m.rows > 0:
        _lib.call("vmoe_gemm_up_fwd", x.data_ptr(), x.stride(0), x.shape[0], _lib.ptr(gm),
                  w1.data_ptr(), w1.stride(0),
                  out.data_ptr(), _lib.ptr(pre) if act == _lib.ACT_RELU_SQUARED else None,
                  out.stride(0), act, _lib.ptr(_f32_rows(row_scale, m.rows, "row_scale")),
                  *_meta_args(m), hidden, m.max_width, m.rows, _lib.stream(x.device))
        if zero_tails:
            _zero_tails(out, m)
            if pre is not None and act == _lib.ACT_RELU_SQUARED:
                _zero_tails(pre, m)
    return out, pre


def down_fwd(h, w2, m: GemmMeta, hidden: int, out: torch.Tensor | None = None):
    """Y_e = H_e @ W2_e; out (nullable): a [rows, hidden] bf16 view to write
    Y into (the rows the experts cover are written)."""
    h = _bf16(h, "grouped_gemm_down intermediate")
    w2 = _bf16(w2, "grouped_gemm_down w2")
    _need(w2.shape[1] == hidden, "w2 columns must equal hidden_size")
    _need(h.shape[0] >= m.rows and h.shape[1] >= m.max_width,
          "intermediate smaller than [rows, max_expert_width]")
    if out is not None:
        _need(out.dtype == torch.bfloat16 and out.stride(1) == 1 and out.shape[0] >= m.rows and
              out.shape[1] == hidden, "out must be bf16 [rows, hidden]")
    y = out if out is not None else _alloc(m.rows, hidden, h, not m.full_rows)
    if m.rows > 0:
        _lib.call("vmoe_gemm_down_fwd", h.data_ptr(), h.stride(0), w2.data_ptr(), w2.stride(0),
                  y.data_ptr(), y.stride(0), *_meta_args(m), hidden, m.max_width, m.rows,
                  _lib.stream(h.device))
    return y


def _same_ld(a, b):
    if b is None or a.stride(0) == b.stride(0):
        return a, b
    return a.contiguous(), b.contiguous()


def relu2_grad(grad_h: torch.Tensor, pre: torch.Tensor) -> torch.Tensor:
    """GA = bf16(pre > 0 ? 2 * grad_h * pre : 0), elementwise (vmoe_relu2_grad)."""
    grad_h, pre = _same_ld(grad_h, pre)
    ga = torch.empty(grad_h.shape, dtype=grad_h.dtype, device=grad_h.device)
    _lib.call("vmoe_relu2_grad", grad_h.data_ptr(), pre.data_ptr(), grad_h.stride(0),
              ga.data_ptr(), ga.stride(0), grad_h.shape[0], grad_h.shape[1],
              _lib.stream(grad_h.device))
    return ga


def up_bwd_dx(ga, w1, m: GemmMeta, hidden: int, out: torch.Tensor | None = None):
    """grad_x in gathered rows = GA_e @ W1_e^T, from GA, the gradient w.r.t. the
    up projection's pre-activation; out as for down_fwd."""
    ga = _bf16(ga, "grouped_gemm_up_backward grad_output")
    w1 = _bf16(w1, "grouped_gemm_up_backward w1")
    _need(w1.shape[0] == hidden, "w1 does not match hidden_size")
    _need(ga.shape[0] >= m.rows and ga.shape[1] >= m.max_width,
          "grad_output smaller than [rows, max_expert_width]")
    if out is not None:
        _need(out.dtype == torch.bfloat16 and out.stride(1) == 1 and out.shape[0] >= m.rows and
              out.shape[1] == hidden, "out must be bf16 [rows, hidden]")
    grad_x = out if out is not None else _alloc(m.rows, hidden, ga, not m.full_rows)
    if m.rows > 0:
        _lib.call("vmoe_gemm_up_bwd_dx", ga.data_ptr(), ga.stride(0), w1.data_ptr(),
                  w1.stride(0), grad_x.data_ptr(), grad_x.stride(0), *_meta_args(m), hidden,
                  m.max_width, m.rows, _lib.stream(ga.device))
    return grad_x


def up_bwd_dw(ga, x, w1, m: GemmMeta, hidden: int, gather_map: torch.Tensor | None,
              out: torch.Tensor | None = None):
    """grad_w1 = X_e^T @ GA_e, X_e read through gather_map when given; out
    (nullable): a tensor like w1 whose experts' columns are written."""
    ga = _bf16(ga, "grouped_gemm_up_backward grad_output")
    x = _bf16(x, "grouped_gemm_up_backward x")
    w1 = _bf16(w1, "grouped_gemm_up_backward w1")
    _need(w1.shape[0] == hidden and x.shape[1] == hidden, "x / w1 do not match hidden_size")
    if gather_map is None:
        _need(x.shape[0] >= m.rows, "x has fewer rows than expert_token_offsets[-1]")
    else:
        _need(gather_map.numel() >= m.rows, "gather_map shorter than the padded row count")
    if out is not None:
        _need(out.shape == w1.shape and out.dtype == w1.dtype and out.stride() == w1.stride(),
              "out must be laid out like w1")
        grad_w1 = out
    else:
        grad_w1 = torch.zeros_like(w1) if not m.full_cols else torch.empty_like(w1)
    if m.rows == 0:  # no routed rows: zero gradients, no launch
        return grad_w1.zero_()
    dev = ga.device
    gm = None if gather_map is None else _i32(gather_map)
    ws = _dw_workspace(m, hidden, dev)
    _lib.call("vmoe_gemm_up_bwd_dw", x.data_ptr(), x.stride(0), x.shape[0], _lib.ptr(gm),
              ga.data_ptr(), ga.stride(0), grad_w1.data_ptr(), grad_w1.stride(0),
              *_meta_args(m), hidden, m.max_width, m.rows, ws.data_ptr(), ws.numel(),
              _lib.stream(dev))
    return grad_w1


def up_bwd_from_ga(ga, x, w1, m: GemmMeta, hidden: int, gather_map: torch.Tensor | None):
    """(grad_x in gathered rows, grad_w1) from GA, the gradient w.r.t. the
    up projection's pre-activation."""
    _need(x.shape[1] == hidden, "x / w1 do not match hidden_size")
    grad_x = up_bwd_dx(ga, w1, m, hidden)
    return grad_x, up_bwd_dw(ga, x, w1, m, hidden, gather_map)


def up_bwd(grad_h, x, w1, pre, m: GemmMeta, hidden: int, act: int,
           gather_map: torch.Tensor | None):
    """(grad_x in gathered rows, grad_w1) from the gradient of the activated output."""
    grad_h = _bf16(grad_h, "grouped_gemm_up_backward grad_output")
    if act == _lib.ACT_RELU_SQUARED:
        pre = _bf16(pre, "grouped_gemm_up_backward pre_act")
        _need(pre.shape == grad_h.shape, "pre_act and grad_output shapes differ")
        ga = relu2_grad(grad_h, pre)
    else:
        ga = grad_h
    return up_bwd_from_ga(ga, x, w1, m, hidden, gather_map)


_ONES_ROWS: dict[tuple[str, int], torch.Tensor] = {}


def _ones_row(d: int, device) -> torch.Tensor:
    key = (str(device), d)
    row = _ONES_ROWS.get(key)
    if row is None:
        row = _ONES_ROWS[key] = torch.ones(1, d, dtype=torch.bfloat16, device=device)
    return row


def _grad_source(grad_y, m: GemmMeta, gather_map):
    """(tensor, leading dimension, rows, scale) of the output-gradient operand.
    Read through a row map, a broadcast scalar c (both strides 0: the gradient
    of out.sum() or out.mean()) becomes a row of ones with ld 0 and the scale
    c, which the GEMM applies to its output; scale is None otherwise."""
    gy_rows = grad_y.shape[0]
    if gather_map is None:
        grad_y = _bf16(grad_y, "grouped_gemm_down_backward grad_output")
        _need(gy_rows >= m.rows, "grad_output has fewer rows than the padded row count")
        return grad_y, grad_y.stride(0), gy_rows, None
    _need(gather_map.numel() >= m.rows, "gather_map shorter than the padded row count")
    if (grad_y.dtype == torch.bfloat16 and gy_rows > 0 and grad_y.stride(0) == 0 and
            grad_y.stride(1) == 0):
        return _ones_row(grad_y.shape[1], grad_y.device), 0, gy_rows, grad_y
    g, ld = _token_source(grad_y)
    return g, ld, gy_rows, None


def down_bwd_dh(grad_y, w2, m: GemmMeta, hidden: int, zero_tails: bool,
                pre: torch.Tensor | None = None, gather_map: torch.Tensor | None = None,
                row_scale: torch.Tensor | None = None, row_dot: torch.Tensor | None = None):
    """grad_intermediate [rows, max_width] = grad_y_e @ W2_e^T; with pre, the
    relu^2 gradient GA instead (fused in the epilogue). With gather_map,
    grad_y holds one row per token and row r is grad_y[gather_map[r]] (-1:
    zeros); with row_scale (fp32 per row) the gradient w.r.t. H is scaled by
    it before the relu^2 rule. row_dot (fp32 [rows, ceil(max_width / 64)],
    needs pre) receives per 64-column block the sums of GH * pre^2."""
    g, ldg, g_rows, gs = _grad_source(grad_y, m, gather_map)
    w2 = _bf16(w2, "grouped_gemm_down_backward w2")
    _need(w2.shape[1] == hidden and g.shape[1] == hidden,
          "grad_output / w2 do not match hidden_size")
    grad_h = _alloc(m.rows, m.max_width, g, not m.full_rows)
    if pre is not None:
        pre = _bf16(pre, "pre_act")
        _need(pre.shape[0] >= m.rows and pre.stride(0) == grad_h.stride(0),
              "pre_act must match the [rows, max_expert_width] layout")
    gm = None if gather_map is None else _i32(gather_map)
    if row_dot is not None:
        _need(pre is not None and row_dot.dtype == torch.float32 and row_dot.stride(1) == 1
              and row_dot.shape[0] >= m.rows and row_dot.shape[1] >= (m.max_width + 63) // 64,
              "row_dot must be fp32 [rows, ceil(max_width / 64)] and needs pre_act")
    if m.rows > 0:
        _lib.call("vmoe_gemm_down_bwd_dh", g.data_ptr(), ldg, g_rows, _lib.ptr(gm),
                  _lib.ptr(gs), w2.data_ptr(), w2.stride(0), _lib.ptr(pre),
                  _lib.ptr(_f32_rows(row_scale, m.rows, "row_scale")), grad_h.data_ptr(),
                  grad_h.stride(0), *_meta_args(m), hidden, m.max_width, m.rows,
                  _lib.ptr(row_dot), 0 if row_dot is None else row_dot.stride(0),
                  _lib.stream(g.device))
        if zero_tails:
            _zero_tails(grad_h, m)
    return grad_h


def down_bwd_dw(grad_y, h, w2, m: GemmMeta, hidden: int,
                gather_map: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """grad_w2 = H_e^T @ grad_y_e (grad_y through gather_map when given); out
    (nullable): a tensor like w2 whose experts' rows are written."""
    g, ldg, g_rows, gs = _grad_source(grad_y, m, gather_map)
    h = _bf16(h, "grouped_gemm_down_backward intermediate")
    w2 = _bf16(w2, "grouped_gemm_down_backward w2")
    _need(w2.shape[1] == hidden and g.shape[1] == hidden,
          "grad_output / w2 do not match hidden_size")
    _need(h.shape[0] >= m.rows and h.shape[1] >= m.max_width,
          "intermediate smaller than [rows, max_expert_width]")
    if out is not None:
        _need(out.shape == w2.shape and out.dtype == w2.dtype and out.stride() == w2.stride(),
              "out must be laid out like w2")
        grad_w2 = out
    else:
        grad_w2 = torch.zeros_like(w2) if not m.full_cols else torch.empty_like(w2)
    if m.rows == 0:  # no routed rows: zero gradients, no launch
        return grad_w2.zero_()
    gm = None if gather_map is None else _i32(gather_map)
    dev = g.device
    ws = _dw_workspace(m, hidden, dev)
    _lib.call("vmoe_gemm_down_bwd_dw", h.data_ptr(), h.stride(0), g.data_ptr(), ldg, g_rows,
              _lib.ptr(gm), _lib.ptr(gs), grad_w2.data_ptr(), grad_w2.stride(0), *_meta_args(m), hidden,
              m.max_width, m.rows, ws.data_ptr(), ws.numel(), _lib.stream(dev))
    return grad_w2


def down_bwd(grad_y, h, w2, m: GemmMeta, hidden: int, zero_tails: bool,
             pre: torch.Tensor | None = None, gather_map: torch.Tensor | None = None,
             row_scale: torch.Tensor | None = None):
    """(grad_intermediate [rows, max_width], grad_w2): down_bwd_dh then
    down_bwd_dw."""
    grad_h = down_bwd_dh(grad_y, w2, m, hidden, zero_tails, pre, gather_map, row_scale)
    return grad_h, down_bwd_dw(grad_y, h, w2, m, hidden, gather_map)


# ---------------------------------------------------------------------------
# fp32 path: float32 weights (the reference's kernels are dtype-generic and
# its autograd tests run fp32, tests/test_grouped_gemm_backward.py:151-208).
# One fp32 VALU kernel per GEMM form (csrc/gemm_f32.hip); outputs are fp32
# and zero outside the rows and columns the experts cover.
# ---------------------------------------------------------------------------


def _is_f32(w: torch.Tensor) -> bool:
    return w.dtype == torch.float32


def _f32(t: torch.Tensor, what: str) -> torch.Tensor:
    """A float32 operand with unit column stride (bf16 inputs are widened,
    as the reference's autograd casts x to the weights' dtype)."""
    if t.dtype == torch.bfloat16:
        t = t.float()
    if t.dtype != torch.float32:
        raise NotImplementedError(f"{what}: expected float32 with float32 weights (got {t.dtype})")
    ok = t.dim() == 2 and t.stride(-1) == 1 and t.stride(0) >= max(t.shape[1], 1)
    return t if ok else t.contiguous()


def _f32_zeros(rows, cols, device):
    return torch.zeros(rows, cols, dtype=torch.float32, device=device)


def f32_up_fwd(x, w1, m: GemmMeta, act: int, gather_map=None, want_out=True, want_pre=False,
               want_up=False):
    """(out, pre, up) of the up projection in fp32: relu^2 pre = relu(z);
    SwiGLU (m = GluMeta.fwd) pre = gate, up = u; tensors not asked for are None."""
    x = _f32(x, "grouped_gemm_up x")
    w1 = _f32(w1, "grouped_gemm_up w1")
    hidden = x.shape[1]
    _need(w1.shape[0] == hidden, "w1 rows must equal the hidden size of x")
    if gather_map is None:
        _need(x.shape[0] >= m.rows, "x has fewer rows than expert_token_offsets[-1]")
    else:
        _need(gather_map.numel() >= m.rows, "gather_map shorter than the padded row count")
    dev = x.device
    out = _f32_zeros(m.rows, m.max_width, dev) if want_out else None
    pre = _f32_zeros(m.rows, m.max_width, dev) if want_pre else None
    up = _f32_zeros(m.rows, m.max_width, dev) if want_up and act == ACT_SWIGLU else None
    gm = None if gather_map is None else _i32(gather_map)
    if m.rows > 0:
        _lib.call("vmoe_gemm_f32_up_fwd", x.data_ptr(), x.stride(0), x.shape[0], _lib.ptr(gm),
                  w1.data_ptr(), w1.stride(0), _lib.ptr(out),
                  _lib.ptr(pre) if act != _lib.ACT_NONE else None, _lib.ptr(up), m.max_width,
                  act, *_meta_args(m), hidden, m.max_width, m.rows, _lib.stream(dev))
    return out, pre, up


def f32_down_fwd(h, w2, m: GemmMeta, hidden: int):
    h = _f32(h, "grouped_gemm_down intermediate")
    w2 = _f32(w2, "grouped_gemm_down w2")
    _need(w2.shape[1] == hidden, "w2 columns must equal hidden_size")
    _need(h.shape[0] >= m.rows and h.shape[1] >= m.max_width,
          "intermediate smaller than [rows, max_expert_width]")
    y = _f32_zeros(m.rows, hidden, h.device)
    if m.rows > 0:
        _lib.call("vmoe_gemm_f32_down_fwd", h.data_ptr(), h.stride(0), w2.data_ptr(),
                  w2.stride(0), y.data_ptr(), y.stride(0), *_meta_args(m), hidden, m.max_width,
                  m.rows, _lib.stream(h.device))
    return y


def f32_up_bwd(grad_h, x, w1, pre, up, m: GemmMeta, hidden: int, act: int, gather_map=None):
    """(grad_x in gathered rows, grad_w1) in fp32 from the gradient of the
    activated output; pre is relu(z) (relu^2) or the gate (SwiGLU, with up)."""
    grad_h = _f32(grad_h, "grouped_gemm_up_backward grad_output").contiguous()
    x = _f32(x, "grouped_gemm_up_backward x")
    w1 = _f32(w1, "grouped_gemm_up_backward w1")
    _need(w1.shape[0] == hidden and x.shape[1] == hidden, "x / w1 do not match hidden_size")
    _need(grad_h.shape[0] >= m.rows and grad_h.shape[1] >= m.max_width,
          "grad_output smaller than [rows, max_expert_width]")
    ops = [grad_h]
    for t, what, needed in ((pre, "pre_act", act != _lib.ACT_NONE),
                            (up, "up", act == ACT_SWIGLU)):
        if not needed:
            ops.append(None)
            continue
        _need(t is not None, f"grouped_gemm_up_backward needs {what}")
        t = _f32(t, f"grouped_gemm_up_backward {what}").contiguous()
        _need(t.shape == grad_h.shape, f"{what} and grad_output shapes differ")
        ops.append(t)
    if gather_map is None:
        _need(x.shape[0] >= m.rows, "x has fewer rows than expert_token_offsets[-1]")
    else:
        _need(gather_map.numel() >= m.rows, "gather_map shorter than the padded row count")
    dev = grad_h.device
    grad_x = _f32_zeros(m.rows, hidden, dev)
    grad_w1 = torch.zeros(w1.shape, dtype=torch.float32, device=dev)
    gm = None if gather_map is None else _i32(gather_map)
    g, p_, u = ops
    if act == _lib.ACT_RELU_SQUARED and g.numel() > 0:
        # GA formed once; both GEMMs then read it as a plain operand
        ga = torch.empty_like(g)
        _lib.call("vmoe_f32_relu2_grad", g.data_ptr(), p_.data_ptr(), g.stride(0), ga.data_ptr(),
                  ga.stride(0), g.shape[0], g.shape[1], _lib.stream(dev))
        g, p_, act = ga, None, _lib.ACT_NONE
    if m.rows > 0:
        _lib.call("vmoe_gemm_f32_up_bwd_dx", g.data_ptr(), _lib.ptr(p_), _lib.ptr(u),
                  g.stride(0), act, w1.data_ptr(), w1.stride(0), grad_x.data_ptr(),
                  grad_x.stride(0), *_meta_args(m), hidden, m.max_width, m.rows,
                  _lib.stream(dev))
        _lib.call("vmoe_gemm_f32_up_bwd_dw", x.data_ptr(), x.stride(0), x.shape[0],
                  _lib.ptr(gm), g.data_ptr(), _lib.ptr(p_), _lib.ptr(u), g.stride(0), act,
                  grad_w1.data_ptr(), grad_w1.stride(0), *_meta_args(m), hidden, m.max_width,
                  m.rows, _lib.stream(dev))
    return grad_x, grad_w1


def f32_down_bwd(grad_y, h, w2, m: GemmMeta, hidden: int):
    """(grad_intermediate [rows, max_width], grad_w2) in fp32."""
    grad_y = _f32(grad_y, "grouped_gemm_down_backward grad_output")
    h = _f32(h, "grouped_gemm_down_backward intermediate")
    w2 = _f32(w2, "grouped_gemm_down_backward w2")
    _need(w2.shape[1] == hidden and grad_y.shape[1] == hidden,
          "grad_output / w2 do not match hidden_size")
    _need(grad_y.shape[0] >= m.rows, "grad_output has fewer rows than the padded row count")
    _need(h.shape[0] >= m.rows and h.shape[1] >= m.max_width,
          "intermediate smaller than [rows, max_expert_width]")
    dev = grad_y.device
    grad_h = _f32_zeros(m.rows, m.max_width, dev)
    grad_w2 = torch.zeros(w2.shape, dtype=torch.float32, device=dev)
    if m.rows > 0:
        _lib.call("vmoe_gemm_f32_down_bwd_dh", grad_y.data_ptr(), grad_y.stride(0),
                  w2.data_ptr(), w2.stride(0), grad_h.data_ptr(), grad_h.stride(0),
                  *_meta_args(m), hidden, m.max_width, m.rows, _lib.stream(dev))
        _lib.call("vmoe_gemm_f32_down_bwd_dw", h.data_ptr(), h.stride(0), grad_y.data_ptr(),
                  grad_y.stride(0), grad_w2.data_ptr(), grad_w2.stride(0), *_meta_args(m),
                  hidden, m.max_width, m.rows, _lib.stream(dev))
    return grad_h, grad_w2


# ---------------------------------------------------------------------------
# Public API (reference signatures)
# ---------------------------------------------------------------------------


@torch.compiler.disable
def precompute_gather_map(indices, bin_ids, bins, padded_bins, top_k):
    """[padded_bins[-1]] int32 map from gathered row to original token row (0 on pad rows)."""
    _lib.require_gpu(indices)
    total_padded = int(padded_bins[-1].item())
    _, gm, _ = row_maps(indices, bin_ids, bins, padded_bins, top_k, total_padded, 0,
                        want_row_src=False, want_gather_map=True)
    return gm


# ---------------------------------------------------------------------------
# SwiGLU: expert e's gate columns are W1[:, ewo_e : ewo_e + w_e] and its up
# columns W1[:, ewo_e + w_e : ewo_e + 2 w_e] (the reference's layout,
# grouped_gemm.py:295-297). The forward is one grouped GEMM whose epilogue
# forms H = bf16(silu(g) u) from the fp32 accumulators (vmoe_gemm_up_glu);
# the backward writes [dG | dU] per expert row (vmoe_glu_grad), the
# gradient of the expert's 2 w_e W1 columns, so grad_x and grad_w1 are one
# dX and one dW GEMM over widths 2 w_e.
# ---------------------------------------------------------------------------


@dataclass
class GluMeta:
    """fwd: the forward's metadata (widths w_e, gate columns at ewo_e);
    bwd: the backward GEMMs' (widths 2 w_e over contiguous column ranges);
    cols: W1 columns of those ranges when W1's own expert ranges are not
    contiguous (None: bwd addresses W1 directly)."""

    fwd: GemmMeta
    bwd: GemmMeta
    cols: torch.Tensor | None


def glu_meta(eto, ewo, widths, tpe, max_width: int, hidden: int, w1_cols: int,
             align8: bool = True) -> GluMeta:
    """Validates swiglu metadata on the host (one device->host copy); align8
    as for host_meta."""
    E = int(torch.as_tensor(widths).numel())
    if E == 0:
        raise ValueError("expert_widths is empty")
    eto_d, ewo_d, w_d, tpe_d = _i32(eto), _i32(ewo), _i32(widths), _i32(tpe)
    if eto_d.numel() < E + 1 or ewo_d.numel() < E + 1 or tpe_d.numel() < E:
        raise ValueError("expert metadata shorter than num_experts (+1)")
    h_ewo = ewo_d[:E + 1].cpu().tolist()
    h_w = w_d[:E].cpu().tolist()
    if any(w < 0 or o < 0 or o + 2 * w > w1_cols for o, w in zip(h_ewo, h_w)):
        raise ValueError("swiglu: expert gate/up columns exceed the weight matrix")
    # The forward reads only ewo_e (gate) and ewo_e + w_e (up) of each
    # expert; rows, widths and alignment are checked as for any grouped GEMM
    # (widths 2 w_e over a contiguous stand-in column layout).
    cum = [0]
    for w in h_w:
        cum.append(cum[-1] + 2 * w)
    cum_d = torch.tensor(cum, dtype=torch.int32, device=w_d.device)
    if align8 and any(o % 8 for o in h_ewo):
        raise NotImplementedError("expert weight offsets must be multiples of 8")
    chk = host_meta(eto_d, cum_d, w_d * 2, tpe_d, 2 * int(max_width), hidden, None, cum[-1],
                    align8)
    if any(w > max_width for w in h_w):
        raise ValueError("expert width outside [0, max_expert_width]")
    fwd = GemmMeta(eto_d, ewo_d, w_d, tpe_d, E, int(max_width), chk.rows, chk.full_rows, False,
                   all(w == max_width for w in h_w))
    contiguous = all(h_ewo[e + 1] == h_ewo[e] + 2 * h_w[e] for e in range(E))
    cols = None
    dev = w_d.device
    if contiguous:
        bwd = host_meta(eto_d, ewo_d, w_d * 2, tpe_d, 2 * int(max_width), hidden, None, w1_cols,
                        align8)
    else:
        cols = torch.cat([torch.arange(o, o + 2 * w) for o, w in zip(h_ewo, h_w)]).to(dev)
        bwd = chk
    return GluMeta(fwd, bwd, cols)


def glu_fwd(x, w1, m: GemmMeta, want_h: bool, want_gate: bool, want_up: bool,
            gather_map=None):
    """(H, gate, up) of the swiglu up projection, each [rows, max_width] with
    zero column tails (None where not wanted)."""
    x = _bf16(x, "grouped_gemm_up x")
    w1 = _bf16(w1, "grouped_gemm_up w1")
    hidden = x.shape[1]
    _need(w1.shape[0] == hidden, "w1 rows must equal the hidden size of x")
    if gather_map is None:
        _need(x.shape[0] >= m.rows, "x has fewer rows than expert_token_offsets[-1]")
    else:
        _need(gather_map.numel() >= m.rows, "gather_map shorter than the padded row count")
    outs = [_alloc(m.rows, m.max_width, x, not m.full_rows) if want else None
            for want in (want_h, want_gate, want_up)]
    gm = None if gather_map is None else _i32(gather_map)
    if m.rows > 0:
        _lib.call("vmoe_gemm_up_glu", x.data_ptr(), x.stride(0), x.shape[0], _lib.ptr(gm),
                  w1.data_ptr(), w1.stride(0), *(_lib.ptr(o) for o in outs), m.max_width, None,
                  *_meta_args(m), hidden, m.max_width, m.rows, _lib.stream(x.device))
        for o in outs:
            if o is not None:
                _zero_tails(o, m)
    return tuple(outs)


def glu_bwd(grad_h, x, w1, gate, up, gm_: GluMeta, hidden: int, gather_map=None):
    """(grad_x in gathered rows, grad_w1 in W1's gate/up layout)."""
    w1 = _bf16(w1, "grouped_gemm_up_backward w1")
    grad_h = _bf16(grad_h, "grouped_gemm_up_backward grad_output")
    m = gm_.fwd
    _need(grad_h.shape == gate.shape == up.shape, "grad_output and pre_act shapes differ")
    _need(grad_h.shape[0] >= m.rows and grad_h.shape[1] >= m.max_width,
          "grad_output smaller than [rows, max_expert_width]")
    ggu = torch.empty(m.rows, 2 * m.max_width, dtype=torch.bfloat16, device=grad_h.device)
    if m.rows > 0:
        gate, up = _same_ld(gate, up)
        _lib.call("vmoe_glu_grad", grad_h.data_ptr(), grad_h.stride(0), gate.data_ptr(),
                  up.data_ptr(), gate.stride(0), ggu.data_ptr(), ggu.stride(0),
                  m.eto.data_ptr(), m.widths.data_ptr(), m.tpe.data_ptr(), m.num_experts,
                  m.rows, m.max_width, _lib.stream(grad_h.device))
    wb = w1 if gm_.cols is None else w1.index_select(1, gm_.cols)
    grad_x = up_bwd_dx(ggu, wb, gm_.bwd, hidden)
    gw = up_bwd_dw(ggu, x, wb, gm_.bwd, hidden, gather_map)
    if gm_.cols is None:
        return grad_x, gw
    grad_w1 = torch.zeros_like(w1)
    grad_w1.index_copy_(1, gm_.cols, gw)
    return grad_x, grad_w1


@torch.compiler.disable
def grouped_gemm_up(x, w1, expert_token_offsets, expert_weight_offsets, expert_widths,
                    tokens_per_expert, max_expert_width, activation="relu_squared",
                    save_pre_act=False, gather_map=None):
    """Grouped up-projection with fused activation.

    Returns [total_tokens, max_expert_width] (and pre_act if save_pre_act),
    total_tokens = expert_token_offsets[-1]; columns >= width_e are zero.
    """
    _lib.require_gpu(x)
    act = _activation_code(activation)
    if act == ACT_SWIGLU:
        gmeta = glu_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                         tokens_per_expert, int(max_expert_width), x.shape[1], w1.shape[1],
                         align8=not _is_f32(w1))
        # pre_act is the gate, as the reference saves it (grouped_gemm.py:339-346)
        if _is_f32(w1):
            h, g, _ = f32_up_fwd(x, w1, gmeta.fwd, act, gather_map, want_pre=save_pre_act)
        else:
            h, g, _ = glu_fwd(x, w1, gmeta.fwd, True, save_pre_act, False, gather_map)
        return (h, g) if save_pre_act else h
    m = host_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                  tokens_per_expert, int(max_expert_width), x.shape[1], None, w1.shape[1],
                  align8=not _is_f32(w1))
    if _is_f32(w1):
        out, pre, _ = f32_up_fwd(x, w1, m, act, gather_map, want_pre=save_pre_act)
        return (out, pre) if save_pre_act else out
    # With gather_map, rows are read as x[gather_map[row]] inside the kernel
    # (the reference's USE_GATHER_MAP path, grouped_gemm.py:289-292).
    out, pre = up_fwd(x, w1, m, act, save_pre_act, zero_tails=True, gather_map=gather_map)
    if save_pre_act:
        return out, pre
    return out


@torch.compiler.disable
def grouped_gemm_down(intermediate, w2, expert_token_offsets, expert_weight_offsets,
                      expert_widths, tokens_per_expert, hidden_size):
    """Grouped down-projection: [total_tokens, hidden_size], total_tokens = intermediate rows."""
    _lib.require_gpu(intermediate)
    m = host_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                  tokens_per_expert, intermediate.shape[1], int(hidden_size),
                  intermediate.shape[0], w2.shape[0],
                  align8=not _is_f32(w2))
    if _is_f32(w2):
        return f32_down_fwd(intermediate, w2, m, int(hidden_size))
    return down_fwd(intermediate, w2, m, int(hidden_size))


@torch.compiler.disable
def grouped_gemm_up_backward(grad_output, x, w1, pre_act, expert_token_offsets,
                             expert_weight_offsets, expert_widths, tokens_per_expert,
                             hidden_size, activation="relu_squared", gather_map=None):
    """(grad_x [total_tokens, hidden] in gathered space, grad_w1 like w1)."""
    _lib.require_gpu(grad_output)
    act = _activation_code(activation)
    if act == ACT_SWIGLU:
        # pre_act holds the gate; the up half is recomputed from x (the
        # reference keeps only the gate and leaves this backward unfinished,
        # grouped_gemm.py:768-790).
        gmeta = glu_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                         tokens_per_expert, grad_output.shape[1], int(hidden_size), w1.shape[1],
                         align8=not _is_f32(w1))
        if _is_f32(w1):
            _, _, up = f32_up_fwd(x, w1, gmeta.fwd, act, gather_map, want_out=False,
                                  want_up=True)
            return f32_up_bwd(grad_output, x, w1, pre_act, up, gmeta.fwd, int(hidden_size), act,
                              gather_map)
        _, _, up = glu_fwd(x, w1, gmeta.fwd, False, False, True, gather_map)
        gate = _bf16(pre_act, "grouped_gemm_up_backward pre_act")
        return glu_bwd(grad_output, x, w1, gate, up, gmeta, int(hidden_size), gather_map)
    m = host_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                  tokens_per_expert, grad_output.shape[1], int(hidden_size), None,
                  w1.shape[1],
                  align8=not _is_f32(w1))
    if _is_f32(w1):
        return f32_up_bwd(grad_output, x, w1, pre_act, None, m, int(hidden_size), act,
                          gather_map)
    return up_bwd(grad_output, x, w1, pre_act, m, int(hidden_size), act, gather_map)


@torch.compiler.disable
def grouped_gemm_down_backward(grad_output, intermediate, w2, expert_token_offsets,
                               expert_weight_offsets, expert_widths, tokens_per_expert,
                               hidden_size, max_expert_width):
    """(grad_intermediate [total_tokens, max_expert_width], grad_w2 like w2)."""
    _lib.require_gpu(grad_output)
    m = host_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                  tokens_per_expert, int(max_expert_width), int(hidden_size),
                  intermediate.shape[0], w2.shape[0],
                  align8=not _is_f32(w2))
    if _is_f32(w2):
        return f32_down_bwd(grad_output, intermediate, w2, m, int(hidden_size))
    return down_bwd(grad_output, intermediate, w2, m, int(hidden_size), zero_tails=True)


class GroupedGemmUp(torch.autograd.Function):
    """Autograd function for the grouped up-projection with fused activation.

    With x_flat and gather_map, backward reads x_flat through gather_map
    instead of keeping x_gathered alive (grouped_gemm.py:1442-1475).
    """

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x, w1, expert_token_offsets, expert_weight_offsets, expert_widths,
                tokens_per_expert, max_expert_width, hidden_size, activation, x_flat,
                gather_map):
        _lib.require_gpu(x)
        x = x.to(w1.dtype)
        act = _activation_code(activation)
        use_gm = x_flat is not None and gather_map is not None
        ctx.use_gather_map = use_gm
        xs = (x_flat.to(w1.dtype), w1) if use_gm else (x, w1)
        ctx.f32 = _is_f32(w1)
        if act == ACT_SWIGLU:
            gmeta = glu_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                             tokens_per_expert, int(max_expert_width), x.shape[1], w1.shape[1],
                             align8=not _is_f32(w1))
            if ctx.f32:
                out, gate, up = f32_up_fwd(x, w1, gmeta.fwd, act, want_pre=True, want_up=True)
            else:
                out, gate, up = glu_fwd(x, w1, gmeta.fwd, True, True, True)
            ctx.save_for_backward(*xs, gate, up, *((gather_map,) if use_gm else ()))
            ctx.meta = gmeta
            ctx.hidden_size = hidden_size
            ctx.act = act
            return out
        m = host_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                      tokens_per_expert, int(max_expert_width), x.shape[1], None, w1.shape[1],
                      align8=not _is_f32(w1))
        if ctx.f32:
            out, pre, _ = f32_up_fwd(x, w1, m, act, want_pre=True)
        else:
            out, pre = up_fwd(x, w1, m, act, True, zero_tails=True)
        ctx.save_for_backward(*xs, pre, *((gather_map,) if use_gm else ()))
        ctx.meta = m
        ctx.hidden_size = hidden_size
        ctx.act = act
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, grad_output):
        if ctx.act == ACT_SWIGLU:
            saved = ctx.saved_tensors
            x_for_dw, w1, gate, up = saved[:4]
            gm = saved[4] if ctx.use_gather_map else None
            if ctx.f32:
                grad_x, grad_w1 = f32_up_bwd(grad_output, x_for_dw, w1, gate, up, ctx.meta.fwd,
                                             int(ctx.hidden_size), ctx.act, gm)
            else:
                grad_x, grad_w1 = glu_bwd(grad_output, x_for_dw, w1, gate, up, ctx.meta,
                                          int(ctx.hidden_size), gm)
            return grad_x, grad_w1, None, None, None, None, None, None, None, None, None
        if ctx.use_gather_map:
            x_for_dw, w1, pre, gm = ctx.saved_tensors
        else:
            (x_for_dw, w1, pre), gm = ctx.saved_tensors, None
        if ctx.f32:
            grad_x, grad_w1 = f32_up_bwd(grad_output, x_for_dw, w1, pre, None, ctx.meta,
                                         int(ctx.hidden_size), ctx.act, gm)
        else:
            grad_x, grad_w1 = up_bwd(grad_output, x_for_dw, w1, pre, ctx.meta,
                                     int(ctx.hidden_size), ctx.act, gm)
        return grad_x, grad_w1, None, None, None, None, None, None, None, None, None


class GroupedGemmDown(torch.autograd.Function):
    """Autograd function for the grouped down-projection."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, intermediate, w2, expert_token_offsets, expert_weight_offsets,
                expert_widths, tokens_per_expert, hidden_size, max_expert_width):
        _lib.require_gpu(intermediate)
        intermediate = intermediate.to(w2.dtype)
        m = host_meta(expert_token_offsets, expert_weight_offsets, expert_widths,
                      tokens_per_expert, int(max_expert_width), int(hidden_size),
                      intermediate.shape[0], w2.shape[0],
                      align8=not _is_f32(w2))
        ctx.f32 = _is_f32(w2)
        out = (f32_down_fwd if ctx.f32 else down_fwd)(intermediate, w2, m, int(hidden_size))
        ctx.save_for_backward(intermediate, w2)
        ctx.meta = m
        ctx.hidden_size = hidden_size
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, grad_output):
        intermediate, w2 = ctx.saved_tensors
        if ctx.f32:
            grad_int, grad_w2 = f32_down_bwd(grad_output, intermediate, w2, ctx.meta,
                                             int(ctx.hidden_size))
        else:
            grad_int, grad_w2 = down_bwd(grad_output, intermediate, w2, ctx.meta,
                                         int(ctx.hidden_size), zero_tails=True)
        return grad_int, grad_w2, None, None, None, None, None, None


def grouped_gemm_up_autograd(x, w1, expert_token_offsets, expert_weight_offsets, expert_widths,
                             tokens_per_expert, max_expert_width, hidden_size,
                             activation="relu_squared", x_flat=None, gather_map=None):
    """Grouped GEMM up-projection with autograd support."""
    return GroupedGemmUp.apply(x, w1, expert_token_offsets, expert_weight_offsets,
                               expert_widths, tokens_per_expert, max_expert_width, hidden_size,
                               activation, x_flat, gather_map)


def grouped_gemm_down_autograd(intermediate, w2, expert_token_offsets, expert_weight_offsets,
                               expert_widths, tokens_per_expert, hidden_size, max_expert_width):
    """Grouped GEMM down-projection with autograd support."""
    return GroupedGemmDown.apply(intermediate, w2, expert_token_offsets, expert_weight_offsets,
                                 expert_widths, tokens_per_expert, hidden_size,
                                 max_expert_width)


# ---------------------------------------------------------------------------
# Sync-free module path
# ---------------------------------------------------------------------------


_SIDE_STREAMS: dict[int, torch.cuda.Stream] = {}
# The module's backward runs its weight-gradient GEMMs on a side stream
# (beside dH and dX) when True, keeps every launch on the current stream
# when False, and decides by size when None. On one stream the fused path
# (vmoe_moe_backward) pairs each weight-gradient GEMM with dH / dX in one
# launch, each on half of the CUs; the per-kernel path (and its timing)
# launches them one after the other. Measured per eager step (same box,
# interleaved): cfg3 0.779-0.781 ms paired against 0.789-0.791 with the
# second stream, cfg4 5.29 against 5.01-5.05; cfg1 / cfg2 pay 75-80 us of
# host time for the second stream's event hand-overs. HIP-graph replays
# follow the same rule (the side stream joins the capture through the
# stream waits): cfg4 5.12-5.13 ms with it against 5.30-5.32 paired.
BACKWARD_SIDE_STREAM: bool | None = None
SIDE_STREAM_MIN_WORK = 2 ** 37  # assignments x max expert width x hidden


def _use_side_stream(assignments: int, max_width: int, hidden: int) -> bool:
    if BACKWARD_SIDE_STREAM is not None:
        return BACKWARD_SIDE_STREAM
    return assignments * max_width * hidden >= SIDE_STREAM_MIN_WORK


_ORDER_EVENTS: dict[int, list] = {}


def _order(waiter: torch.cuda.Stream, signaler: torch.cuda.Stream, slot: int) -> None:
    """waiter waits for the work queued on signaler so far: one of a few
    reused events per device, recorded on signaler, waited on by waiter
    (Stream.wait_stream makes a new event every time, about twice the cost).
    A slot's event is recorded again only after its wait was queued, so
    reuse never loses a dependency."""
    idx = signaler.device.index
    evs = _ORDER_EVENTS.get(idx)
    if evs is None:
        evs = _ORDER_EVENTS[idx] = [torch.cuda.Event() for _ in range(3)]
    ev = evs[slot]
    ev.record(signaler)
    waiter.wait_event(ev)


def _side_stream(device) -> torch.cuda.Stream:
    """One extra stream per device (default priority) for GEMMs that can run
    beside the ones on the current stream."""
    device = torch.device(device)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    st = _SIDE_STREAMS.get(idx)
    if st is None:
        st = torch.cuda.Stream(device=idx)
        _SIDE_STREAMS[idx] = st
    return st


# The module's bf16 expert path as one library call per direction
# (ExpertPathOp); False: one call per kernel (RoutedMoEOp), the same kernels
# and bits. The per-kernel form also runs whenever a launch timer is set.
FUSED_EXPERT_PATH = True

_LAYOUTS: dict[tuple, tuple] = {}


def expert_layout(T: int, E: int, k: int, block_size: int, hidden: int, max_width: int,
                  counted: bool) -> tuple:
    """(saved_bytes, fwd_scratch_bytes, bwd_scratch_bytes, rows_bound, slot offsets) of
    vmoe_expert_forward / _backward, cached per shape."""
    key = (T, E, k, block_size, hidden, max_width, counted)
    lay = _LAYOUTS.get(key)
    if lay is None:
        out = (ctypes.c_int64 * (4 + _lib.X_NSLOTS))()
        _lib.check(_lib.lib().vmoe_expert_layout(T, E, k, block_size, hidden, max_width,
                                                  int(counted), out), "vmoe_expert_layout")
        lay = _LAYOUTS[key] = (out[0], out[1], out[2], out[3], tuple(out[4:]))
    return lay


class ExpertPathOp(torch.autograd.Function):
    """RoutedMoEOp's forward and backward, each as one library call
    (vmoe_expert_forward / vmoe_expert_backward): the same kernels in the
    same order with the same operands, so the same bits, without the
    per-kernel wrappers, allocations and stream hand-overs in Python.
    Buffers: one `saved` block (routing arrays, row weights, H', PRE) kept
    for the backward and one scratch block per direction.

    forward(x_flat, w1, w2, weights, selected, route_ws, widths, ewo, top_k,
    block_size, max_width, weights_grad) -> (out, tokens_per_expert): weights
    bf16 [T k] (differentiated when weights_grad), selected int32/int64
    [T k], route_ws the counted routing workspace or None."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x_flat, w1, w2, weights, selected, route_ws, widths, ewo, top_k,
                block_size, max_width, weights_grad):
        T, d = x_flat.shape
        E = widths.numel()
        dev = x_flat.device
        x_flat = _bf16(x_flat, "TritonMoEMLP x")
        saved_b, fwd_b, _, rows, slots = expert_layout(T, E, top_k, block_size, d, max_width,
                                                       route_ws is not None)
        saved = torch.empty(saved_b, dtype=torch.uint8, device=dev)
        scratch = torch.empty(fwd_b, dtype=torch.uint8, device=dev)
        out = torch.empty(T, d, dtype=torch.bfloat16, device=dev)
        sel = selected.reshape(-1)
        if T == 0:
            saved.zero_()  # no routing runs: zero counts
        _lib.call("vmoe_expert_forward", sel.data_ptr(), int(sel.dtype == torch.int64),
                  weights.data_ptr(), T, E, top_k, block_size, _lib.ptr(route_ws),
                  0 if route_ws is None else route_ws.numel() * route_ws.element_size(),
                  x_flat.data_ptr(), x_flat.stride(0), w1.data_ptr(), w1.stride(0),
                  w2.data_ptr(), w2.stride(0), ewo.data_ptr(), widths.data_ptr(), d, max_width,
                  saved.data_ptr(), scratch.data_ptr(), out.data_ptr(), out.stride(0),
                  _lib.stream(dev))
        o = slots[_lib.X_TPE]
        tpe = saved[o:o + 4 * E].view(torch.int32)
        ctx.save_for_backward(x_flat, w1, w2, widths, ewo, saved)
        ctx.dims = (T, E, top_k, block_size, d, max_width, rows)
        ctx.weights_grad = bool(weights_grad)
        ctx.mark_non_differentiable(tpe)
        return out, tpe

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, grad_out, _grad_tpe):
        x_flat, w1, w2, widths, ewo, saved = ctx.saved_tensors
        T, E, k, b, d, max_width, rows = ctx.dims
        dev = grad_out.device
        _, _, bwd_b, _, _ = expert_layout(T, E, k, b, d, max_width, True)
        if (grad_out.dtype == torch.bfloat16 and T > 0 and grad_out.stride(0) == 0 and
                grad_out.stride(1) == 0):
            g, ldg, gs = _ones_row(d, dev), 0, grad_out  # c * out.sum(): ones, scaled by c
        else:
            (g, ldg), gs = _token_source(grad_out), None
        grad_x = torch.empty(T, d, dtype=torch.bfloat16, device=dev)
        # no tokens: the library writes nothing, the weight gradients are zero
        grad_w1 = torch.empty_like(w1) if T > 0 else torch.zeros_like(w1)
        grad_w2 = torch.empty_like(w2) if T > 0 else torch.zeros_like(w2)
        grad_w = (torch.empty(T * k, dtype=torch.bfloat16, device=dev) if ctx.weights_grad
                  and ctx.needs_input_grad[3] else None)
        scratch = torch.empty(bwd_b, dtype=torch.uint8, device=dev)
        main = torch.cuda.current_stream(dev)
        side = _side_stream(dev) if _use_side_stream(T * k, max_width, d) else None
        ws = _dw_workspace_bytes(E, d, max_width, rows, dev,
                                 side.cuda_stream if side is not None else main.cuda_stream)
        _lib.call("vmoe_expert_backward", saved.data_ptr(), T, E, k, b, x_flat.data_ptr(),
                  x_flat.stride(0), w1.data_ptr(), w1.stride(0), w2.data_ptr(), w2.stride(0),
                  ewo.data_ptr(), widths.data_ptr(), d, max_width, g.data_ptr(), ldg,
                  _lib.ptr(gs), grad_x.data_ptr(), grad_x.stride(0), grad_w1.data_ptr(),
                  grad_w1.stride(0), grad_w2.data_ptr(), grad_w2.stride(0), _lib.ptr(grad_w),
                  scratch.data_ptr(), ws.data_ptr(), ws.numel(), main.cuda_stream,
                  None if side is None else side.cuda_stream)
        return (grad_x, grad_w1, grad_w2, grad_w, None, None, None, None, None, None, None,
                None)


def moe_layout(T: int, E: int, k: int, block_size: int, hidden: int, max_width: int) -> tuple:
    """(saved_bytes, fwd_scratch_bytes, bwd_scratch_bytes, rows_bound, expert slot
    offsets, layer slot offsets, counted) of vmoe_moe_forward / _backward, cached."""
    key = ("moe", T, E, k, block_size, hidden, max_width)
    lay = _LAYOUTS.get(key)
    if lay is None:
        n = 5 + _lib.X_NSLOTS + _lib.M_NSLOTS
        out = (ctypes.c_int64 * n)()
        _lib.check(_lib.lib().vmoe_moe_layout(T, E, k, block_size, hidden, max_width, out),
                   "vmoe_moe_layout")
        xs = 4 + _lib.X_NSLOTS
        lay = _LAYOUTS[key] = (out[0], out[1], out[2], out[3], tuple(out[4:xs]),
                               tuple(out[xs:xs + _lib.M_NSLOTS]), bool(out[n - 1]))
    return lay


_MOE_PLANS: dict[tuple, tuple] = {}


def _moe_plan(T: int, E: int, k: int, block_size: int, hidden: int, max_width: int,
              device: torch.device) -> tuple:
    """Everything MoELayerOp's two calls need that depends on the shape only,
    looked up once: (saved_bytes, fwd_scratch_bytes, bwd_scratch_bytes,
    rows_bound, dW workspace bytes, side stream by size, the ones row of
    out.sum()'s gradient, the two library functions). An eager step at cfg1
    is host-bound, so per-step Python is step time."""
    key = (T, E, k, block_size, hidden, max_width, device.index)
    plan = _MOE_PLANS.get(key)
    if plan is None:
        saved_b, fwd_b, bwd_b, rows, _, _, _ = moe_layout(T, E, k, block_size, hidden, max_width)
        ws_n = max(int(_lib.lib().vmoe_gemm_dw_workspace_bytes(E, hidden, max_width,
                                                               max(rows, 1))), 16)
        plan = _MOE_PLANS[key] = (
            saved_b, fwd_b, bwd_b, rows, ws_n,
            T * k * max_width * hidden >= SIDE_STREAM_MIN_WORK, _ones_row(hidden, device),
            _lib.lib().vmoe_moe_forward, _lib.lib().vmoe_moe_backward)
    return plan


class MoELayerOp(torch.autograd.Function):
    """TritonMoEMLP.forward after the router Linear as one autograd node and
    one library call per direction (vmoe_moe_forward / vmoe_moe_backward):
    top-k, routing, the expert path and the auxiliary losses, with the
    kernels, operands and order of the per-op path (router_topk,
    ExpertPathOp / RoutedMoEOp, RouterAuxOp, RouterWeightOp), so the same
    bits.

    forward(logits, x_flat, w1, w2, consts) -> (out, z_loss,
    load_balance_loss, compute_loss, f_i), consts = (widths, ewo, coef, wn,
    top_k, block_size, max_width, normalize, weight_grad): the module's
    constant tables and settings in one argument, since autograd's per-call
    work grows with the argument count. The logits get the auxiliary losses'
    gradient and, with weight_grad, the routing weights' chain; f_i has none.

    Unlike the per-kernel ops it carries no torch.amp custom_fwd / custom_bwd:
    neither direction runs an op that autocast would change (allocations with
    explicit dtypes and one library call), so the autocast context those
    decorators enter around the backward (~12 us of host time per eager cfg1
    step, whose pace the host sets on slower host CPUs) changes nothing but
    the time."""

    @staticmethod
    def forward(ctx, logits, x_flat, w1, w2, consts):
        widths, ewo, coef, wn, top_k, block_size, max_width, normalize, weight_grad = consts
        T, d = x_flat.shape
        E = widths.shape[0]
        dev = x_flat.device
        x_flat = _bf16(x_flat, "TritonMoEMLP x")
        if not logits.is_contiguous() or logits.data_ptr() % 16:
            logits = logits.clone(memory_format=torch.contiguous_format)
        plan = _moe_plan(T, E, top_k, block_size, d, max_width, dev)
        saved = torch.empty(plan[0], dtype=torch.uint8, device=dev)
        scratch = torch.empty(plan[1], dtype=torch.uint8, device=dev)
        out = torch.empty(T, d, dtype=torch.bfloat16, device=dev)
        z = torch.empty((), dtype=torch.bfloat16, device=dev)
        losses = torch.empty(2, dtype=torch.float32, device=dev)
        f_i = torch.empty(E, dtype=torch.bfloat16, device=dev)
        if T == 0:
            z.zero_(), losses.zero_(), f_i.zero_()
        st = plan[7](logits.data_ptr(), T, E, top_k, int(bool(normalize)), block_size,
                     x_flat.data_ptr(), x_flat.stride(0), w1.data_ptr(), w1.stride(0),
                     w2.data_ptr(), w2.stride(0), ewo.data_ptr(), widths.data_ptr(), d, max_width,
                     coef.data_ptr(), wn.data_ptr(), saved.data_ptr(), scratch.data_ptr(),
                     out.data_ptr(), d, z.data_ptr(), losses.data_ptr(), f_i.data_ptr(),
                     _lib.stream(dev))
        if st != _lib.OK:
            _lib.check(st, "vmoe_moe_forward")
        ctx.save_for_backward(logits, x_flat, w1, w2, saved)
        # the module's constant tables (buffers, never written in place)
        ctx.consts = consts
        ctx.dims = (T, E, d, int(bool(normalize)))
        ctx.mark_non_differentiable(f_i)
        # unused outputs arrive as None (not zeros), so a loss that leaves out
        # the auxiliary losses gives the router no gradient, as in the reference
        ctx.set_materialize_grads(False)
        return out, z, losses[0], losses[1], f_i

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out, g_z, g_lb, g_cl, _g_fi):
        logits, x_flat, w1, w2, saved = ctx.saved_tensors
        widths, ewo, coef, wn, k, b, max_width, _, weight_grad = ctx.consts
        T, E, d, norm = ctx.dims
        dev = logits.device
        plan = _moe_plan(T, E, k, b, d, max_width, dev)

        def scalar(g):
            return None if g is None else g.detach().to(torch.float32).reshape(()).contiguous()

        gz, glb, gcl = scalar(g_z), scalar(g_lb), scalar(g_cl)
        need = ctx.needs_input_grad
        want_x = grad_out is not None and (need[1] or need[2] or need[3])
        want_logits = need[0] and (
            gz is not None or glb is not None or gcl is not None or (weight_grad and want_x))
        grad_x = grad_w1 = grad_w2 = grad_logits = None
        g = gs = None
        ldg = 0
        if want_x:
            if (grad_out.dtype == torch.bfloat16 and T > 0 and grad_out.stride(0) == 0 and
                    grad_out.stride(1) == 0):
                g, ldg, gs = plan[6], 0, grad_out  # c * out.sum(): ones times c
            else:
                (g, ldg), gs = _token_source(grad_out), None
            grad_x = torch.empty(T, d, dtype=torch.bfloat16, device=dev)
            # no tokens: the library writes nothing, the weight gradients are zero
            grad_w1 = torch.empty_like(w1) if T > 0 else torch.zeros_like(w1)
            grad_w2 = torch.empty_like(w2) if T > 0 else torch.zeros_like(w2)
        if want_logits:
            grad_logits = torch.empty(T, E, dtype=torch.bfloat16, device=dev)
        if not want_x and not want_logits:
            return None, None, None, None, None
        scratch = torch.empty(plan[2], dtype=torch.uint8, device=dev)
        main = _lib.stream(dev)
        use_side = BACKWARD_SIDE_STREAM if BACKWARD_SIDE_STREAM is not None else plan[5]
        side = _side_stream(dev).cuda_stream if use_side else None
        ws_stream = side if side is not None else main
        ws = _DW_WORKSPACES.get((dev.index, ws_stream))
        if ws is None or ws.numel() < plan[4]:
            ws = _dw_workspace_bytes(E, d, max_width, plan[3], dev, ws_stream)
        ptr = _lib.ptr
        st = plan[8](saved.data_ptr(), logits.data_ptr(), T, E, k, norm, b,
                     x_flat.data_ptr(), x_flat.stride(0), w1.data_ptr(), w1.stride(0),
                     w2.data_ptr(), w2.stride(0), ewo.data_ptr(), widths.data_ptr(), d, max_width,
                     coef.data_ptr(), wn.data_ptr(), ptr(g), ldg, ptr(gs), ptr(gz), ptr(glb),
                     ptr(gcl), int(bool(weight_grad)), ptr(grad_x), d, ptr(grad_w1), w1.stride(0),
                     ptr(grad_w2), w2.stride(0), ptr(grad_logits), scratch.data_ptr(),
                     ws.data_ptr(), ws.numel(), main, side)
        if st != _lib.OK:
            _lib.check(st, "vmoe_moe_backward")
        return grad_logits, grad_x, grad_w1, grad_w2, None


class NoTokensOp(torch.autograd.Function):
    """The expert path of a batch without tokens: forward(x_flat [0, d], w1,
    w2) -> an empty [0, d] output; the backward gives an empty input gradient
    and zero weight gradients, as the reference's grouped GEMMs return zeros
    for empty inputs (grouped_gemm.py:1214-1215, 1333-1334)."""

    @staticmethod
    def forward(ctx, x_flat, w1, w2):
        ctx.save_for_backward(w1, w2)
        return x_flat.new_empty(0, x_flat.shape[1])

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        w1, w2 = ctx.saved_tensors
        return (grad_out.new_empty(0, grad_out.shape[1]), torch.zeros_like(w1),
                torch.zeros_like(w2))


class CompactRoutedMoEOp(torch.autograd.Function):
    """RoutedMoEOp with its per-row intermediates (H', PRE, GA) stored per
    width group instead of in one [rows, max_width] block: each group of
    consecutive experts of one width w_g keeps [rows of the group, w_g], so
    the three take sum_e rows_e w_e elements instead of rows x max_width
    (the compact layout the reference's grouped_gemm.py:13-16 leaves for a
    later version). The kernels are the same, launched once per group on the
    group's rows (row maps, row weights and outputs as views at the group's
    first row); Y' and the dX rows stay [rows, hidden] for the combines.
    Needs the groups' exact row counts, so the caller reads the routing's
    padded counts back once per forward (TritonMoEConfig.compact_intermediates).

    groups: [(GemmMeta of the group, first row, (first, last) weight rows /
    columns)], rows: the routed row count. The routing weights get no
    gradient here."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x_flat, w1, w2, groups, gather_map, row_weight, assignment_row, top_k,
                hidden_size, rows):
        from .gather import combine_rows

        dev = x_flat.device
        y = torch.empty(rows, hidden_size, dtype=torch.bfloat16, device=dev)
        hs, pres = [], []
        for m, r0, _cols in groups:
            r1 = r0 + m.rows
            h, pre = up_fwd(x_flat, w1, m, _lib.ACT_RELU_SQUARED, True, zero_tails=False,
                            gather_map=gather_map[r0:r1], row_scale=row_weight[r0:r1])
            down_fwd(h, w2, m, hidden_size, out=y[r0:r1])
            hs.append(h)
            pres.append(pre)
        out = combine_rows(y, assignment_row, top_k, x_flat.shape[0])
        ctx.save_for_backward(x_flat, w1, w2, gather_map, row_weight, assignment_row, *hs, *pres)
        ctx.groups = groups
        ctx.hidden_size = hidden_size
        ctx.top_k = top_k
        ctx.rows = rows
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, grad_out):
        from .gather import combine_rows

        x_flat, w1, w2, gm, rw, ar, *rest = ctx.saved_tensors
        n = len(ctx.groups)
        hs, pres = rest[:n], rest[n:]
        d = ctx.hidden_size
        dev = grad_out.device
        grad_xg = torch.empty(ctx.rows, d, dtype=torch.bfloat16, device=dev)
        grad_w1 = torch.empty_like(w1)
        grad_w2 = torch.empty_like(w2)
        for (m, r0, (c0, c1)), h, pre in zip(ctx.groups, hs, pres):
            if m.rows == 0:  # no rows routed to the group: its weight gradients are 0
                grad_w1[:, c0:c1].zero_()
                grad_w2[c0:c1].zero_()
                continue
            r1 = r0 + m.rows
            ga = down_bwd_dh(grad_out, w2, m, d, False, pre=pre, gather_map=gm[r0:r1],
                             row_scale=rw[r0:r1])
            down_bwd_dw(grad_out, h, w2, m, d, gather_map=gm[r0:r1], out=grad_w2)
            up_bwd_dx(ga, w1, m, d, out=grad_xg[r0:r1])
            up_bwd_dw(ga, x_flat, w1, m, d, gm[r0:r1], out=grad_w1)
        grad_x = combine_rows(grad_xg, ar, ctx.top_k, x_flat.shape[0])
        return grad_x, grad_w1, grad_w2, None, None, None, None, None, None, None


class RoutedMoEOpF32(torch.autograd.Function):
    """The module's expert path for float32 parameters, as one autograd node:
    the reference's chain in fp32 (padded_gather, grouped_gemm_up/down and
    padded_scatter as TritonMoEMLP.forward calls them, moe.py:203-240, its
    kernels being dtype-generic) on the fp32 kernels. The up GEMM reads
    x_flat through the row map (relu^2, PRE = relu(z) kept), the down GEMM
    writes Y, and the combine weights and sums each token's k rows, the
    weight on Y as in the reference. Backward: the output gradient gathered
    into rows with the weights (GY[r] = G[t] w, scatter.py:141-189), dH and
    dW2 from GY, the relu^2 rule once (GA), dX and dW1 (x through the map),
    and the unweighted combine of dX. `weights` (fp32 [A]) gets
    dL/dw = G[t] . Y[row] when it requires grad (opt-in; the reference
    returns None, scatter.py:176)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x_flat, w1, w2, meta, gather_map, row_src, assignment_row, weights, top_k,
                hidden_size):
        from .gather import combine_rows

        h, pre, _ = f32_up_fwd(x_flat, w1, meta, _lib.ACT_RELU_SQUARED, gather_map,
                               want_pre=True)
        y = f32_down_fwd(h, w2, meta, hidden_size)
        out = combine_rows(y, assignment_row, top_k, x_flat.shape[0], weights=weights)
        ctx.save_for_backward(x_flat, w1, w2, h, pre, y, gather_map, row_src, assignment_row,
                              weights)
        ctx.meta = meta
        ctx.hidden_size = hidden_size
        ctx.top_k = top_k
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, grad_out):
        from .gather import combine_rows, combine_weight_grad, gather_rows

        x_flat, w1, w2, h, pre, y, gm, rs, ar, weights = ctx.saved_tensors
        m, d, k = ctx.meta, ctx.hidden_size, ctx.top_k
        T = x_flat.shape[0]
        grad_out = grad_out.to(torch.float32)
        gy = gather_rows(grad_out, rs, k, m.rows, weights=weights)
        grad_h, grad_w2 = f32_down_bwd(gy, h, w2, m, d)
        grad_xg, grad_w1 = f32_up_bwd(grad_h, x_flat, w1, pre, None, m, d,
                                      _lib.ACT_RELU_SQUARED, gm)
        grad_x = combine_rows(grad_xg, ar, k, T)
        grad_w = None
        if ctx.needs_input_grad[7]:
            grad_w = combine_weight_grad(grad_out, y, ar, k).to(weights.dtype)
        return grad_x, grad_w1, grad_w2, None, None, None, None, grad_w, None, None


class RoutedMoEOp(torch.autograd.Function):
    """The module's expert path after routing, as one autograd node: token
    gather, grouped GEMM up with relu^2, grouped GEMM down, weighted combine,
    and their backward (reference: padded_gather, grouped_gemm_up/down and
    padded_scatter as called by TritonMoEMLP.forward, moe.py:203-240).

    The gather is fused into the GEMMs' operand staging: the up GEMM and its
    dW read x_flat through the row map (row -> token, -1 on pad rows, which
    read zeros), so the gathered copy of x is never written.

    The routing weight of each row is applied to H instead of to the down
    projection's output: the up GEMM writes H' = bf16(w_row * relu(z)^2), so
    Y' = H' @ W2 = w * Y and the combine is the plain sum over a token's k
    rows. The backward then needs no weighted copy of the output gradient
    G (the reference's GY = bf16(G * w), scatter.py:141-189): the dH GEMM
    reads G through the row map and scales row r by w_r before the relu^2
    rule (w_r (G @ W2^T) = GY @ W2^T), and the dW2 GEMM reads G through the
    map against H' (H'^T G = H^T GY). The products are the reference's; only
    where they round to bf16 moves. The routing weights get no gradient, as
    in the reference (scatter.py:176), unless they are passed as `weights`
    (bf16 [A], the tensor row_weight was formed from): then the dH GEMM also
    sums GH * PRE^2 per row and block, and dL/dw = that sum / w (H' = w h,
    h = relu(z)^2 read back as PRE^2) is returned for them.
    """

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x_flat, w1, w2, meta, gather_map, row_weight, assignment_row, top_k,
                hidden_size, weights=None):
        from .gather import combine_rows

        h, pre = up_fwd(x_flat, w1, meta, _lib.ACT_RELU_SQUARED, True, zero_tails=False,
                        gather_map=gather_map, row_scale=row_weight)
        y = down_fwd(h, w2, meta, hidden_size)
        out = combine_rows(y, assignment_row, top_k, x_flat.shape[0])
        ctx.save_for_backward(x_flat, w1, w2, h, pre, gather_map, row_weight, assignment_row)
        ctx.meta = meta
        ctx.hidden_size = hidden_size
        ctx.top_k = top_k
        ctx.weights_shape = None if weights is None else weights.shape
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    @once_differentiable
    def backward(ctx, grad_out):
        from .gather import combine_rows

        x_flat, w1, w2, h, pre, gm, rw, ar = ctx.saved_tensors
        m, d = ctx.meta, ctx.hidden_size
        # Two streams: the weight-gradient GEMMs run on a side stream, dW2
        # (it needs only G and H') beside dH, dW1 beside dX once GA exists.
        # Each GEMM keeps every CU busy until its last tiles, which are
        # fewer than the CUs; the other stream's workgroups take the CUs
        # those tails leave idle.
        main = torch.cuda.current_stream(grad_out.device)
        side = (_side_stream(grad_out.device)
                if _use_side_stream(ctx.top_k * x_flat.shape[0], m.max_width, d) else main)
        if side is not main:
            _order(side, main, 0)
        row_dot = None
        if ctx.weights_shape is not None and ctx.needs_input_grad[9]:
            nblk = (m.max_width + 63) // 64
            alloc = torch.empty if m.uniform else torch.zeros  # blocks past w_e stay 0
            row_dot = alloc(m.rows, nblk, dtype=torch.float32, device=grad_out.device)
        ga = down_bwd_dh(grad_out, w2, m, d, False, pre=pre, gather_map=gm, row_scale=rw,
                         row_dot=row_dot)
        with torch.cuda.stream(side):
            grad_w2 = down_bwd_dw(grad_out, h, w2, m, d, gather_map=gm)
        if side is not main:
            _order(side, main, 1)
        with torch.cuda.stream(side):
            grad_w1 = up_bwd_dw(ga, x_flat, w1, m, d, gm)
        grad_xg = up_bwd_dx(ga, w1, m, d)
        grad_x = combine_rows(grad_xg, ar, ctx.top_k, x_flat.shape[0])
        if side is not main:
            _order(main, side, 2)
        # Cross-stream lifetimes for the caching allocator: main's tensors
        # read on the side stream, the side stream's results used on main.
        # (Under graph capture the graph's private pool keeps them alive.)
        if side is not main and not torch.cuda.is_current_stream_capturing():
            for t in (grad_out, ga, h, x_flat, gm, w1, w2):
                t.record_stream(side)
            for t in (grad_w1, grad_w2):
                t.record_stream(main)
        grad_weights = None
        if row_dot is not None:
            grad_weights = torch.empty(ctx.weights_shape, dtype=torch.bfloat16,
                                       device=grad_out.device)
            st = _lib.stream(grad_out.device)
            _lib.call("vmoe_routing_weight_grad", row_dot.data_ptr(), row_dot.stride(0),
                      row_dot.shape[1], m.rows, rw.data_ptr(), ar.data_ptr(), ar.numel(),
                      grad_weights.data_ptr(), st)
            # weights of magnitude below 2^-64 (zero included): from the
            # unscaled gradient, which the division above cannot recover
            g, ldg, g_rows, gs = _grad_source(grad_out, m, gm)
            _lib.call("vmoe_routing_weight_grad_direct", g.data_ptr(), ldg, g_rows,
                      _lib.ptr(gs), w2.data_ptr(), w2.stride(0), pre.data_ptr(), pre.stride(0),
                      rw.data_ptr(), ar.data_ptr(), ar.numel(), ctx.top_k, m.eto.data_ptr(),
                      m.ewo.data_ptr(), m.widths.data_ptr(), m.num_experts, d, m.rows,
                      grad_weights.data_ptr(), st)
        return grad_x, grad_w1, grad_w2, None, None, None, None, None, None, grad_weights
