"""Tensor-level calls into libisa_ekv_hip.so (LUT forward/backward, table build and pack,
and the exact-formula forward/backward).

Every function validates on the host what the kernels assume (device, dtype, shape,
contiguity, 16-byte alignment) before launching, allocates outputs and workspace with
the caching allocator, and enqueues on the current stream of the tensors' device.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from isa.kernels.transformer_ffn import _hip

MAX_ENTRIES_FORWARD = 16384   # forward table resident in LDS up to this size
MAX_ENTRIES_BACKWARD = 8192   # backward table resident in LDS; the reference's shared-backward limit
MAX_ENTRIES = 1 << 22         # larger tables up to this size are read from global memory


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")


def as_kernel_f32(t: torch.Tensor) -> torch.Tensor:
    """fp32, contiguous and 16-byte aligned (a copy only when needed)."""
    if t.dtype is torch.float32 and t.is_contiguous() and not t.data_ptr() & 15:
        return t  # the common case, without the conversions' dispatch cost
    t = t.to(dtype=torch.float32).contiguous()
    if t.numel() and t.data_ptr() % 16:
        t = t.clone()
    return t


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _workspace(nbytes: int, device: torch.device, given: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The call's workspace: `given` (a caller's uint8 device buffer, checked) or a new one of
    `nbytes` (the workspace query's bound). A given buffer's size is checked by the library
    against the call's own plan (plan_info's workspace_bytes), which the bound may exceed."""
    if given is None:
        return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)
    _require_cuda(given, "workspace")
    if given.dtype != torch.uint8 or not given.is_contiguous() or given.device != device:
        raise RuntimeError(f"workspace must be a contiguous uint8 tensor on {device}")
    if given.data_ptr() % 256:
        raise RuntimeError("workspace must start at a 256-byte aligned address")
    return given


_PLAN_KINDS = {"forward": _hip.PLAN_FORWARD, "backward": _hip.PLAN_BACKWARD,
               "layer_backward": _hip.PLAN_LAYER_BACKWARD}


def plan_info(kind: str, M: int, K: int, O: int, n_entries: int, need_grad_x: bool = True,
              need_grad_w: bool = True) -> dict:
    """The library's plan for a LUT call at this shape (isa_ekv_plan_info): workspace bytes,
    the byte offset of the table-copy mode word in the workspace (-1 when the call has none),
    K splits (forward) or token splits (backward), tokens (forward) or inputs (backward) per
    wave, main-kernel blocks, waves per block, LDS bytes per block and (backward with dVth)
    the dVth partial planes."""
    lib = _hip.load()
    info = (ctypes.c_int64 * _hip.PLAN_INFO_LEN)()
    rc = lib.isa_ekv_plan_info(_PLAN_KINDS[kind], int(M), int(K), int(O), int(n_entries), int(need_grad_x),
                               int(need_grad_w), info, _hip.PLAN_INFO_LEN)
    _hip.check(rc, "isa_ekv_plan_info")
    keys = ("workspace_bytes", "mode_offset", "splits", "per_wave", "blocks", "waves_per_block", "lds_bytes",
            "dv_planes")
    return dict(zip(keys, (int(v) for v in info)))


def copy_min_cells(value: Optional[int] = None) -> int:
    """The library's ISA_EKV_OPT_COPY_MIN_CELLS (calls of fewer cells M*K*O run one table
    copy); sets it when value is given. Returns the value before the call."""
    lib = _hip.load()
    prev = ctypes.c_int64()
    rc = lib.isa_ekv_set_option(_hip.OPT_COPY_MIN_CELLS, -1 if value is None else int(value), ctypes.byref(prev))
    _hip.check(rc, "isa_ekv_set_option")
    return int(prev.value)


def ranked_backward(value: Optional[bool] = None) -> bool:
    """The library's ISA_EKV_OPT_RANKED (whether table backwards that consider the second copy
    may run the ranked kernel); sets it when value is given. Returns the value before the call."""
    lib = _hip.load()
    prev = ctypes.c_int64()
    rc = lib.isa_ekv_set_option(_hip.OPT_RANKED, -1 if value is None else int(bool(value)), ctypes.byref(prev))
    _hip.check(rc, "isa_ekv_set_option")
    return bool(prev.value)


def window_copies(value: Optional[int] = None) -> int:
    """The library's ISA_EKV_OPT_WINDOW_COPIES (the most windowed table copies a LUT forward, or
    a table backward's two-copy launch, may hold: 3 to 32, default 32; below 3 none); sets it
    when value is given. Returns the value before
    the call."""
    lib = _hip.load()
    prev = ctypes.c_int64()
    rc = lib.isa_ekv_set_option(_hip.OPT_WINDOW_COPIES, -1 if value is None else int(value), ctypes.byref(prev))
    _hip.check(rc, "isa_ekv_set_option")
    return int(prev.value)


def _int_option(option: int, value: Optional[int]) -> int:
    lib = _hip.load()
    prev = ctypes.c_int64()
    rc = lib.isa_ekv_set_option(option, -1 if value is None else int(value), ctypes.byref(prev))
    _hip.check(rc, "isa_ekv_set_option")
    return int(prev.value)


def rank_max_spread(value: Optional[int] = None) -> int:
    """The library's ISA_EKV_OPT_RANK_MAX_SPREAD (the widest threshold spread, in table records,
    the ranked backward takes; default 420); sets it when value is given. Returns the value
    before the call."""
    return _int_option(_hip.OPT_RANK_MAX_SPREAD, value)


def rank_greedy_min(value: Optional[int] = None) -> int:
    """The library's ISA_EKV_OPT_RANK_GREEDY_MIN (threshold spreads, in table records, past which
    the ranked backward's branches are dealt by the greedy bank-aware deal instead of by rank;
    default 4128, i.e. never); sets it when value is given. Returns the value before the call."""
    return _int_option(_hip.OPT_RANK_GREEDY_MIN, value)


def rank_xcd_order(value: Optional[bool] = None) -> bool:
    """The library's ISA_EKV_OPT_RANK_XCD_ORDER (whether each XCD runs a contiguous range of the
    ranked backward's blocks); sets it when value is given. Returns the value before the call."""
    return bool(_int_option(_hip.OPT_RANK_XCD_ORDER, None if value is None else int(bool(value))))


def copy_mode(workspace: torch.Tensor, plan: dict) -> Optional[int]:
    """After a call that used `workspace` (and synchronised), which table mode its main kernel
    ran in: 1 the second table copy, 0 one copy, 2 the ranked backward, 3 to 32 the forward's
    windowed copies (their number); None when the plan has no second copy."""
    off = plan["mode_offset"]
    if off < 0:
        return None
    return int(workspace[off:off + 4].view(torch.int32).item())


def build_plain_tables(params: Tuple[float, float, float, float], delta_min: float, delta_max: float,
                       size: int, device: torch.device, bf16: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """(table_i, table_ddelta), each [size], evaluated on the device (delta_lut.py:12-35)."""
    lib = _hip.load()
    dtype = torch.bfloat16 if bf16 else torch.float32
    layout = _hip.LUT_PLAIN_BF16 if bf16 else _hip.LUT_PLAIN_F32
    buf = torch.empty(2 * size, dtype=dtype, device=device)
    arr = (ctypes.c_double * 4)(*[float(v) for v in params])
    with _hip.on_device(device):
        rc = lib.isa_ekv_lut_build(arr, float(delta_min), float(delta_max), int(size), layout, buf.data_ptr(),
                                   _hip.stream_handle(device))
    _hip.check(rc, "isa_ekv_lut_build")
    return buf[:size], buf[size:]


def pack_tables(table_i: torch.Tensor, table_ddelta: Optional[torch.Tensor], layout: int) -> torch.Tensor:
    """Padded kernel records from plain tables (fp32, or bf16 widened to fp32)."""
    lib = _hip.load()
    _require_cuda(table_i, "table_i")
    n = table_i.numel()
    if table_i.dtype not in (torch.float32, torch.bfloat16):
        table_i = table_i.float()
    src = _hip.LUT_PLAIN_BF16 if table_i.dtype == torch.bfloat16 else _hip.LUT_PLAIN_F32
    table_i = table_i.contiguous()
    if table_ddelta is None:
        table_ddelta = table_i
    table_ddelta = table_ddelta.to(dtype=table_i.dtype).contiguous()
    if table_ddelta.numel() != n:
        raise RuntimeError("table_i and table_ddelta must have the same LUT_DELTA_SIZE")
    out = torch.empty(lib.isa_ekv_lut_bytes(n, layout), dtype=torch.uint8, device=table_i.device)
    dtype_code = 1 if src == _hip.LUT_PLAIN_BF16 else 0
    with _hip.on_device(table_i.device):
        rc = lib.isa_ekv_lut_pack(table_i.data_ptr(), table_ddelta.data_ptr(), n, dtype_code, layout,
                                  out.data_ptr(), _hip.stream_handle(table_i.device))
    _hip.check(rc, "isa_ekv_lut_pack")
    return out


def _check_operands(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor) -> Tuple[int, int, int]:
    for t, name in ((x, "x"), (wpos, "wpos"), (wneg, "wneg")):
        _require_cuda(t, name)
    if x.dim() != 2:
        raise RuntimeError(f"x must be 2-D [M, K], got shape {tuple(x.shape)}")
    if wpos.dim() != 2 or wpos.shape != wneg.shape:
        raise RuntimeError(f"wpos/wneg must both be [O, K], got {tuple(wpos.shape)} and {tuple(wneg.shape)}")
    if wpos.shape[1] != x.shape[1]:
        raise RuntimeError(f"in_features mismatch: x has K={x.shape[1]}, wpos has K={wpos.shape[1]}")
    if wpos.device != x.device or wneg.device != x.device:
        raise RuntimeError("x, wpos and wneg must be on the same device")
    return int(x.shape[0]), int(x.shape[1]), int(wpos.shape[0])


def lut_forward(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, fwd_records: torch.Tensor,
                n_entries: int, delta_min: float, delta_max: float, v_sat: float,
                out_min: float, out_max: float, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Idiff[M, O] fp32 (clamped to [out_min, out_max]). workspace: optional caller buffer
    (uint8, at least isa_ekv_forward_workspace bytes)."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    if n_entries > MAX_ENTRIES:
        raise RuntimeError(f"LUT forward supports LUT_DELTA_SIZE <= {MAX_ENTRIES}")
    dev = x.device
    out = torch.empty((M, O), dtype=torch.float32, device=dev)
    if M == 0 or O == 0:
        return out
    x32, wp32, wn32 = as_kernel_f32(x), as_kernel_f32(wpos), as_kernel_f32(wneg)
    ws_bytes = lib.isa_ekv_forward_workspace(M, K, O)
    ws = _workspace(ws_bytes, dev, workspace)
    with _hip.on_device(dev):
        rc = lib.isa_ekv_forward(_ptr(x32), _ptr(wp32), _ptr(wn32), fwd_records.data_ptr(), M, K, O,
                                 int(n_entries), float(delta_min), float(delta_max), float(v_sat),
                                 float(out_min), float(out_max), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                 _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_forward")
    return out


def lut_forward_noalloc(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, fwd_records: torch.Tensor,
                        n_entries: int, delta_min: float, delta_max: float, v_sat: float, out_min: float,
                        out_max: float, out: torch.Tensor) -> torch.Tensor:
    """lut_forward through isa_ekv_forward_noalloc: the library's own fixed scratch instead of
    a workspace, for callers that cannot allocate (e.g. inside HIP graph capture). The caller
    passes `out` [M, O] fp32 and fp32 contiguous operands, so this function allocates nothing
    either; shapes needing more than NOALLOC_MAX_BYTES of scratch raise."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    for t, name in ((x, "x"), (wpos, "wpos"), (wneg, "wneg"), (out, "out")):
        if t.dtype != torch.float32 or not t.is_contiguous() or (t.numel() and t.data_ptr() % 16):
            raise RuntimeError(f"{name} must be fp32, contiguous and 16-byte aligned")
    _require_cuda(out, "out")
    if tuple(out.shape) != (M, O) or out.device != x.device:
        raise RuntimeError(f"out must be [{M}, {O}] on {x.device}")
    if n_entries > MAX_ENTRIES:
        raise RuntimeError(f"LUT forward supports LUT_DELTA_SIZE <= {MAX_ENTRIES}")
    dev = x.device
    with _hip.on_device(dev):
        rc = lib.isa_ekv_forward_noalloc(_ptr(x), _ptr(wpos), _ptr(wneg), fwd_records.data_ptr(), M, K, O,
                                         int(n_entries), float(delta_min), float(delta_max), float(v_sat),
                                         float(out_min), float(out_max), out.data_ptr(), _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_forward_noalloc")
    return out


def lut_backward(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, grad_out: torch.Tensor,
                 bwd_records: torch.Tensor, n_entries: int, delta_min: float, delta_max: float, v_sat: float,
                 need_grad_x: bool, need_grad_w: bool, workspace: Optional[torch.Tensor] = None):
    """(dX | None, dVth+ | None, dVth- | None), all fp32. workspace: optional caller buffer."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    _require_cuda(grad_out, "grad_out")
    if tuple(grad_out.shape) != (M, O):
        raise RuntimeError(f"grad_out must be [{M}, {O}], got {tuple(grad_out.shape)}")
    if n_entries > MAX_ENTRIES:
        raise RuntimeError(f"LUT backward supports LUT_DELTA_SIZE <= {MAX_ENTRIES}")
    dev = x.device
    gx = torch.empty((M, K), dtype=torch.float32, device=dev) if need_grad_x else None
    gp = torch.empty((O, K), dtype=torch.float32, device=dev) if need_grad_w else None
    gn = torch.empty((O, K), dtype=torch.float32, device=dev) if need_grad_w else None
    if not (need_grad_x or need_grad_w):
        return gx, gp, gn
    x32, wp32, wn32, g32 = (as_kernel_f32(t) for t in (x, wpos, wneg, grad_out))
    ws_bytes = lib.isa_ekv_backward_workspace(M, K, O, int(n_entries), int(need_grad_x), int(need_grad_w))
    ws = _workspace(ws_bytes, dev, workspace)
    with _hip.on_device(dev):
        rc = lib.isa_ekv_backward(_ptr(x32), _ptr(wp32), _ptr(wn32), _ptr(g32), bwd_records.data_ptr(), M, K, O,
                                  int(n_entries), float(delta_min), float(delta_max), float(v_sat),
                                  _ptr(gx), _ptr(gp), _ptr(gn), ws.data_ptr(), ws.numel(),
                                  _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_backward")
    return gx, gp, gn


def _exact_params(params) -> ctypes.Array:
    """{n, U_T, I_S, V_D} as the library's double[4]."""
    return (ctypes.c_double * 4)(*[float(v) for v in params])


def exact_forward(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor,
                  params: Tuple[float, float, float, float], v_sat: float) -> torch.Tensor:
    """Idiff[M, O] fp32 by the exact EKV formula (no clamp)."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    dev = x.device
    out = torch.empty((M, O), dtype=torch.float32, device=dev)
    if M == 0 or O == 0:
        return out
    x32, wp32, wn32 = as_kernel_f32(x), as_kernel_f32(wpos), as_kernel_f32(wneg)
    ws = _workspace(lib.isa_ekv_exact_forward_workspace(M, K, O), dev)
    with _hip.on_device(dev):
        rc = lib.isa_ekv_exact_forward(_ptr(x32), _ptr(wp32), _ptr(wn32), M, K, O, _exact_params(params),
                                       float(v_sat), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                       _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_exact_forward")
    return out


def exact_backward(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, grad_out: torch.Tensor,
                   params: Tuple[float, float, float, float], v_sat: float, need_grad_x: bool, need_grad_w: bool):
    """(dX | None, dVth+ | None, dVth- | None) of sum(grad_out * Idiff), exact formula, fp32."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    _require_cuda(grad_out, "grad_out")
    if tuple(grad_out.shape) != (M, O):
        raise RuntimeError(f"grad_out must be [{M}, {O}], got {tuple(grad_out.shape)}")
    dev = x.device
    gx = torch.empty((M, K), dtype=torch.float32, device=dev) if need_grad_x else None
    gp = torch.empty((O, K), dtype=torch.float32, device=dev) if need_grad_w else None
    gn = torch.empty((O, K), dtype=torch.float32, device=dev) if need_grad_w else None
    if not (need_grad_x or need_grad_w):
        return gx, gp, gn
    x32, wp32, wn32, g32 = (as_kernel_f32(t) for t in (x, wpos, wneg, grad_out))
    ws = _workspace(lib.isa_ekv_exact_backward_workspace(M, K, O, int(need_grad_x), int(need_grad_w)), dev)
    with _hip.on_device(dev):
        rc = lib.isa_ekv_exact_backward(_ptr(x32), _ptr(wp32), _ptr(wn32), _ptr(g32), M, K, O,
                                        _exact_params(params), float(v_sat), _ptr(gx), _ptr(gp), _ptr(gn),
                                        ws.data_ptr(), ws.numel(), _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_exact_backward")
    return gx, gp, gn


def _glue_struct(in_affine, in_range, r_tia, y_range, adc_scale, adc_shift, stat_abs_max=None,
                 stat_total=None, r_log_scale=None, r_log_range=(0.0, 0.0)) -> "_hip.Glue":
    g = _hip.Glue()
    g.in_affine = _ptr(in_affine)
    g.in_lo, g.in_hi = (float(v) for v in in_range)
    g.r_tia = _ptr(r_tia)
    g.y_lo, g.y_hi = (float(v) for v in y_range)
    g.adc_scale = _ptr(adc_scale)
    g.adc_shift = _ptr(adc_shift)
    g.stat_abs_max = _ptr(stat_abs_max)
    g.stat_total = _ptr(stat_total)
    g.r_log_scale = _ptr(r_log_scale)
    g.r_log_lo, g.r_log_hi = (float(v) for v in r_log_range)
    return g


def _stat_buffer(t: Optional[torch.Tensor], dtype: torch.dtype, name: str, device) -> Optional[torch.Tensor]:
    """An output-statistics buffer the library updates in place: one contiguous element."""
    if t is None:
        return None
    _require_cuda(t, name)
    if t.device != device or t.dtype != dtype or t.numel() != 1 or not t.is_contiguous():
        raise RuntimeError(f"{name} must be one contiguous {dtype} element on {device}")
    return t


def _glue_operand(t: Optional[torch.Tensor], numel: int, name: str, device) -> Optional[torch.Tensor]:
    if t is None:
        return None
    _require_cuda(t, name)
    if t.device != device:
        raise RuntimeError(f"{name} must be on {device}")
    # only the data pointer reaches the library: no autograd view is needed
    if not (t.dtype is torch.float32 and t.is_contiguous() and not t.data_ptr() & 15):
        t = as_kernel_f32(t.detach().reshape(-1))
    if t.numel() != numel:
        raise RuntimeError(f"{name} must have {numel} elements, got {t.numel()}")
    return t


def lut_layer_forward(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, fwd_records: torch.Tensor,
                      n_entries: int, delta_min: float, delta_max: float, v_sat: float, idiff_min: float,
                      idiff_max: float, *, in_affine: Optional[torch.Tensor] = None, in_range=(0.0, 4.0),
                      r_tia: Optional[torch.Tensor] = None, y_range=(-4.0, 4.0),
                      adc_scale: Optional[torch.Tensor] = None, adc_shift: Optional[torch.Tensor] = None,
                      stat_abs_max: Optional[torch.Tensor] = None, stat_total: Optional[torch.Tensor] = None,
                      r_log_scale: Optional[torch.Tensor] = None, r_log_range=(-2.0, 2.0),
                      workspace: Optional[torch.Tensor] = None):
    """(out, idiff) of the LUT projection with its glue fused: x -> clamp(x*s + b) ->
    Idiff (clamped to [idiff_min, idiff_max]) -> y = clamp(Idiff * r) -> y * adc_scale +
    adc_shift, with the gain r = r_tia, or r_tia * exp(clamp(r_log_scale, *r_log_range)) when
    r_log_scale is given (CIMLinear's r_tia_base and learnable log scale). stat_abs_max (fp32)
    and stat_total (fp64), one element each, are CIMLinear's output statistics
    (cim.py:194-198), updated in place: maximum with max|y|, plus M * O. workspace: optional
    caller buffer."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    if n_entries > MAX_ENTRIES:
        raise RuntimeError(f"LUT forward supports LUT_DELTA_SIZE <= {MAX_ENTRIES}")
    dev = x.device
    aff = _glue_operand(in_affine, 2, "in_affine", dev)
    r = _glue_operand(r_tia, 1, "r_tia", dev)
    r_ls = _glue_operand(r_log_scale, 1, "r_log_scale", dev)
    if r_ls is not None and r is None:
        raise RuntimeError("r_log_scale needs r_tia (the base gain)")
    a_s = _glue_operand(adc_scale, O, "adc_scale", dev)
    a_c = _glue_operand(adc_shift, O, "adc_shift", dev)
    if (a_s is None) != (a_c is None):
        raise RuntimeError("adc_scale and adc_shift go together")
    s_max = _stat_buffer(stat_abs_max, torch.float32, "stat_abs_max", dev)
    s_tot = _stat_buffer(stat_total, torch.float64, "stat_total", dev)
    out = torch.empty((M, O), dtype=torch.float32, device=dev)
    idiff = torch.empty((M, O), dtype=torch.float32, device=dev)
    if M == 0 or O == 0:
        return out, idiff
    x32, wp32, wn32 = as_kernel_f32(x), as_kernel_f32(wpos), as_kernel_f32(wneg)
    glue = _glue_struct(aff, in_range, r, y_range, a_s, a_c, s_max, s_tot, r_ls, r_log_range)
    ws = _workspace(lib.isa_ekv_layer_forward_workspace(M, K, O), dev, workspace)
    with _hip.on_device(dev):
        rc = lib.isa_ekv_layer_forward(_ptr(x32), _ptr(wp32), _ptr(wn32), fwd_records.data_ptr(), M, K, O,
                                       int(n_entries), float(delta_min), float(delta_max), float(v_sat),
                                       float(idiff_min), float(idiff_max), ctypes.byref(glue), idiff.data_ptr(),
                                       out.data_ptr(), ws.data_ptr(), ws.numel(), _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_layer_forward")
    return out, idiff


def lut_layer_backward(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, grad_out: torch.Tensor,
                       idiff: torch.Tensor, bwd_records: torch.Tensor, n_entries: int, delta_min: float,
                       delta_max: float, v_sat: float, *, need_grad_x: bool, need_grad_w: bool,
                       in_affine: Optional[torch.Tensor] = None, in_range=(0.0, 4.0),
                       r_tia: Optional[torch.Tensor] = None, y_range=(-4.0, 4.0),
                       adc_scale: Optional[torch.Tensor] = None, adc_shift: Optional[torch.Tensor] = None,
                       need_in_affine: bool = False, need_r_tia: bool = False, need_adc: bool = False,
                       r_log_scale: Optional[torch.Tensor] = None, r_log_range=(-2.0, 2.0),
                       need_r_log_scale: bool = False, workspace: Optional[torch.Tensor] = None):
    """Gradients of lut_layer_forward's out: dict with dx, dvth_pos, dvth_neg, d_in_affine,
    d_r_tia (for the gain r), d_r_log_scale, d_adc_scale, d_adc_shift (None where not
    requested), all fp32. workspace: optional caller buffer."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    _require_cuda(grad_out, "grad_out")
    if tuple(grad_out.shape) != (M, O) or tuple(idiff.shape) != (M, O):
        raise RuntimeError(f"grad_out and idiff must be [{M}, {O}]")
    if n_entries > MAX_ENTRIES:
        raise RuntimeError(f"LUT backward supports LUT_DELTA_SIZE <= {MAX_ENTRIES}")
    dev = x.device
    aff = _glue_operand(in_affine, 2, "in_affine", dev)
    r = _glue_operand(r_tia, 1, "r_tia", dev)
    r_ls = _glue_operand(r_log_scale, 1, "r_log_scale", dev)
    if r_ls is not None and r is None:
        raise RuntimeError("r_log_scale needs r_tia (the base gain)")
    a_s = _glue_operand(adc_scale, O, "adc_scale", dev)
    a_c = _glue_operand(adc_shift, O, "adc_shift", dev)
    need_in_affine = need_in_affine and aff is not None
    need_x = need_grad_x or need_in_affine  # the mapping's gradient is formed from dX
    f32 = dict(dtype=torch.float32, device=dev)
    res = {
        "dx": torch.empty((M, K), **f32) if need_x else None,
        "dvth_pos": torch.empty((O, K), **f32) if need_grad_w else None,
        "dvth_neg": torch.empty((O, K), **f32) if need_grad_w else None,
        "d_in_affine": torch.empty(2, **f32) if need_in_affine else None,
        "d_r_tia": torch.empty(1, **f32) if (need_r_tia and r is not None) else None,
        "d_r_log_scale": torch.empty(1, **f32) if (need_r_log_scale and r_ls is not None) else None,
        "d_adc_scale": torch.empty(O, **f32) if (need_adc and a_s is not None) else None,
        "d_adc_shift": torch.empty(O, **f32) if (need_adc and a_s is not None) else None,
    }
    grads = _hip.GlueGrads()
    grads.in_affine = _ptr(res["d_in_affine"])
    grads.r_tia = _ptr(res["d_r_tia"])
    grads.adc_scale = _ptr(res["d_adc_scale"])
    grads.adc_shift = _ptr(res["d_adc_shift"])
    grads.r_log_scale = _ptr(res["d_r_log_scale"])
    if not (need_x or need_grad_w or any(res[k] is not None for k in ("d_r_tia", "d_r_log_scale", "d_adc_scale"))):
        return res
    x32, wp32, wn32, g32, id32 = (as_kernel_f32(t) for t in (x, wpos, wneg, grad_out, idiff))
    glue = _glue_struct(aff, in_range, r, y_range, a_s, a_c, r_log_scale=r_ls, r_log_range=r_log_range)
    ws = _workspace(lib.isa_ekv_layer_backward_workspace(M, K, O, int(n_entries), int(need_x), int(need_grad_w)), dev,
                    workspace)
    with _hip.on_device(dev):
        rc = lib.isa_ekv_layer_backward(_ptr(x32), _ptr(wp32), _ptr(wn32), _ptr(g32), _ptr(id32),
                                        bwd_records.data_ptr(), M, K, O, int(n_entries), float(delta_min),
                                        float(delta_max), float(v_sat), ctypes.byref(glue), _ptr(res["dx"]),
                                        _ptr(res["dvth_pos"]), _ptr(res["dvth_neg"]), ctypes.byref(grads),
                                        ws.data_ptr(), ws.numel(), _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_layer_backward")
    if not need_grad_x:
        res["dx"] = None
    return res


def _ids16(t: torch.Tensor, name: str, shape, device) -> torch.Tensor:
    _require_cuda(t, name)
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.device != device:
        raise RuntimeError(f"{name} must be on {device}")
    return t.to(dtype=torch.int16).contiguous()


def _codebook(slopes, intercepts, seg_mode, vg, voltage_min, inverse_step, lookup_min, lookup_max, device):
    for t, name in ((slopes, "slopes"), (intercepts, "intercepts")):
        _require_cuda(t, name)
        if t.device != device:
            raise RuntimeError(f"{name} must be on {device}")
    if slopes.dim() != 2 or intercepts.shape != slopes.shape:
        raise RuntimeError("slope/intercept tables must have matching 2-D shapes [curves, segments]")
    if slopes.shape[0] > 32767:
        raise RuntimeError("the codebook holds at most 32767 curves (int16 state ids)")
    sl, ic = as_kernel_f32(slopes), as_kernel_f32(intercepts)
    v = None
    if seg_mode == _hip.SEG_SEARCH:
        v = as_kernel_f32(vg.reshape(-1))
        if v.numel() != sl.shape[1] + 1:
            raise RuntimeError("vg must have one more point than the tables have segments")
    cb = _hip.Codebook()
    cb.slopes, cb.intercepts = sl.data_ptr(), ic.data_ptr()
    cb.n_seg, cb.n_rows = int(sl.shape[1]), int(sl.shape[0])
    cb.seg_mode = int(seg_mode)
    cb.vg = _ptr(v)
    cb.voltage_min, cb.inverse_step = float(voltage_min), float(inverse_step)
    cb.lookup_min, cb.lookup_max = float(lookup_min), float(lookup_max)
    return cb, (sl, ic, v)  # keep the tensors alive for the call


def measured_forward(x: torch.Tensor, ids_a: torch.Tensor, ids_b: Optional[torch.Tensor], slopes: torch.Tensor,
                     intercepts: torch.Tensor, *, seg_mode: int, vg: Optional[torch.Tensor] = None,
                     voltage_min: float = 0.0, inverse_step: float = 1.0, lookup_min: float = 0.0,
                     lookup_max: float = 4.0, current_scale: float = 1.0, r_tia: torch.Tensor,
                     out_min: float = -4.0, out_max: float = 4.0):
    """(out, out_pre) of the measured-codebook projection, fp32 [M, O]."""
    lib = _hip.load()
    _require_cuda(x, "x")
    if x.dim() != 2:
        raise RuntimeError(f"x must be 2-D [M, K], got shape {tuple(x.shape)}")
    dev = x.device
    M, K = int(x.shape[0]), int(x.shape[1])
    if ids_a.dim() != 2 or ids_a.shape[1] != K:
        raise RuntimeError(f"ids_a must be [O, {K}], got {tuple(ids_a.shape)}")
    O = int(ids_a.shape[0])
    a16 = _ids16(ids_a, "ids_a", (O, K), dev)
    b16 = None if ids_b is None else _ids16(ids_b, "ids_b", (O, K), dev)
    cb, keep = _codebook(slopes, intercepts, seg_mode, vg, voltage_min, inverse_step, lookup_min, lookup_max, dev)
    r = _glue_operand(r_tia, 1, "r_tia", dev)
    out = torch.empty((M, O), dtype=torch.float32, device=dev)
    pre = torch.empty((M, O), dtype=torch.float32, device=dev)
    if M == 0 or O == 0:
        return out, pre
    x32 = as_kernel_f32(x)
    ws = _workspace(lib.isa_ekv_measured_forward_workspace(M, K, O, cb.n_seg, cb.n_rows), dev)
    with _hip.on_device(dev):
        rc = lib.isa_ekv_measured_forward(_ptr(x32), a16.data_ptr(), _ptr(b16), M, K, O, ctypes.byref(cb),
                                          float(current_scale), r.data_ptr(), float(out_min), float(out_max),
                                          pre.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                          _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_measured_forward")
    del keep
    return out, pre


def measured_backward(x: torch.Tensor, ids_a: torch.Tensor, ids_b: Optional[torch.Tensor], slopes: torch.Tensor,
                      intercepts: torch.Tensor, grad_out: torch.Tensor, out_pre: torch.Tensor, *, seg_mode: int,
                      vg: Optional[torch.Tensor] = None, voltage_min: float = 0.0, inverse_step: float = 1.0,
                      lookup_min: float = 0.0, lookup_max: float = 4.0, current_scale: float = 1.0,
                      r_tia: torch.Tensor, out_min: float = -4.0, out_max: float = 4.0) -> torch.Tensor:
    """dX [M, K] fp32 of the measured-codebook projection's output."""
    lib = _hip.load()
    dev = x.device
    M, K = int(x.shape[0]), int(x.shape[1])
    O = int(ids_a.shape[0])
    a16 = _ids16(ids_a, "ids_a", (O, K), dev)
    b16 = None if ids_b is None else _ids16(ids_b, "ids_b", (O, K), dev)
    if tuple(grad_out.shape) != (M, O) or tuple(out_pre.shape) != (M, O):
        raise RuntimeError(f"grad_out and out_pre must be [{M}, {O}]")
    cb, keep = _codebook(slopes, intercepts, seg_mode, vg, voltage_min, inverse_step, lookup_min, lookup_max, dev)
    r = _glue_operand(r_tia, 1, "r_tia", dev)
    gx = torch.empty((M, K), dtype=torch.float32, device=dev)
    x32, g32, p32 = as_kernel_f32(x), as_kernel_f32(grad_out), as_kernel_f32(out_pre)
    ws = _workspace(lib.isa_ekv_measured_backward_workspace(M, K, O, cb.n_seg, cb.n_rows), dev)
    with _hip.on_device(dev):
        rc = lib.isa_ekv_measured_backward(_ptr(x32), a16.data_ptr(), _ptr(b16), M, K, O, ctypes.byref(cb),
                                           float(current_scale), _ptr(g32), _ptr(p32), r.data_ptr(),
                                           float(out_min), float(out_max), gx.data_ptr(), ws.data_ptr(), ws.numel(),
                                           _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_measured_backward")
    del keep
    return gx


def probe_lds_gather(window_records: int, record_bytes: int = 8, iterations: int = 2048,
                     device: Optional[torch.device] = None, repeats: int = 5, clock: Optional[dict] = None) -> float:
    """Average nanoseconds per wave-level LDS gather per CU for random `record_bytes`
    gathers whose 64 lanes draw indices uniformly from `window_records` entries (one
    `isa_ekv_probe_lds_gather` launch per repeat, after one untimed launch, timed with HIP
    events on the current stream). A measurement aid for the table kernels' LDS bound.
    clock: a dict that receives the shader clock the CUs sustained during the timed launches
    ("ghz": median over blocks and launches of clock64 cycles / wall_clock64 time)."""
    lib = _hip.load()
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    out = torch.empty(2 * cus * 1024, dtype=torch.float32, device=dev)
    clocks = torch.zeros((repeats, 2 * cus, 2), dtype=torch.int64, device=dev)
    per_cu = ctypes.c_int(0)
    khz = ctypes.c_int(0)
    with _hip.on_device(dev):
        stream = _hip.stream_handle(dev)

        def launch(slot):
            ptr = None if slot is None else clocks[slot].data_ptr()
            rc = lib.isa_ekv_probe_lds_gather(int(window_records), int(record_bytes), int(iterations),
                                              out.data_ptr(), out.numel(), ctypes.byref(per_cu), ptr,
                                              ctypes.byref(khz), stream)
            _hip.check(rc, "isa_ekv_probe_lds_gather")

        launch(None)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for r in range(repeats):
            launch(r if clock is not None else None)
        e1.record()
        torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / repeats
    if clock is not None and khz.value > 0:
        c = clocks.reshape(-1, 2).double()
        ghz = c[:, 0] / (c[:, 1] / (khz.value * 1e3)) / 1e9
        clock["ghz"] = float(ghz.median())
        clock["wall_clock_khz"] = khz.value
    return ms * 1e6 / per_cu.value


VALU_MIXES = {"fma": 0, "ranked_backward": 1, "forward": 2, "forward_int_address": 3}


def probe_valu_issue(mix: str, iterations: int = 4096, device: Optional[torch.device] = None,
                     repeats: int = 3) -> dict:
    """VALU wave-instructions a CU issues per shader cycle for one of the table kernels'
    instruction mixes replayed on registers only (isa_ekv_probe_valu_issue): "fma" (32
    independent fma chains), "ranked_backward", "forward" or "forward_int_address" (the forward's
    cell with the cvt and shift-add record address in place of the float-bits one). One untimed launch, then
    `repeats` launches; returns {"instr_per_cu_cycle": median over CUs and launches of the CU's
    loop instructions / the shader cycles of the interval its two blocks kept it busy, "ghz":
    the CUs' shader clock (clock64 / wall_clock64), "ms": mean launch time by HIP events, ...}.
    A measurement aid: the issue rate a kernel of that mix cannot exceed."""
    lib = _hip.load()
    code = VALU_MIXES[mix]
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    waves = 8 if mix.startswith("forward") else 16
    out = torch.empty(2 * cus * 64 * waves, dtype=torch.float32, device=dev)
    clocks = torch.zeros((repeats, 2 * cus, 4), dtype=torch.int64, device=dev)
    g = torch.Generator().manual_seed(1)
    tok = torch.stack([torch.rand(64, generator=g) * 3000.0 + 600.0, torch.rand(64, generator=g) * 0.5 + 0.5,
                       -torch.rand(64, generator=g) * 0.1, torch.zeros(64)], dim=1).to(dev).contiguous()
    per_cu = ctypes.c_double(0.0)
    khz = ctypes.c_int(0)
    with _hip.on_device(dev):
        stream = _hip.stream_handle(dev)

        def launch(slot):
            ptr = None if slot is None else clocks[slot].data_ptr()
            rc = lib.isa_ekv_probe_valu_issue(code, int(iterations), tok.data_ptr(), out.data_ptr(), out.numel(),
                                              ptr, ctypes.byref(per_cu), ctypes.byref(khz), stream)
            _hip.check(rc, "isa_ekv_probe_valu_issue")

        launch(None)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for r in range(repeats):
            launch(r)
        e1.record()
        torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / repeats
    res = {"ms": ms, "instr_per_cu": per_cu.value, "mix": mix}
    if khz.value <= 0:
        raise RuntimeError("isa_ekv_probe_valu_issue: the device reports no wall clock rate")
    # per launch and CU: the interval its blocks kept it busy (first start to last end, wall
    # ticks) in shader cycles at its blocks' clock; the CU's loop instructions over that
    c = clocks.cpu().double()
    rates, ghzs = [], []
    per_block_instr = per_cu.value / 2.0
    for r in range(repeats):
        groups = {}
        for cyc, span, start, cu in c[r].tolist():
            groups.setdefault(int(cu), []).append((cyc, span, start))
        for blocks in groups.values():
            t0 = min(b[2] for b in blocks)
            t1 = max(b[2] + b[1] for b in blocks)
            ghz = sum(b[0] for b in blocks) / (sum(b[1] for b in blocks) / (khz.value * 1e3)) / 1e9
            rates.append(per_block_instr * len(blocks) / ((t1 - t0) / (khz.value * 1e3) * ghz * 1e9))
            ghzs.append(ghz)
    rt = torch.tensor(rates, dtype=torch.float64)
    res["instr_per_cu_cycle"] = float(rt.median())
    res["instr_per_cu_cycle_max"] = float(rt.max())
    res["ghz"] = float(torch.tensor(ghzs, dtype=torch.float64).median())
    res["blocks_per_cu"] = float(c.shape[1] / len(groups))
    # the same over the whole launch time (HIP events: dispatch ramp and tail included)
    res["instr_per_cu_cycle_launch"] = per_cu.value / (ms * 1e-3 * res["ghz"] * 1e9)
    return res
