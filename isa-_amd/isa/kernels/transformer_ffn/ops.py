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

MAX_ENTRIES_FORWARD = 16384
MAX_ENTRIES_BACKWARD = 8192


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")


def as_kernel_f32(t: torch.Tensor) -> torch.Tensor:
    """fp32, contiguous and 16-byte aligned (a copy only when needed)."""
    t = t.to(dtype=torch.float32).contiguous()
    if t.numel() and t.data_ptr() % 16:
        t = t.clone()
    return t


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


def build_plain_tables(params: Tuple[float, float, float, float], delta_min: float, delta_max: float,
                       size: int, device: torch.device, bf16: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """(table_i, table_ddelta), each [size], evaluated on the device (delta_lut.py:12-35)."""
    lib = _hip.load()
    dtype = torch.bfloat16 if bf16 else torch.float32
    layout = _hip.LUT_PLAIN_BF16 if bf16 else _hip.LUT_PLAIN_F32
    buf = torch.empty(2 * size, dtype=dtype, device=device)
    arr = (ctypes.c_double * 4)(*[float(v) for v in params])
    with torch.cuda.device(device):
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
    with torch.cuda.device(table_i.device):
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
                out_min: float, out_max: float) -> torch.Tensor:
    """Idiff[M, O] fp32 (clamped to [out_min, out_max])."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    if n_entries > MAX_ENTRIES_FORWARD:
        raise RuntimeError(f"LDS-resident LUT forward supports LUT_DELTA_SIZE <= {MAX_ENTRIES_FORWARD}")
    dev = x.device
    out = torch.empty((M, O), dtype=torch.float32, device=dev)
    if M == 0 or O == 0:
        return out
    x32, wp32, wn32 = as_kernel_f32(x), as_kernel_f32(wpos), as_kernel_f32(wneg)
    ws_bytes = lib.isa_ekv_forward_workspace(M, K, O)
    ws = _workspace(ws_bytes, dev)
    with torch.cuda.device(dev):
        rc = lib.isa_ekv_forward(_ptr(x32), _ptr(wp32), _ptr(wn32), fwd_records.data_ptr(), M, K, O,
                                 int(n_entries), float(delta_min), float(delta_max), float(v_sat),
                                 float(out_min), float(out_max), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                 _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_forward")
    return out


def lut_backward(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, grad_out: torch.Tensor,
                 bwd_records: torch.Tensor, n_entries: int, delta_min: float, delta_max: float, v_sat: float,
                 need_grad_x: bool, need_grad_w: bool):
    """(dX | None, dVth+ | None, dVth- | None), all fp32."""
    lib = _hip.load()
    M, K, O = _check_operands(x, wpos, wneg)
    _require_cuda(grad_out, "grad_out")
    if tuple(grad_out.shape) != (M, O):
        raise RuntimeError(f"grad_out must be [{M}, {O}], got {tuple(grad_out.shape)}")
    if n_entries > MAX_ENTRIES_BACKWARD:
        raise RuntimeError(f"shared backward supports LUT_DELTA_SIZE <= {MAX_ENTRIES_BACKWARD}")
    dev = x.device
    gx = torch.empty((M, K), dtype=torch.float32, device=dev) if need_grad_x else None
    gp = torch.empty((O, K), dtype=torch.float32, device=dev) if need_grad_w else None
    gn = torch.empty((O, K), dtype=torch.float32, device=dev) if need_grad_w else None
    if not (need_grad_x or need_grad_w):
        return gx, gp, gn
    x32, wp32, wn32, g32 = (as_kernel_f32(t) for t in (x, wpos, wneg, grad_out))
    ws_bytes = lib.isa_ekv_backward_workspace(M, K, O, int(n_entries), int(need_grad_x), int(need_grad_w))
    ws = _workspace(ws_bytes, dev)
    with torch.cuda.device(dev):
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
    with torch.cuda.device(dev):
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
    with torch.cuda.device(dev):
        rc = lib.isa_ekv_exact_backward(_ptr(x32), _ptr(wp32), _ptr(wn32), _ptr(g32), M, K, O,
                                        _exact_params(params), float(v_sat), _ptr(gx), _ptr(gp), _ptr(gn),
                                        ws.data_ptr(), ws.numel(), _hip.stream_handle(dev))
    _hip.check(rc, "isa_ekv_exact_backward")
    return gx, gp, gn
