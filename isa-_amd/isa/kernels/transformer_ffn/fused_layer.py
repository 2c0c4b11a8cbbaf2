"""CIM layer with its elementwise glue fused into the LUT kernels.

No reference counterpart as a module: the reference runs the projection
(`triton_lut_ekv_matmul`) and then separate PyTorch ops for the input voltage mapping
(`cim.py:37-39`), the learnable TIA gain and output clamp (`cim.py:190-193`) and
PhysicalFFN's ADC affine (`cim.py:243`), and CIMLinear's optional output statistics
(`cim.py:194-198`). Here one library call does all of them in the forward (prep prologue,
kernel epilogue) and one call the backward (a gradient prep pass
for the clamp mask, TIA and ADC gradients, and the mapping's backward inside the dX
reduction). Values and gradients equal the unfused composition's up to the order of the
parameter-gradient sums.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from isa.approximations.delta_lut import get_packed_tables, lut_range
from isa.kernels.transformer_ffn import ops


class FusedCIMLayerFn(torch.autograd.Function):
    """out = adc(clamp(clamp(Idiff(map(x)), lo, hi) * r, lo, hi)) with the gain r = r_tia, or
    r_tia * exp(clamp(r_log_scale, *r_log_range)) when r_log_scale is given; the optional
    pieces (in_affine, r_tia, r_log_scale, adc_scale/adc_shift) may be None. stats: None or the
    (abs_max fp32, total fp64) buffers the forward updates in place."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, in_affine: Optional[torch.Tensor],
                r_tia: Optional[torch.Tensor], adc_scale: Optional[torch.Tensor], adc_shift: Optional[torch.Tensor],
                r_log_scale: Optional[torch.Tensor], cfg: Dict[str, Any], in_range: Tuple[float, float],
                r_log_range: Tuple[float, float], stats=None):
        delta_min, delta_max, size = lut_range(cfg)
        lo = float(cfg.get("V_signed_min", -4.0))
        hi = float(cfg.get("V_signed_max", 4.0))
        fwd_records, bwd_records = get_packed_tables(cfg, x.device)
        out, idiff = ops.lut_layer_forward(
            x, wpos, wneg, fwd_records, size, delta_min, delta_max, float(cfg["V_sat"]), lo, hi,
            in_affine=in_affine, in_range=in_range, r_tia=r_tia, y_range=(lo, hi),
            adc_scale=adc_scale, adc_shift=adc_shift,
            stat_abs_max=stats[0] if stats else None, stat_total=stats[1] if stats else None,
            r_log_scale=r_log_scale, r_log_range=r_log_range)
        ctx.save_for_backward(x, wpos, wneg, idiff, in_affine, r_tia, adc_scale, adc_shift, r_log_scale)
        ctx.bwd_records = bwd_records
        ctx.meta = (delta_min, delta_max, size, float(cfg["V_sat"]), lo, hi, tuple(in_range), tuple(r_log_range))
        ctx.shared_backward = bool(cfg.get("CUDA_SHARED_BACKWARD", False))
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        x, wpos, wneg, idiff, in_affine, r_tia, adc_scale, adc_shift, r_log_scale = ctx.saved_tensors
        delta_min, delta_max, size, v_sat, lo, hi, in_range, r_log_range = ctx.meta
        if ctx.shared_backward and size > ops.MAX_ENTRIES_BACKWARD:  # the reference's limit and message
            raise RuntimeError("CUDA shared EKV backward requires LUT_DELTA_SIZE <= 8192")
        need = ctx.needs_input_grad
        res = ops.lut_layer_backward(
            x, wpos, wneg, grad_out, idiff, ctx.bwd_records, size, delta_min, delta_max, v_sat,
            need_grad_x=bool(need[0]), need_grad_w=bool(need[1] or need[2]),
            in_affine=in_affine, in_range=in_range, r_tia=r_tia, y_range=(lo, hi),
            adc_scale=adc_scale, adc_shift=adc_shift,
            need_in_affine=bool(need[3]), need_r_tia=bool(need[4]), need_adc=bool(need[5] or need[6]),
            r_log_scale=r_log_scale, r_log_range=r_log_range, need_r_log_scale=bool(need[7]))

        def cast(t, like):
            if t is None or like is None:
                return None
            if t.shape != like.shape:
                t = t.reshape(like.shape)
            return t if t.dtype is like.dtype else t.to(dtype=like.dtype)

        return (
            cast(res["dx"], x) if need[0] else None,
            cast(res["dvth_pos"], wpos) if need[1] else None,
            cast(res["dvth_neg"], wneg) if need[2] else None,
            cast(res["d_in_affine"], in_affine) if need[3] else None,
            cast(res["d_r_tia"], r_tia) if need[4] else None,
            cast(res["d_adc_scale"], adc_scale) if need[5] else None,
            cast(res["d_adc_shift"], adc_shift) if need[6] else None,
            cast(res["d_r_log_scale"], r_log_scale) if need[7] else None,
            None,
            None,
            None,
            None,
        )


def fused_cim_layer(x2d: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, cfg: Dict[str, Any], *,
                    in_affine: Optional[torch.Tensor] = None, in_range: Tuple[float, float] = (0.0, 4.0),
                    r_tia: Optional[torch.Tensor] = None, adc_scale: Optional[torch.Tensor] = None,
                    adc_shift: Optional[torch.Tensor] = None,
                    stats: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                    r_log_scale: Optional[torch.Tensor] = None,
                    r_log_range: Tuple[float, float] = (-2.0, 2.0)) -> torch.Tensor:
    """[M, K] -> [M, O] fp32 through FusedCIMLayerFn; stats = (abs_max, total) buffers to
    update with the layer's output statistics, or None. With r_log_scale, r_tia is the base
    gain and the layer applies r_tia * exp(clamp(r_log_scale, *r_log_range)) itself
    (CIMLinear.r_tia, cim.py:74-77), returning r_log_scale's gradient."""
    return FusedCIMLayerFn.apply(x2d, wpos, wneg, in_affine, r_tia, adc_scale, adc_shift, r_log_scale, cfg,
                                 (float(in_range[0]), float(in_range[1])),
                                 (float(r_log_range[0]), float(r_log_range[1])), stats)
