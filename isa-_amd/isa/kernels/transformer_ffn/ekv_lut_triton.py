"""LUT-interpolated fused EKV matmul: autograd glue and public entry.

The module name and API are kept from the reference
(`src/isa/kernels/transformer_ffn/ekv_lut_triton.py:131-224`) so `CIMLinear` and other
callers import it unchanged; there is no Triton here. Forward and backward both run the
HIP kernels of libisa_ekv_hip.so. Behaviour follows the reference:

* forward: builds or fetches the tables for `cfg`, computes Idiff[M, O] in fp32 clamped to
  [V_signed_min, V_signed_max] (`ekv_lut_triton.py:136-161`);
* backward: gradients for the inputs that need them, cast back to their dtypes, with the
  reference's LUT_DELTA_SIZE <= 8192 limit and message when `CUDA_SHARED_BACKWARD` is set
  (`:171-191`). With it off the reference runs its Triton backward (split-M atomics,
  `:193-218`) at any table size; here the same deterministic HIP backward serves both
  settings, reading tables past 8192 entries from global memory.
"""

from __future__ import annotations

from typing import Any, Dict

import torch

from isa.approximations.delta_lut import get_ekv_lut_tables, get_packed_tables, lut_range
from isa.kernels.transformer_ffn import ops


def _meta(cfg: Dict[str, Any]):
    delta_min, delta_max, delta_size = lut_range(cfg)
    v_sat = float(cfg["V_sat"])
    v_out_min = float(cfg.get("V_signed_min", -4.0))
    v_out_max = float(cfg.get("V_signed_max", 4.0))
    return delta_min, delta_max, delta_size, v_sat, v_out_min, v_out_max


class LUTTritonEKVMatmulFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, cfg: Dict[str, Any]):
        delta_min, delta_max, delta_size, v_sat, v_out_min, v_out_max = _meta(cfg)
        table_i, table_ddelta = get_ekv_lut_tables(cfg, x.device)
        fwd_records, bwd_records = get_packed_tables(cfg, x.device)
        out = ops.lut_forward(x, wpos, wneg, fwd_records, delta_size, delta_min, delta_max, v_sat,
                              v_out_min, v_out_max)
        ctx.save_for_backward(x, wpos, wneg, table_i, table_ddelta)
        ctx.bwd_records = bwd_records
        ctx.cfg = dict(cfg)
        ctx.meta = (delta_min, delta_max, delta_size, v_sat)
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        x, wpos, wneg, _table_i, _table_ddelta = ctx.saved_tensors
        delta_min, delta_max, delta_size, v_sat = ctx.meta
        if bool(ctx.cfg.get("CUDA_SHARED_BACKWARD", False)) and delta_size > ops.MAX_ENTRIES_BACKWARD:
            raise RuntimeError("CUDA shared EKV backward requires LUT_DELTA_SIZE <= 8192")
        need_x = bool(ctx.needs_input_grad[0])
        need_w = bool(ctx.needs_input_grad[1] or ctx.needs_input_grad[2])
        gx, gp, gn = ops.lut_backward(x, wpos, wneg, grad_out, ctx.bwd_records, delta_size, delta_min, delta_max,
                                      v_sat, need_x, need_w)
        return (
            gx.to(dtype=x.dtype) if gx is not None else None,
            gp.to(dtype=wpos.dtype) if gp is not None else None,
            gn.to(dtype=wneg.dtype) if gn is not None else None,
            None,
        )


def triton_lut_ekv_matmul(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, cfg: Dict[str, Any]) -> torch.Tensor:
    """Idiff[M, O] = clamp(sum_k (L(x - wpos) - L(x - wneg)) / (1 + x/V_sat)); ekv_lut_triton.py:221-224."""
    return LUTTritonEKVMatmulFn.apply(x, wpos, wneg, cfg)
