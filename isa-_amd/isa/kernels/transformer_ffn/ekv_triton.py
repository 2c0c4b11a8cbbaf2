"""Exact-formula fused EKV matmul: autograd glue and public entry.

Module name and API follow the reference (`src/isa/kernels/transformer_ffn/ekv_triton.py:
172-214`), so `CIMLinear` with `ekv_approx != "lut"` and the other callers of
`TritonEKVMatmulFn` / `triton_ekv_matmul` import it unchanged. There is no Triton here:
forward and backward run the exact-formula HIP kernels of libisa_ekv_hip.so, which
evaluate the EKV current per cell,

    I(v, vth) = I_S [sp(u1)^2 - sp(u2)^2] / (1 + v/V_sat),
    u1 = (v - vth)/(2 n U_T),  u2 = u1 - V_D/(2 n U_T),

with no table and no clamp. Behaviour follows the reference:

* forward: Idiff[M, O] = sum_k (I(x, wpos) - I(x, wneg)), returned in x's dtype
  (`ekv_triton.py:175-191`); `cfg` needs only n, U_T, I_S, V_D and V_sat;
* backward: dX only when x needs a gradient, dWpos and dWneg always, each cast back to
  its input's dtype (`ekv_triton.py:193-211`). The reference's Triton block sizes
  (`TRITON_BLOCK_M/O/K`) are accepted and ignored.
"""

from __future__ import annotations

from typing import Any, Dict

import torch

from isa.kernels.transformer_ffn import ops


def _params(cfg: Dict[str, Any]):
    return (float(cfg["n"]), float(cfg["U_T"]), float(cfg["I_S"]), float(cfg["V_D"])), float(cfg["V_sat"])


class TritonEKVMatmulFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, cfg: Dict[str, Any]):
        params, v_sat = _params(cfg)
        out = ops.exact_forward(x, wpos, wneg, params, v_sat)
        ctx.save_for_backward(x, wpos, wneg)
        ctx.cfg = dict(cfg)
        return out.to(dtype=x.dtype)

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        x, wpos, wneg = ctx.saved_tensors
        params, v_sat = _params(ctx.cfg)
        need_x = bool(ctx.needs_input_grad[0])
        gx, gp, gn = ops.exact_backward(x, wpos, wneg, grad_out, params, v_sat, need_x, True)
        return (
            gx.to(dtype=x.dtype) if gx is not None else None,
            gp.to(dtype=wpos.dtype),
            gn.to(dtype=wneg.dtype),
            None,
        )


def triton_ekv_matmul(x: torch.Tensor, wpos: torch.Tensor, wneg: torch.Tensor, cfg: Dict[str, Any]) -> torch.Tensor:
    """Idiff[M, O] = sum_k (I(x - wpos) - I(x - wneg)) by the exact formula; ekv_triton.py:211-214."""
    return TritonEKVMatmulFn.apply(x, wpos, wneg, cfg)
