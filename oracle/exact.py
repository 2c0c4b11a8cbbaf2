"""Exact-formula Flash-EKV path restated from the reference (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this module. It serves three purposes:

* the closed form that pins the LUT oracle (as N grows the LUT forward and backward
  converge to it), restated from ``src/isa/device_models/flash_transistor.py:22-131``;
* the reference's PyTorch CPU path, timed as the CPU baseline: ``CIMLinear.forward``'s
  CPU branch chunked over 64 outputs (``src/isa/operators/cim.py:201-214``) with
  ``EKVDiffCurrentFn``'s analytic backward (``flash_transistor.py:95-131``);
* the float64 checker of the exact-formula kernels (``diff_current_f64`` and
  ``diff_current_grads_f64``): the same closed form and analytic gradients evaluated in
  the inputs' dtype, without the fp32 cast of ``flash_transistor.py:107``, in the
  products of ``kernels/transformer_ffn/ekv_triton.py:69-169``.
"""

from __future__ import annotations

from typing import Dict, Optional

import torch
import torch.nn.functional as F


def _sig_from_sp(sp: torch.Tensor) -> torch.Tensor:
    """flash_transistor.py:27-29."""
    return torch.where(sp > 20.0, torch.ones_like(sp), 1.0 - torch.exp(-sp))


def ekv_current(vgs, vth, cfg):
    """flash_transistor.py:32-46: I = I_S[sp(u1)^2 - sp(u2)^2] / (1 + V/V_sat)."""
    inv_2nut = 1.0 / (2.0 * cfg["n"] * cfg["U_T"])
    u1 = (vgs - vth) * inv_2nut
    u2 = (vgs - vth - cfg["V_D"]) * inv_2nut
    sp1 = F.softplus(u1)
    sp2 = F.softplus(u2)
    return cfg["I_S"] * (sp1 * sp1 - sp2 * sp2) / (1.0 + vgs / cfg["V_sat"])


def ekv_current_grad_v(vgs, vth, cfg):
    """flash_transistor.py:49-68."""
    inv_2nut = 1.0 / (2.0 * cfg["n"] * cfg["U_T"])
    u1 = (vgs - vth) * inv_2nut
    u2 = (vgs - vth - cfg["V_D"]) * inv_2nut
    sp1 = F.softplus(u1)
    sp2 = F.softplus(u2)
    sig1 = _sig_from_sp(sp1)
    sig2 = _sig_from_sp(sp2)
    num = 2.0 * sp1 * sig1 * inv_2nut - 2.0 * sp2 * sig2 * inv_2nut
    basic = sp1 * sp1 - sp2 * sp2
    denom = 1.0 + vgs / cfg["V_sat"]
    return cfg["I_S"] * (num / denom - basic / (cfg["V_sat"] * denom * denom))


def ekv_current_grad_vth(vgs, vth, cfg):
    """flash_transistor.py:71-82."""
    inv_2nut = 1.0 / (2.0 * cfg["n"] * cfg["U_T"])
    u1 = (vgs - vth) * inv_2nut
    u2 = (vgs - vth - cfg["V_D"]) * inv_2nut
    sp1 = F.softplus(u1)
    sp2 = F.softplus(u2)
    sig1 = _sig_from_sp(sp1)
    sig2 = _sig_from_sp(sp2)
    di = -2.0 * sp1 * sig1 * inv_2nut + 2.0 * sp2 * sig2 * inv_2nut
    return cfg["I_S"] * di / (1.0 + vgs / cfg["V_sat"])


class EKVDiffCurrentFn(torch.autograd.Function):
    """flash_transistor.py:95-131: differential current with the analytic backward."""

    @staticmethod
    def forward(ctx, vgs, vth_pos, vth_neg, cfg):
        out = ekv_current(vgs.float(), vth_pos.float(), cfg) - ekv_current(vgs.float(), vth_neg.float(), cfg)
        ctx.save_for_backward(vgs, vth_pos, vth_neg)
        ctx.cfg = cfg
        return out.to(dtype=vgs.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        vgs, vth_pos, vth_neg = ctx.saved_tensors
        cfg = ctx.cfg
        g = grad_output.float()
        v, vp, vn = vgs.float(), vth_pos.float(), vth_neg.float()
        gv = gp = gn = None
        if ctx.needs_input_grad[0]:
            gv = (g * (ekv_current_grad_v(v, vp, cfg) - ekv_current_grad_v(v, vn, cfg))).to(vgs.dtype)
        if ctx.needs_input_grad[1]:
            gp = (g * ekv_current_grad_vth(v, vp, cfg)).to(vth_pos.dtype)
        if ctx.needs_input_grad[2]:
            gn = (g * (-ekv_current_grad_vth(v, vn, cfg))).to(vth_neg.dtype)
        return gv, gp, gn, None


def cim_idiff_cpu(x: torch.Tensor, vth_pos: torch.Tensor, vth_neg: torch.Tensor, cfg: Dict,
                  chunk: int = 64) -> torch.Tensor:
    """cim.py:201-213 without the TIA gain: x [B,N,K] -> Idiff [B,N,O], chunked over O."""
    outputs = []
    x_exp = x.unsqueeze(-1)
    out_features = vth_pos.shape[0]
    for o_start in range(0, out_features, chunk):
        o_end = min(o_start + chunk, out_features)
        vp = vth_pos[o_start:o_end]
        vn = vth_neg[o_start:o_end]
        vgs = x_exp.expand(-1, -1, -1, vp.shape[0])
        vp_b = vp.t().unsqueeze(0).unsqueeze(0)
        vn_b = vn.t().unsqueeze(0).unsqueeze(0)
        outputs.append(EKVDiffCurrentFn.apply(vgs, vp_b, vn_b, cfg).sum(dim=2))
    return torch.cat(outputs, dim=-1)


def exact_forward(x2d: torch.Tensor, vth_pos: torch.Tensor, vth_neg: torch.Tensor, cfg: Dict,
                  chunk: int = 64) -> torch.Tensor:
    """Idiff[M,O] by the exact formula (no clamp) for a 2-D input, in x's dtype."""
    return cim_idiff_cpu(x2d.unsqueeze(0), vth_pos, vth_neg, cfg, chunk)[0]


def exact_backward(x2d, vth_pos, vth_neg, grad, cfg, chunk: int = 64):
    """(dX, dVth+, dVth-) of sum(grad * Idiff) by the exact analytic gradients."""
    x = x2d.detach().clone().requires_grad_(True)
    vp = vth_pos.detach().clone().requires_grad_(True)
    vn = vth_neg.detach().clone().requires_grad_(True)
    out = exact_forward(x, vp, vn, cfg, chunk)
    out.backward(grad)
    return x.grad, vp.grad, vn.grad


def diff_current_f64(x2d: torch.Tensor, vth_pos: torch.Tensor, vth_neg: torch.Tensor, cfg: Dict,
                     chunk: int = 64) -> torch.Tensor:
    """Idiff[M,O] = sum_k (I(x, vth_pos) - I(x, vth_neg)) in x's dtype (ekv_triton.py:69-91)."""
    x = x2d.unsqueeze(-1)  # [M, K, 1]
    outs = []
    for o0 in range(0, vth_pos.shape[0], chunk):
        vp = vth_pos[o0:o0 + chunk].t().unsqueeze(0)  # [1, K, c]
        vn = vth_neg[o0:o0 + chunk].t().unsqueeze(0)
        outs.append((ekv_current(x, vp, cfg) - ekv_current(x, vn, cfg)).sum(dim=1))
    return torch.cat(outs, dim=-1)


def diff_current_grads_f64(x2d: torch.Tensor, vth_pos: torch.Tensor, vth_neg: torch.Tensor, grad: torch.Tensor,
                           cfg: Dict, chunk: int = 64):
    """(dX, dVth+, dVth-) of sum(grad * Idiff) from the analytic gradients in x's dtype
    (ekv_triton.py:94-169): dX = sum_o G (dI/dv(+) - dI/dv(-)), dVth+ = sum_m G dI/dvth(+),
    dVth- = -sum_m G dI/dvth(-)."""
    x = x2d.unsqueeze(-1)
    dx = torch.zeros_like(x2d)
    dps, dns = [], []
    for o0 in range(0, vth_pos.shape[0], chunk):
        vp = vth_pos[o0:o0 + chunk].t().unsqueeze(0)
        vn = vth_neg[o0:o0 + chunk].t().unsqueeze(0)
        g = grad[:, o0:o0 + chunk].unsqueeze(1)  # [M, 1, c]
        dx += (g * (ekv_current_grad_v(x, vp, cfg) - ekv_current_grad_v(x, vn, cfg))).sum(dim=2)
        dps.append((g * ekv_current_grad_vth(x, vp, cfg)).sum(dim=0).t())
        dns.append((-(g * ekv_current_grad_vth(x, vn, cfg))).sum(dim=0).t())
    return dx, torch.cat(dps, dim=0), torch.cat(dns, dim=0)
