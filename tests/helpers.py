"""Shared input generators and checks for the parity tests."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle

# cim.py:71, :129-133: U(2.5 +- 0.5 * 2 n U_T)
VTH_LO = 2.5 - 0.5 * 2.0 * 4.1360 * 0.0259
VTH_HI = 2.5 + 0.5 * 2.0 * 4.1360 * 0.0259


def flash_cfg(size: int = 4096, **over):
    cfg = dict(oracle.FLASH_PARAMS)
    cfg.update({"LUT_DELTA_SIZE": size, "use_triton": True, "ekv_approx": "lut", "FORWARD_CHUNK_SIZE": 64,
                "CUDA_SHARED_BACKWARD": True, "R_TIA_LOG_SCALE_MIN": -2.0, "R_TIA_LOG_SCALE_MAX": 2.0,
                "LUT_DTYPE": "float32"})
    cfg.update(over)
    return cfg


def make_inputs(M: int, K: int, O: int, seed: int = 0, x_mode: str = "mapped", vth_mode: str = "init"):
    """Seeded CPU fp32 tensors (x [M,K], vth_pos/vth_neg [O,K], grad [M,O])."""
    g = torch.Generator().manual_seed(seed)
    if x_mode == "mapped":          # VoltageMapping defaults: clamp(N(0,1), 0, 4)
        x = torch.randn(M, K, generator=g).clamp(0.0, 4.0)
    elif x_mode == "signed":        # fc2-like inputs in [-4, 4]
        x = (torch.rand(M, K, generator=g) * 8.0 - 4.0)
    elif x_mode == "fc2init":       # fc2 at initialisation: TIA outputs within +-0.3 V of 0
        x = (torch.rand(M, K, generator=g) * 0.6 - 0.3)
    elif x_mode == "wide":          # drives coordinates past both table ends
        x = torch.rand(M, K, generator=g) * 40.0 - 20.0
    else:
        raise ValueError(x_mode)
    if vth_mode == "init":
        vp = torch.empty(O, K).uniform_(VTH_LO, VTH_HI, generator=g)
        vn = torch.empty(O, K).uniform_(VTH_LO, VTH_HI, generator=g)
    elif vth_mode == "full":        # trained-model-like spread over [0, 5]
        vp = torch.rand(O, K, generator=g) * 5.0
        vn = torch.rand(O, K, generator=g) * 5.0
    elif vth_mode == "wide":
        vp = torch.rand(O, K, generator=g) * 11.0 - 3.0
        vn = torch.rand(O, K, generator=g) * 11.0 - 3.0
    else:
        raise ValueError(vth_mode)
    grad = torch.randn(M, O, generator=g)
    return x, vp, vn, grad


def oracle_tables(cfg):
    """The oracle's fp32 (table_i, table_ddelta) for cfg's table mode: the rounded fp64 table
    (LUT_DTYPE float32), or the reference's bf16 bytes widened to fp32 (LUT_DTYPE bfloat16,
    delta_lut.py:25-35 and the .float() of cuda_backend.py:68-69)."""
    if str(cfg.get("LUT_DTYPE", "float32")).lower() in ("bfloat16", "bf16"):
        _, _, bi, bd = oracle.reference_lut_tables(cfg)
        return bi.float().numpy(), bd.float().numpy()
    return oracle.lut_tables(cfg)


def oracle_all(x, vp, vn, grad, cfg, out_min=-4.0, out_max=4.0):
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, td = oracle_tables(cfg)
    xs, ps, ns, gs = (t.numpy() if isinstance(t, torch.Tensor) else t for t in (x, vp, vn, grad))
    out = oracle.forward(xs, ps, ns, ti, dmin, dmax, cfg["V_sat"], out_min, out_max)
    dx = oracle.grad_x(xs, ps, ns, gs, ti, td, dmin, dmax, cfg["V_sat"])
    gp, gn = oracle.grad_w(xs, ps, ns, gs, td, dmin, dmax, cfg["V_sat"])
    return out, dx, gp, gn


def errs(actual: torch.Tensor, expected: np.ndarray):
    a = actual.detach().double().cpu().numpy()
    return oracle.normwise_error(a, expected), oracle.elementwise_error(a, expected, 1e-3)


def make_codebook(n_states: int = 24, n_points: int = 61, lo: float = 0.0, hi: float = 4.0, seed: int = 0,
                  uniform: bool = True):
    """Synthetic measured I-V codebook: vg [n_points] (uniform, or strictly increasing with
    jittered steps) and monotone curves [n_states, n_points] in amperes (EKV-like turn-on
    at state-dependent thresholds, nA to uA), fp32 CPU tensors."""
    g = torch.Generator().manual_seed(seed)
    if uniform:
        vg = torch.linspace(lo, hi, n_points)
    else:
        steps = torch.rand(n_points - 1, generator=g) + 0.5
        vg = torch.cat([torch.zeros(1), torch.cumsum(steps, 0)])
        vg = (lo + (hi - lo) * vg / vg[-1]).float()
    vt = torch.linspace(0.4, 3.6, n_states)[torch.randperm(n_states, generator=g)]
    slope = 0.08 + 0.04 * torch.rand(n_states, generator=g)
    sp = torch.nn.functional.softplus((vg[None, :] - vt[:, None]) / slope[:, None])
    currents = (2e-9 * sp * sp + 4e-10).float()
    return vg.float(), currents
