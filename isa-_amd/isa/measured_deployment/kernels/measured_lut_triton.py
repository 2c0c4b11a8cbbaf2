"""Fused measured-IV lookup and reduction (drop-in for
`src/isa/measured_deployment/kernels/measured_lut_triton.py`).

`fused_measured_forward` keeps the reference's signature, validation and semantics
(`:159-267`): inputs clamped to the lookup range, uniform-grid segment
`int((x - voltage_min) * inverse_step)`, per cell `S[a] x + C[a]` (pair mode, the ids name
difference curves) or `(S[a] - S[b]) x + (C[a] - C[b])` (member mode), summed over the
inputs, scaled by `current_scale * r_tia` and clamped. The work runs in the HIP kernel
`isa_ekv_measured_forward`; there is no Triton. The Triton block sizes are accepted and
ignored.
"""

from __future__ import annotations

import torch

from isa.kernels.transformer_ffn import _hip, ops


def _uniform_voltage_grid(voltage_v: torch.Tensor) -> tuple[float, float]:
    """measured_lut_triton.py:145-154."""
    if voltage_v.ndim != 1 or voltage_v.numel() < 2:
        raise ValueError("voltage_v must be a 1-D grid with at least two points")
    delta = voltage_v[1:] - voltage_v[:-1]
    if not bool(torch.all(delta > 0)):
        raise ValueError("voltage_v must be strictly increasing")
    reference = delta[0]
    if not bool(torch.allclose(delta, reference, atol=1e-6, rtol=1e-5)):
        raise ValueError("the fused kernel currently requires a uniform voltage grid")
    return float(voltage_v[0].item()), 1.0 / float(reference.item())


@torch.no_grad()
def fused_measured_forward(
    x: torch.Tensor,
    assignment_a: torch.Tensor,
    slopes: torch.Tensor,
    intercepts: torch.Tensor,
    voltage_v: torch.Tensor,
    *,
    assignment_b: torch.Tensor | None = None,
    pair_mode: bool,
    lookup_min: float = 0.0,
    lookup_max: float = 4.0,
    current_scale: float = 1e-9,
    r_tia: float | torch.Tensor = 1.0,
    signed_min: float = -4.0,
    signed_max: float = 4.0,
    block_b: int = 2,
    block_o: int = 32,
    block_k: int = 32,
    num_warps: int = 4,
    voltage_min: float | None = None,
    inverse_voltage_step: float | None = None,
) -> torch.Tensor:
    if not x.is_cuda:
        raise ValueError("x must be a CUDA tensor")
    if x.shape[-1] != assignment_a.shape[1]:
        raise ValueError("x input dimension and assignment width differ")
    if assignment_a.ndim != 2:
        raise ValueError("assignment_a must have shape [out_features, in_features]")
    if not pair_mode and (assignment_b is None or assignment_b.shape != assignment_a.shape):
        raise ValueError("member mode requires assignment_b with matching shape")
    if slopes.ndim != 2 or intercepts.shape != slopes.shape:
        raise ValueError("slope/intercept tables must have matching 2-D shapes")
    if slopes.shape[1] != voltage_v.numel() - 1:
        raise ValueError("coefficient segment count does not match voltage grid")
    if assignment_a.device != x.device:
        raise ValueError("assignments and x must be on the same CUDA device")
    if slopes.device != x.device or intercepts.device != x.device:
        raise ValueError("coefficient tables and x must be on the same CUDA device")
    if (voltage_min is None) != (inverse_voltage_step is None):
        raise ValueError("voltage_min and inverse_voltage_step must be provided together")
    if voltage_min is None:
        voltage_min, inverse_step = _uniform_voltage_grid(voltage_v)
    else:
        inverse_step = float(inverse_voltage_step)
        voltage_min = float(voltage_min)
        if inverse_step <= 0:
            raise ValueError("inverse_voltage_step must be positive")
    if isinstance(r_tia, torch.Tensor):
        if r_tia.numel() != 1:
            raise ValueError("tensor-valued r_tia must contain one scalar")
        if r_tia.device != x.device:
            raise ValueError("tensor-valued r_tia and x must be on the same device")
        gain = r_tia.detach().float().reshape(1)
    else:
        gain = torch.full((1,), float(r_tia), dtype=torch.float32, device=x.device)
    original_shape = x.shape
    flat = x.reshape(-1, original_shape[-1]).float()
    out, _ = ops.measured_forward(
        flat, assignment_a, None if pair_mode else assignment_b, slopes, intercepts,
        seg_mode=_hip.SEG_UNIFORM, voltage_min=voltage_min, inverse_step=inverse_step,
        lookup_min=float(lookup_min), lookup_max=float(lookup_max), current_scale=float(current_scale),
        r_tia=gain, out_min=float(signed_min), out_max=float(signed_max))
    return out.reshape(*original_shape[:-1], assignment_a.shape[0]).to(x.dtype)
