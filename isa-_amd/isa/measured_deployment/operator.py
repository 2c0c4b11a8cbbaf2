"""Fixed measured-codebook forward with an EKV straight-through gradient (drop-in for
`src/isa/measured_deployment/operator.py`).

`DeploymentAwareCIMLinear` keeps the reference's class, parameter and buffer names, modes
(`continuous`, `measured`, `ste`), codebook/assignment API and validation, so checkpoints
and callers work unchanged. What differs is how the measured forward runs: the reference
expands one slope and one intercept matrix per voltage segment (`diff_a`, `diff_b`:
[segments, O, K]) and launches two GEMMs per segment over masked inputs
(`operator.py:164-224`); here the HIP kernel gathers each cell's curve coefficients from
the compact codebook held in LDS and reduces over the inputs in one pass, with the same
piecewise-linear value and the same gradient for the input (`isa_ekv_measured_forward` /
`_backward`). The expanded buffers stay empty.
"""

from __future__ import annotations

from collections.abc import Iterable
from typing import ClassVar

import torch
from torch import nn

from isa.kernels.transformer_ffn import _hip, ops
from isa.operators.cim import CIMLinear


class _MeasuredFn(torch.autograd.Function):
    """Measured projection with the gradient for x (the codebook and ids are fixed buffers,
    r_tia is detached, as in the reference)."""

    @staticmethod
    def forward(ctx, flat, ids_a, ids_b, slopes, intercepts, vg, r_tia, meta):
        seg_mode, voltage_min, inverse_step, lookup_min, lookup_max, out_min, out_max = meta
        out, pre = ops.measured_forward(
            flat, ids_a, ids_b, slopes, intercepts, seg_mode=seg_mode, vg=vg, voltage_min=voltage_min,
            inverse_step=inverse_step, lookup_min=lookup_min, lookup_max=lookup_max, current_scale=1.0,
            r_tia=r_tia, out_min=out_min, out_max=out_max)
        ctx.save_for_backward(flat, ids_a, ids_b, slopes, intercepts, vg, r_tia, pre)
        ctx.meta = meta
        return out

    @staticmethod
    def backward(ctx, grad_out):
        flat, ids_a, ids_b, slopes, intercepts, vg, r_tia, pre = ctx.saved_tensors
        seg_mode, voltage_min, inverse_step, lookup_min, lookup_max, out_min, out_max = ctx.meta
        gx = None
        if ctx.needs_input_grad[0]:
            gx = ops.measured_backward(
                flat, ids_a, ids_b, slopes, intercepts, grad_out, pre, seg_mode=seg_mode, vg=vg,
                voltage_min=voltage_min, inverse_step=inverse_step, lookup_min=lookup_min, lookup_max=lookup_max,
                current_scale=1.0, r_tia=r_tia, out_min=out_min, out_max=out_max)
        return gx, None, None, None, None, None, None, None


class DeploymentAwareCIMLinear(CIMLinear):
    """CIMLinear whose forward can be continuous, measured, or measured+STE (operator.py:21-233)."""

    MODES: ClassVar[set[str]] = {"continuous", "measured", "ste"}

    def __init__(self, in_features: int, out_features: int, physical_config=None) -> None:
        super().__init__(in_features, out_features, physical_config)
        self.forward_mode = "continuous"
        self.vin_lut_bins = 0
        self.lookup_min = float(self.cfg.get("V_min", 0.0))
        self.lookup_max = float(self.cfg.get("V_max", 4.0))
        self.register_buffer("measured_vg", torch.empty(0), persistent=False)
        self.register_buffer("measured_currents", torch.empty(0), persistent=False)
        self.register_buffer("pos_idx", torch.empty(0, dtype=torch.int16), persistent=False)
        self.register_buffer("neg_idx", torch.empty(0, dtype=torch.int16), persistent=False)
        self.register_buffer("active_segments", torch.empty(0, dtype=torch.long), persistent=False)
        self.register_buffer("diff_a", torch.empty(0), persistent=False)
        self.register_buffer("diff_b", torch.empty(0), persistent=False)
        self.register_buffer("bin_centers", torch.empty(0), persistent=False)
        self.register_buffer("diff_current", torch.empty(0), persistent=False)
        # compact codebook tables of the kernel: [curves, segments] slope/intercept
        self.register_buffer("curve_slopes", torch.empty(0), persistent=False)
        self.register_buffer("curve_intercepts", torch.empty(0), persistent=False)

    @classmethod
    def from_cimlinear(cls, original: CIMLinear) -> "DeploymentAwareCIMLinear":
        replacement = cls(original.in_features, original.out_features, original.cfg)
        replacement.load_state_dict(original.state_dict(), strict=True)
        replacement.to(device=original.vth_pos.device, dtype=original.vth_pos.dtype)
        return replacement

    def set_forward_mode(self, mode: str) -> None:
        if mode not in self.MODES:
            raise ValueError(f"Unsupported deployment-aware forward mode: {mode}")
        self.forward_mode = mode

    @torch.no_grad()
    def configure_codebook(self, vg: torch.Tensor, currents_a: torch.Tensor, vin_lut_bins: int = 0) -> None:
        """operator.py:56-75."""
        device = self.vth_pos.device
        vg = vg.detach().to(device=device, dtype=torch.float32).contiguous()
        currents = currents_a.detach().to(device=device, dtype=torch.float32).contiguous()
        if vg.ndim != 1 or currents.ndim != 2 or currents.shape[1] != vg.numel():
            raise ValueError("Measured codebook tensors have inconsistent shapes")
        if vg.numel() < 2 or not bool(torch.all(vg[1:] > vg[:-1])):
            raise ValueError("Measured Vg grid must be strictly increasing")
        self.measured_vg = vg
        self.measured_currents = currents
        self.lookup_min = max(float(vg[0].item()), float(self.cfg.get("V_min", 0.0)))
        self.lookup_max = min(float(vg[-1].item()), float(self.cfg.get("V_max", 4.0)))
        self.vin_lut_bins = int(vin_lut_bins)
        if self.vin_lut_bins < 0:
            raise ValueError("vin_lut_bins must be non-negative")

    @torch.no_grad()
    def set_assignment(self, pos_idx: torch.Tensor, neg_idx: torch.Tensor) -> None:
        """operator.py:77-146: validation and the per-mode coefficient tables. The kernel
        reads the compact [curves, segments] tables instead of the expanded per-cell ones."""
        if self.measured_vg.numel() == 0:
            raise RuntimeError("configure_codebook must be called before set_assignment")
        expected = (self.out_features, self.in_features)
        if tuple(pos_idx.shape) != expected or tuple(neg_idx.shape) != expected:
            raise ValueError(f"Assignment shape must be {expected}")
        device = self.vth_pos.device
        self.pos_idx = pos_idx.to(device=device, dtype=torch.int16).contiguous()
        self.neg_idx = neg_idx.to(device=device, dtype=torch.int16).contiguous()
        pos = self.pos_idx.long()
        neg = self.neg_idx.long()
        if int(pos.min()) < 0 or int(neg.min()) < 0:
            raise ValueError("Assignment contains negative state indices")
        state_count = int(self.measured_currents.shape[0])
        if int(pos.max()) >= state_count or int(neg.max()) >= state_count:
            raise ValueError("Assignment references a state outside the codebook")

        if self.vin_lut_bins > 0:
            centers = torch.linspace(self.lookup_min, self.lookup_max, self.vin_lut_bins, device=device,
                                     dtype=torch.float32)
            # currents of every state at every bin centre: [states, bins], zero slopes
            at_centers = torch.stack([self.currents_at(center) for center in centers], dim=1)
            self.bin_centers = centers
            self.curve_slopes = torch.zeros_like(at_centers)
            self.curve_intercepts = at_centers.contiguous()
            self.active_segments = torch.empty(0, dtype=torch.long, device=device)
            return

        vg = self.measured_vg
        currents = self.measured_currents
        dv = vg[1:] - vg[:-1]
        slopes = (currents[:, 1:] - currents[:, :-1]) / dv.unsqueeze(0)
        intercepts = currents[:, :-1] - slopes * vg[:-1].unsqueeze(0)
        self.active_segments = torch.nonzero(
            (vg[:-1] <= self.lookup_max) & (vg[1:] >= self.lookup_min), as_tuple=False
        ).flatten()
        self.curve_slopes = slopes.contiguous()
        self.curve_intercepts = intercepts.contiguous()
        self.bin_centers = torch.empty(0, device=device)

    def currents_at(self, voltage: torch.Tensor | float) -> torch.Tensor:
        """operator.py:148-162: every state's current at `voltage` (linear interpolation)."""
        if self.measured_vg.numel() == 0:
            raise RuntimeError("Measured codebook has not been configured")
        value = torch.as_tensor(voltage, device=self.measured_vg.device, dtype=torch.float32).clamp(
            self.measured_vg[0], self.measured_vg[-1])
        upper = torch.searchsorted(self.measured_vg, value, right=True).clamp(1, self.measured_vg.numel() - 1)
        lower = upper - 1
        alpha = (value - self.measured_vg[lower]) / (self.measured_vg[upper] - self.measured_vg[lower])
        return self.measured_currents[:, lower] + alpha * (
            self.measured_currents[:, upper] - self.measured_currents[:, lower])

    def measured_forward(self, x: torch.Tensor) -> torch.Tensor:
        """operator.py:164-224 on the HIP kernel: fp32 even under autocast, output
        clamp(sum * R_TIA) in x's dtype, exact piecewise-linear gradient for x."""
        if self.pos_idx.numel() == 0:
            raise RuntimeError("Measured assignment is not initialized")
        if not x.is_cuda:
            raise RuntimeError("DeploymentAwareCIMLinear.measured_forward runs on a ROCm device only")
        original_dtype = x.dtype
        shape = x.shape
        flat = x.float().reshape(-1, self.in_features)
        if self.vin_lut_bins > 0:
            bins = self.vin_lut_bins
            scale = (bins - 1) / (self.lookup_max - self.lookup_min) if bins > 1 else 1.0
            seg_mode, vg = _hip.SEG_ROUND, None
        else:
            scale = 1.0
            seg_mode, vg = _hip.SEG_SEARCH, self.measured_vg
        meta = (seg_mode, 0.0, float(scale), float(self.lookup_min), float(self.lookup_max),
                float(self.cfg.get("V_signed_min", -4.0)), float(self.cfg.get("V_signed_max", 4.0)))
        r_tia = self.r_tia.detach().float().reshape(1).to(x.device)
        with torch.autocast("cuda", enabled=False):
            out = _MeasuredFn.apply(flat, self.pos_idx, self.neg_idx, self.curve_slopes, self.curve_intercepts,
                                    vg, r_tia, meta)
        return out.reshape(*shape[:-1], self.out_features).to(original_dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.forward_mode == "continuous":
            return super().forward(x)
        if self.forward_mode == "measured":
            return self.measured_forward(x)
        # STE: forward equals measured; backward equals the continuous EKV surrogate.
        with torch.no_grad():
            measured = self.measured_forward(x)
        continuous = super().forward(x)
        return continuous + (measured - continuous).detach()


def replace_physical_fc1(model: nn.Module) -> list[DeploymentAwareCIMLinear]:
    """operator.py:227-237."""
    layers: list[DeploymentAwareCIMLinear] = []
    for block_id, block in enumerate(model.blocks):
        original = block.mlp.fc1
        if not isinstance(original, CIMLinear):
            raise TypeError(f"blocks.{block_id}.mlp.fc1 is not CIMLinear")
        replacement = DeploymentAwareCIMLinear.from_cimlinear(original)
        block.mlp.fc1 = replacement
        layers.append(replacement)
    return layers


def iter_deployment_fc1(model: nn.Module) -> Iterable[tuple[int, DeploymentAwareCIMLinear]]:
    for block_id, block in enumerate(model.blocks):
        layer = block.mlp.fc1
        if not isinstance(layer, DeploymentAwareCIMLinear):
            raise TypeError(f"blocks.{block_id}.mlp.fc1 is not deployment-aware")
        yield block_id, layer


def set_fc1_forward_mode(model: nn.Module, mode: str) -> None:
    for _, layer in iter_deployment_fc1(model):
        layer.set_forward_mode(mode)
