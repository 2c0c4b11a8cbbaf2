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


def _codebook_tables(vg: torch.Tensor, currents_a: torch.Tensor, device: torch.device, bins: int,
                     v_min: float, v_max: float) -> dict[str, object]:
    """The validated codebook on `device` and its compact coefficient tables: per-segment line
    slopes and intercepts of every measured curve ([states, segments]: I = S v + C on segment
    s), and the tables the kernel reads: those lines, or in vin_lut_bins mode every state's
    current at each bin centre as a zero-slope table ([states, bins])."""
    mvg = vg.detach().to(device=device, dtype=torch.float32).contiguous()
    cur = currents_a.detach().to(device=device, dtype=torch.float32).contiguous()
    if mvg.ndim != 1 or cur.ndim != 2 or cur.shape[1] != mvg.numel():
        raise ValueError("Measured codebook tensors have inconsistent shapes")
    if mvg.numel() < 2 or not bool(torch.all(mvg[1:] > mvg[:-1])):
        raise ValueError("Measured Vg grid must be strictly increasing")
    lookup = (max(float(mvg[0].item()), v_min), min(float(mvg[-1].item()), v_max))
    step = mvg[1:] - mvg[:-1]
    seg_s = ((cur[:, 1:] - cur[:, :-1]) / step.unsqueeze(0)).contiguous()
    seg_c = (cur[:, :-1] - seg_s * mvg[:-1].unsqueeze(0)).contiguous()
    book = {"vg": mvg, "currents": cur, "lookup": lookup,
            "segment_slopes": seg_s, "segment_intercepts": seg_c}
    if bins > 0:
        centers = torch.linspace(lookup[0], lookup[1], bins, device=device, dtype=torch.float32)
        seg = (torch.searchsorted(mvg, centers, right=True) - 1).clamp(0, mvg.numel() - 2)
        at_centers = (seg_s[:, seg] * centers.unsqueeze(0) + seg_c[:, seg]).contiguous()
        book.update(table_slopes=torch.zeros_like(at_centers), table_intercepts=at_centers,
                    active_segments=torch.empty(0, dtype=torch.long, device=device), bin_centers=centers)
    else:
        active = torch.nonzero((mvg[:-1] <= lookup[1]) & (mvg[1:] >= lookup[0]), as_tuple=False).flatten()
        book.update(table_slopes=seg_s, table_intercepts=seg_c, active_segments=active,
                    bin_centers=torch.empty(0, device=device))
    return book


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
        # segment lines of the measured curves ([curves, segments]), for currents_at
        self.register_buffer("_segment_slopes", torch.empty(0), persistent=False)
        self.register_buffer("_segment_intercepts", torch.empty(0), persistent=False)

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
        """operator.py:56-75: validate and hold the codebook, plus the compact coefficient tables
        the kernel reads (they depend on the codebook only, not on the assignment). With
        install_fused_backend() in effect, layers configured from the same source tensors on
        one device share one copy of all of them (fused_backend.py:37-131)."""
        if int(vin_lut_bins) < 0:
            raise ValueError("vin_lut_bins must be non-negative")
        device = self.vth_pos.device
        bins, v_min, v_max = int(vin_lut_bins), float(self.cfg.get("V_min", 0.0)), float(self.cfg.get("V_max", 4.0))
        if bool(getattr(type(self), "_fg50_fused_backend_installed", False)):
            from isa.measured_deployment.fused_backend import shared_codebook

            book = shared_codebook(vg, currents_a, device, bins, v_min, v_max, _codebook_tables)
        else:
            book = _codebook_tables(vg, currents_a, device, bins, v_min, v_max)
        self.measured_vg = book["vg"]
        self.measured_currents = book["currents"]
        self.lookup_min, self.lookup_max = book["lookup"]
        self.vin_lut_bins = int(vin_lut_bins)
        self._segment_slopes = book["segment_slopes"]
        self._segment_intercepts = book["segment_intercepts"]
        self.curve_slopes = book["table_slopes"]
        self.curve_intercepts = book["table_intercepts"]
        self.active_segments = book["active_segments"]
        self.bin_centers = book["bin_centers"]

    @torch.no_grad()
    def set_assignment(self, pos_idx: torch.Tensor, neg_idx: torch.Tensor) -> None:
        """operator.py:77-146: the assignment's validation, with the reference's messages. The
        kernel reads the compact per-state tables configure_codebook holds instead of the
        expanded per-cell ones."""
        if self.measured_vg.numel() == 0:
            raise RuntimeError("configure_codebook must be called before set_assignment")
        expected = (self.out_features, self.in_features)
        if tuple(pos_idx.shape) != expected or tuple(neg_idx.shape) != expected:
            raise ValueError(f"Assignment shape must be {expected}")
        device = self.vth_pos.device
        pos = pos_idx.to(device=device, dtype=torch.int16).contiguous()
        neg = neg_idx.to(device=device, dtype=torch.int16).contiguous()
        if int(torch.minimum(pos.min(), neg.min())) < 0:
            raise ValueError("Assignment contains negative state indices")
        state_count = int(self.measured_currents.shape[0])
        if int(torch.maximum(pos.max(), neg.max())) >= state_count:
            raise ValueError("Assignment references a state outside the codebook")
        self.pos_idx, self.neg_idx = pos, neg

    def currents_at(self, voltage: torch.Tensor | float) -> torch.Tensor:
        """Every state's current at `voltage` (operator.py:148-162): [states] for a scalar,
        [states, *voltage.shape] for a tensor. Evaluated as the kernel's cells evaluate the
        curves, S[state, seg] * v + C[state, seg] on the segment seg holding v (clamped to
        the measured grid)."""
        if self.measured_vg.numel() == 0:
            raise RuntimeError("Measured codebook has not been configured")
        vg = self.measured_vg
        v = torch.as_tensor(voltage, device=vg.device, dtype=torch.float32).clamp(vg[0], vg[-1])
        seg = (torch.searchsorted(vg, v.reshape(-1), right=True) - 1).clamp(0, vg.numel() - 2)
        out = self._segment_slopes[:, seg] * v.reshape(1, -1) + self._segment_intercepts[:, seg]
        return out.reshape(self._segment_slopes.shape[0], *v.shape)

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
