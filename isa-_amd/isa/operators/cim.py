"""CIM-based physical FFN layers (drop-in for `src/isa/operators/cim.py`).

`CIMLinear`, `VoltageMapping`, `PhysicalFFN`, `HybridFFN` and `clamp_signed` keep the
reference's constructors, parameter and buffer names (`vth_pos`, `vth_neg`,
`r_tia_log_scale`, `r_tia_base`), initialisation and clamping, so models and checkpoints
built on the reference load unchanged. The projection dispatches as `cim.py:180-187`:
`ekv_approx == "lut"` runs the HIP LUT kernels through `triton_lut_ekv_matmul`, any other
value the HIP exact-formula kernels through `triton_ekv_matmul`.

Only the device paths exist here: a CPU input or `use_triton=False` raises instead of
silently running another implementation (the reference would fall back to its
exact-formula PyTorch path, `cim.py:201-214`).

On the LUT path the elementwise glue around each projection (TIA gain and output clamp,
and in `PhysicalFFN`/`HybridFFN` the input voltage mapping and the ADC affine) runs fused
into the library's kernels (`fused_layer.py`); `ISA_EKV_FUSE_GLUE=0` (or setting
`FUSE_GLUE = False` here) keeps it as separate PyTorch ops; output-statistics tracking
(`cim.py:194-198`) is fused too. Non-fp32 inputs to the voltage mapping use the separate
ops.
"""

from __future__ import annotations

import os
from typing import Dict, Optional

import torch
import torch.nn as nn

from isa.device_models.config import FLASH_TRANSISTOR_EKV_CONFIG as PHYSICAL_CONFIG
from isa.kernels.transformer_ffn.ekv_lut_triton import triton_lut_ekv_matmul
from isa.kernels.transformer_ffn.ekv_triton import triton_ekv_matmul
from isa.kernels.transformer_ffn.fused_layer import fused_cim_layer

FUSE_GLUE = os.environ.get("ISA_EKV_FUSE_GLUE", "1") != "0"


class VoltageMapping(nn.Module):
    """Map external digital activations to the first-layer gate voltage range (cim.py:23-39)."""

    def __init__(self, voltage_max: float = 4.0):
        super().__init__()
        self.voltage_max = voltage_max
        self.scale = nn.Parameter(torch.tensor(1.0))
        self.shift = nn.Parameter(torch.tensor(0.0))

    @torch.no_grad()
    def set_affine(self, scale: float, shift: float) -> None:
        self.scale.fill_(float(scale))
        self.shift.fill_(float(shift))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        v = (x.float() * self.scale + self.shift).clamp(0.0, self.voltage_max)
        return v.to(dtype=x.dtype)


def clamp_signed(v: torch.Tensor, v_min: float = -4.0, v_max: float = 4.0) -> torch.Tensor:
    return v.clamp(v_min, v_max)


def _device_projection(cfg: Dict, x: torch.Tensor, where: str):
    """The projection cim.py:180-187 would pick on a device: LUT or exact formula."""
    if not x.is_cuda:
        raise RuntimeError(
            f"CIMLinear.{where}: this build runs the Flash-EKV projection on a ROCm device only; "
            f"got an input on {x.device}"
        )
    if not bool(cfg.get("use_triton", False)):
        raise NotImplementedError(f"CIMLinear.{where}: use_triton=False (exact PyTorch path) is not part of this build")
    approx = str(cfg.get("ekv_approx", "lut")).lower()
    return triton_lut_ekv_matmul if approx == "lut" else triton_ekv_matmul


class CIMLinear(nn.Module):
    """Compute-and-memory linear layer via EKV differential current and TIA (cim.py:46-214)."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        physical_config: Optional[Dict[str, float]] = None,
    ):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.cfg = dict(physical_config or PHYSICAL_CONFIG)

        self.vth_pos = nn.Parameter(torch.empty(out_features, in_features))
        self.vth_neg = nn.Parameter(torch.empty(out_features, in_features))
        self.register_buffer(
            "r_tia_base",
            torch.full((1,), float(self.cfg.get("R_TIA", 1e5)), dtype=torch.float32),
        )
        self.r_tia_log_scale = nn.Parameter(torch.zeros(1, dtype=torch.float32))
        self.track_output_stats = False
        self.register_buffer("_stat_total", torch.zeros((), dtype=torch.float64), persistent=False)
        self.register_buffer("_stat_clipped", torch.zeros((), dtype=torch.float64), persistent=False)
        self.register_buffer("_stat_abs_max", torch.zeros((), dtype=torch.float32), persistent=False)
        self.reset_vth(mode="centered_random", eps_k=0.5, symmetric=False)

    @property
    def r_tia(self) -> torch.Tensor:
        lo = float(self.cfg.get("R_TIA_LOG_SCALE_MIN", -2.0))
        hi = float(self.cfg.get("R_TIA_LOG_SCALE_MAX", 2.0))
        return self.r_tia_base * self.r_tia_log_scale.clamp(lo, hi).exp()

    def set_r_tia(self, value: float) -> None:
        with torch.no_grad():
            self.r_tia_base.fill_(float(value))
            self.r_tia_log_scale.zero_()

    def reset_output_stats(self) -> None:
        self._stat_total.zero_()
        self._stat_clipped.zero_()
        self._stat_abs_max.zero_()

    def set_output_stats_tracking(self, enabled: bool, reset: bool = False) -> None:
        self.track_output_stats = bool(enabled)
        if reset:
            self.reset_output_stats()

    def output_stats(self) -> Dict[str, float]:
        total = float(self._stat_total.item())
        clipped = float(self._stat_clipped.item())
        return {
            "total": total,
            "clipped": clipped,
            "clip_ratio": clipped / max(total, 1.0),
            "preclamp_abs_max": float(self._stat_abs_max.item()),
        }

    def reset_vth(
        self,
        center: float | torch.Tensor | None = None,
        eps_k: float = 0.5,
        symmetric: bool = True,
        mode: str = "centered_symmetric",
    ) -> None:
        """cim.py:113-138 (same RNG order: vth_pos.uniform_ then vth_neg.uniform_)."""
        v_min = float(self.cfg["V_TH_MIN"])
        v_max = float(self.cfg["V_TH_MAX"])
        if center is None:
            center_t = torch.tensor(0.5 * (v_min + v_max), device=self.vth_pos.device, dtype=self.vth_pos.dtype)
        elif torch.is_tensor(center):
            center_t = center.to(device=self.vth_pos.device, dtype=self.vth_pos.dtype)
        else:
            center_t = torch.tensor(float(center), device=self.vth_pos.device, dtype=self.vth_pos.dtype)
        center_t = center_t.clamp(v_min, v_max)
        eps_scale = float(eps_k) * 2.0 * float(self.cfg["n"]) * float(self.cfg["U_T"])
        with torch.no_grad():
            if mode in {"random", "centered_random"} or not symmetric:
                self.vth_pos.uniform_(-eps_scale, eps_scale).add_(center_t)
                self.vth_neg.uniform_(-eps_scale, eps_scale).add_(center_t)
            else:
                eps = torch.empty_like(self.vth_pos).normal_(0.0, eps_scale)
                self.vth_pos.copy_(center_t + eps)
                self.vth_neg.copy_(center_t - eps)
            self.clamp_vth()

    @torch.no_grad()
    def estimate_idiff(self, x: torch.Tensor, max_rows: int = 4096) -> torch.Tensor:
        """Pre-TIA Idiff of up to `max_rows` input rows (cim.py:140-163)."""
        flat = x.reshape(-1, self.in_features).contiguous()
        if flat.shape[0] > max_rows:
            flat = flat[:max_rows]
        project = _device_projection(self.cfg, flat, "estimate_idiff")
        return project(flat, self.vth_pos, self.vth_neg, self.cfg)

    def clamp_vth(self) -> None:
        v_min = self.cfg["V_TH_MIN"]
        v_max = self.cfg["V_TH_MAX"]
        with torch.no_grad():
            self.vth_pos.clamp_(v_min, v_max)
            self.vth_neg.clamp_(v_min, v_max)

    def fusable(self, x: torch.Tensor) -> bool:
        """Whether the fused LUT layer (projection + glue in the library) serves this input."""
        return (FUSE_GLUE and x.is_cuda and bool(self.cfg.get("use_triton", False))
                and str(self.cfg.get("ekv_approx", "lut")).lower() == "lut")

    def fused_forward(self, x: torch.Tensor, in_affine: Optional[torch.Tensor] = None,
                      in_range=(0.0, 4.0), adc_scale: Optional[torch.Tensor] = None,
                      adc_shift: Optional[torch.Tensor] = None) -> torch.Tensor:
        """forward() with the glue in the library; optionally also the input mapping
        clamp(x * in_affine[0] + in_affine[1], in_range) before and the ADC affine after."""
        b, n, in_f = x.shape
        assert in_f == self.in_features
        flat = x.reshape(b * n, in_f)
        stats = (self._stat_abs_max, self._stat_total) if self.track_output_stats else None
        # the gain r_tia_base * exp(clamp(r_tia_log_scale)) (the r_tia property) is formed in
        # the library, which returns the log scale's gradient
        lo = float(self.cfg.get("R_TIA_LOG_SCALE_MIN", -2.0))
        hi = float(self.cfg.get("R_TIA_LOG_SCALE_MAX", 2.0))
        out = fused_cim_layer(flat, self.vth_pos, self.vth_neg, self.cfg, in_affine=in_affine, in_range=in_range,
                              r_tia=self.r_tia_base, r_log_scale=self.r_tia_log_scale, r_log_range=(lo, hi),
                              adc_scale=adc_scale, adc_shift=adc_shift, stats=stats)
        return out.reshape(b, n, self.out_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, n, in_f = x.shape
        assert in_f == self.in_features
        project = _device_projection(self.cfg, x, "forward")
        if self.fusable(x):
            return self.fused_forward(x)

        r_tia = self.r_tia.to(device=x.device, dtype=torch.float32).view(1, 1, 1)
        v_signed_min = float(self.cfg.get("V_signed_min", -4.0))
        v_signed_max = float(self.cfg.get("V_signed_max", 4.0))

        flat = x.reshape(b * n, in_f).contiguous()
        idiff = project(flat, self.vth_pos, self.vth_neg, self.cfg)
        # the LUT kernel returns I_diff clamped to [v_signed_min, v_signed_max], the exact one
        # unclamped; the learnable TIA gain is applied here so autograd tracks it (cim.py:190-193)
        out = idiff.reshape(b, n, self.out_features) * r_tia
        out = out.clamp(v_signed_min, v_signed_max)
        if self.track_output_stats:
            with torch.no_grad():
                detached = out.detach()
                self._stat_total.add_(detached.numel())
                self._stat_abs_max.copy_(torch.maximum(self._stat_abs_max, detached.abs().max().float()))
        return out


class PhysicalFFN(nn.Module):
    """EKV physical FFN: voltage mapping -> CIMLinear -> CIMLinear -> ADC affine (cim.py:217-247)."""

    def __init__(
        self,
        dim: int,
        hidden_dim: int,
        physical_config: Optional[Dict[str, float]] = None,
        voltage_max: float = 4.0,
    ):
        super().__init__()
        self.input_mapping = VoltageMapping(voltage_max=voltage_max)
        self.fc1 = CIMLinear(dim, hidden_dim, physical_config)
        self.fc2 = CIMLinear(hidden_dim, dim, physical_config)
        self.adc_affine_scale = nn.Parameter(torch.ones(dim))
        self.adc_affine_shift = nn.Parameter(torch.zeros(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype == torch.float32 and self.fc1.fusable(x) and self.fc2.fusable(x):
            _device_projection(self.fc1.cfg, x, "forward")
            m = self.input_mapping
            h = self.fc1.fused_forward(x, in_affine=torch.stack([m.scale, m.shift]).float(),
                                       in_range=(0.0, m.voltage_max))
            return self.fc2.fused_forward(h, adc_scale=self.adc_affine_scale, adc_shift=self.adc_affine_shift)
        x = self.input_mapping(x)
        x = self.fc1(x)
        x = self.fc2(x)
        return x * self.adc_affine_scale + self.adc_affine_shift

    def clamp_vth(self) -> None:
        self.fc1.clamp_vth()
        self.fc2.clamp_vth()


class HybridFFN(nn.Module):
    """Hybrid FFN: CIMLinear up-projection + digital nn.Linear down-projection (cim.py:250-280)."""

    def __init__(
        self,
        dim: int,
        hidden_dim: int,
        physical_config: Optional[Dict[str, float]] = None,
        voltage_max: float = 4.0,
    ):
        super().__init__()
        self.input_mapping = VoltageMapping(voltage_max=voltage_max)
        self.fc1 = CIMLinear(dim, hidden_dim, physical_config)
        self.fc2 = nn.Linear(hidden_dim, dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype == torch.float32 and self.fc1.fusable(x):
            _device_projection(self.fc1.cfg, x, "forward")
            m = self.input_mapping
            x = self.fc1.fused_forward(x, in_affine=torch.stack([m.scale, m.shift]).float(),
                                       in_range=(0.0, m.voltage_max))
        else:
            x = self.input_mapping(x)
            x = self.fc1(x)
        x = self.fc2(x)
        return x

    def clamp_vth(self) -> None:
        self.fc1.clamp_vth()
