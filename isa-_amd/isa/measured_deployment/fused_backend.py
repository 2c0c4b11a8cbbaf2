"""Opt-in fused backend switch (drop-in for `src/isa/measured_deployment/fused_backend.py`).

In the reference, `install_fused_backend()` patches `DeploymentAwareCIMLinear` so that
no-grad measured forwards below a token threshold run the Triton gather kernel, and
everything else the segmented GEMM path. Here `measured_forward` always runs the fused HIP
kernel (with its gradient for x, any voltage grid and the `vin_lut_bins` mode), so
installing is a marker kept for callers that call it.
"""

from __future__ import annotations


def install_fused_backend() -> None:
    from isa.measured_deployment.operator import DeploymentAwareCIMLinear

    DeploymentAwareCIMLinear._fg50_fused_backend_installed = True
