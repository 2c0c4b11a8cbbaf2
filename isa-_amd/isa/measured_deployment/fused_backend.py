"""Opt-in fused backend (drop-in for `src/isa/measured_deployment/fused_backend.py`).

`install_fused_backend()` makes every `DeploymentAwareCIMLinear` configured afterwards from
the same codebook tensors on the same device share one device copy of the codebook and of
its coefficient tables, instead of each layer holding its own (the reference's
`codebook_cache`, `fused_backend.py:37-131`: with the 32,240-curve Monte Carlo codebook
that is ~24 MB per layer). Installing twice is a no-op, and the shared entries keep the
source tensors alive, so their ids are not reused while an entry exists.

What the reference's install also switches, and why it does not apply here: it routes
no-grad measured forwards below a token threshold (`FG50_*_FUSED_TOKEN_THRESHOLD`) to its
Triton gather kernel and the rest to the segmented GEMM path; here `measured_forward`
always runs the fused HIP kernel, with its gradient for x, at every token count. Its
restrictions to uniform voltage grids and `vin_lut_bins == 0` do not apply either (the HIP
kernel supports both); the `FG50_*` variables are not read.
"""

from __future__ import annotations


def install_fused_backend() -> None:
    from isa.measured_deployment.operator import DeploymentAwareCIMLinear

    DeploymentAwareCIMLinear._fg50_fused_backend_installed = True
