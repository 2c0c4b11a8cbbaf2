"""Measured-codebook deployment operator for physical ViT FFNs (drop-in for the operator
and kernel of `src/isa/measured_deployment/`).

Built here: `DeploymentAwareCIMLinear` (continuous / measured / STE forward modes) and the
functional `kernels.measured_lut_triton.fused_measured_forward`, both on the HIP
measured-codebook kernels. The FG50 data pipeline around them (runtime builder, codebook
library, assignment search, post-training, Monte Carlo drivers) is not part of this build.
"""

from isa.measured_deployment.operator import DeploymentAwareCIMLinear

__all__ = ["DeploymentAwareCIMLinear"]
