"""MI355X-native Flash-EKV LUT CIMLinear behind the reference's `isa` module paths.

Mirrors `isa.operators.cim`, `isa.kernels.transformer_ffn` (`ekv_lut_triton`,
`cuda_backend`), `isa.approximations.delta_lut` and `isa.device_models.config` of the
reference (package `in-synapse-activation` 0.1.0); every compute call runs the HIP
library `libisa_ekv_hip.so` built for gfx950.
"""

__version__ = "0.1.0"
