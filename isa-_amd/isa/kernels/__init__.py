"""HIP kernels for gfx950."""
