"""Fused Flash-transistor EKV kernels for Transformer FFNs (HIP, gfx950)."""
