"""Measured-codebook projection restated from the reference (TEST INFRASTRUCTURE ONLY).

Only ``tests/`` may import this module, as the checker of the HIP measured-codebook
kernels. It restates, with numpy (per-cell fp32 terms, float64 sums):

* the coefficient tables of ``DeploymentAwareCIMLinear.set_assignment``
  (``src/isa/measured_deployment/operator.py:126-131``: slopes = dI/dV per segment,
  intercepts = I[:-1] - slopes * Vg[:-1], in fp32),
* the segment rules: ``searchsorted(vg, v, right=True) - 1`` (``operator.py:209-211``), the
  uniform grid of the fused kernel ``int((v - vmin) * inv_step)``
  (``kernels/measured_lut_triton.py:69-72``) and the rounded bins of the ``vin_lut_bins``
  mode (``operator.py:190-201``),
* the forward ``clamp(sum_k ((S[a] - S[b]) v + (C[a] - C[b])) * scale * r_tia)`` with
  ``v = clamp(x, lookup_min, lookup_max)`` (``operator.py:177-224``,
  ``measured_lut_triton.py:58-139``), and its gradient for x.
"""

from __future__ import annotations

import numpy as np

f32 = np.float32


def curve_tables(vg: np.ndarray, currents: np.ndarray):
    """(slopes, intercepts) [curves, segments] in fp32, operator.py:126-131."""
    vg = vg.astype(f32)
    cur = currents.astype(f32)
    dv = (vg[1:] - vg[:-1]).astype(f32)
    slopes = ((cur[:, 1:] - cur[:, :-1]) / dv[None, :]).astype(f32)
    intercepts = (cur[:, :-1] - (slopes * vg[None, :-1]).astype(f32)).astype(f32)
    return slopes, intercepts


def segments_search(v: np.ndarray, vg: np.ndarray) -> np.ndarray:
    s = np.searchsorted(vg.astype(f32), v, side="right") - 1
    return np.clip(s, 0, vg.size - 2)


def segments_uniform(v: np.ndarray, vmin: float, inv_step: float, n_seg: int) -> np.ndarray:
    t = ((v.astype(f32) - f32(vmin)).astype(f32) * f32(inv_step)).astype(f32)
    s = np.where(np.isnan(t), 0, np.trunc(np.nan_to_num(t))).astype(np.int64)
    return np.clip(s, 0, n_seg - 1)


def segments_round(v: np.ndarray, lookup_min: float, scale: float, bins: int) -> np.ndarray:
    if bins == 1:
        return np.zeros(v.shape, dtype=np.int64)
    t = ((v.astype(f32) - f32(lookup_min)).astype(f32) * f32(scale)).astype(f32)
    return np.clip(np.rint(t).astype(np.int64), 0, bins - 1)


def clamp_input(x: np.ndarray, lookup_min: float, lookup_max: float) -> np.ndarray:
    return np.clip(x.astype(f32), f32(lookup_min), f32(lookup_max))


def forward(v: np.ndarray, seg: np.ndarray, ids_a: np.ndarray, ids_b, slopes: np.ndarray, intercepts: np.ndarray,
            current_scale: float, r_tia: float, out_min: float, out_max: float):
    """(out, pre) for clamped inputs v [M,K] and their segments [M,K]; ids [O,K]
    (ids_b None: pair mode). Per-cell fp32 terms, float64 sums."""
    M, K = v.shape
    O = ids_a.shape[0]
    pre = np.zeros((M, O), dtype=np.float64)
    for k in range(K):
        s = seg[:, k][:, None]                    # [M, 1]
        a = ids_a[:, k][None, :]                  # [1, O]
        ds = slopes[a, s]
        dc = intercepts[a, s]
        if ids_b is not None:
            b = ids_b[:, k][None, :]
            ds = (ds - slopes[b, s]).astype(f32)
            dc = (dc - intercepts[b, s]).astype(f32)
        term = ((ds * v[:, k][:, None]).astype(f32) + dc).astype(f32)
        pre += term
    pre = pre * float(current_scale)
    out = np.clip(pre * float(r_tia), out_min, out_max)
    return out, pre


def grad_x(x: np.ndarray, v: np.ndarray, seg: np.ndarray, ids_a: np.ndarray, ids_b, slopes: np.ndarray,
           g: np.ndarray, pre: np.ndarray, current_scale: float, r_tia: float, out_min: float, out_max: float,
           lookup_min: float, lookup_max: float) -> np.ndarray:
    """dX = [lookup_min <= x <= lookup_max] * scale * sum_o G r [out_min <= pre r <= out_max] dS."""
    y0 = pre * float(r_tia)
    gm = g.astype(np.float64) * float(r_tia) * ((y0 >= out_min) & (y0 <= out_max))
    M, K = v.shape
    dx = np.zeros((M, K), dtype=np.float64)
    for k in range(K):
        s = seg[:, k][:, None]
        ds = slopes[ids_a[:, k][None, :], s]
        if ids_b is not None:
            ds = (ds - slopes[ids_b[:, k][None, :], s]).astype(f32)
        dx[:, k] = (gm * ds).sum(axis=1)
    inside = (x >= lookup_min) & (x <= lookup_max)
    return dx * float(current_scale) * inside
