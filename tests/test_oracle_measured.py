"""Pins the measured-codebook oracle (CPU only): its tables against the reference's torch
formulation, its per-cell values against textbook piecewise-linear interpolation, and its
forward and gradient against the reference's masked-GEMM formulation
(operator.py:177-224) evaluated in float64 with torch autograd."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import measured
from tests.helpers import make_codebook


def _reference_tables_torch(vg, currents):
    """operator.py:126-131 on the CPU."""
    dv = vg[1:] - vg[:-1]
    slopes = (currents[:, 1:] - currents[:, :-1]) / dv.unsqueeze(0)
    intercepts = currents[:, :-1] - slopes * vg[:-1].unsqueeze(0)
    return slopes, intercepts


def test_tables_match_reference_ops():
    for uniform in (True, False):
        vg, cur = make_codebook(24, 61, seed=1, uniform=uniform)
        s_ref, c_ref = _reference_tables_torch(vg, cur)
        s, c = measured.curve_tables(vg.numpy(), cur.numpy())
        assert np.array_equal(s, s_ref.numpy()) and np.array_equal(c, c_ref.numpy())


def test_segment_values_are_linear_interpolation():
    """S[a][seg(v)] v + C[a][seg(v)] == np.interp(v, vg, I[a]) (the measured curve itself)."""
    vg, cur = make_codebook(24, 61, seed=2, uniform=False)
    s, c = measured.curve_tables(vg.numpy(), cur.numpy())
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.uniform(0.0, 4.0, 500).astype(np.float32), vg.numpy()])  # includes the nodes
    seg = measured.segments_search(v, vg.numpy())
    for a in range(24):
        got = s[a, seg].astype(np.float64) * v + c[a, seg]
        want = np.interp(v.astype(np.float64), vg.numpy().astype(np.float64), cur[a].numpy().astype(np.float64))
        assert np.max(np.abs(got - want)) <= 2e-6 * np.max(np.abs(want))


def test_uniform_and_search_segments_agree_on_a_uniform_grid():
    vg, _ = make_codebook(4, 61, seed=3)
    v = np.random.default_rng(1).uniform(0.0, 4.0, 20000).astype(np.float32)
    a = measured.segments_search(v, vg.numpy())
    b = measured.segments_uniform(v, float(vg[0]), 1.0 / float(vg[1] - vg[0]), 60)
    assert np.mean(a == b) > 0.999 and np.all(np.abs(a - b) <= 1)


def _reference_forward_f64(x, pos, neg, vg, cur, lookup, r_tia, signed, bins=0):
    """operator.py:177-224 restated with torch in float64: masks and F.linear over the
    expanded per-segment (or per-bin) difference matrices."""
    lmin, lmax = lookup
    flat = x.double().clamp(lmin, lmax)
    out = torch.zeros(flat.shape[0], pos.shape[0], dtype=torch.float64)
    s, c = _reference_tables_torch(vg, cur)
    if bins > 0:
        centers = torch.linspace(lmin, lmax, bins, dtype=torch.float32)
        for b in range(bins):
            value = centers[b].clamp(vg[0], vg[-1])
            up = torch.searchsorted(vg, value, right=True).clamp(1, vg.numel() - 1)
            lo = up - 1
            alpha = (value - vg[lo]) / (vg[up] - vg[lo])
            meas = cur[:, lo] + alpha * (cur[:, up] - cur[:, lo])
            diff = (meas[pos.long()] - meas[neg.long()]).double()
            scale = (bins - 1) / (lmax - lmin) if bins > 1 else 1.0
            bin_id = torch.round((x.float().clamp(lmin, lmax) - lmin) * scale).long().clamp(0, bins - 1)
            out = out + F.linear((bin_id == b).double(), diff)
    else:
        seg = torch.searchsorted(vg, flat.float(), right=True).sub(1).clamp(0, vg.numel() - 2)
        for j in range(vg.numel() - 1):
            mask = (seg == j).double()
            da = (s[:, j][pos.long()] - s[:, j][neg.long()]).double()
            db = (c[:, j][pos.long()] - c[:, j][neg.long()]).double()
            out = out + F.linear(flat * mask, da) + F.linear(mask, db)
    return (out * r_tia).clamp(*signed)


def test_forward_and_gradient_match_reference_formulation():
    vg, cur = make_codebook(24, 61, seed=4, uniform=False)
    g = torch.Generator().manual_seed(5)
    M, K, O = 7, 13, 11
    x = (torch.rand(M, K, generator=g) * 4.6 - 0.3)  # some inputs outside the lookup range
    pos = torch.randint(0, 24, (O, K), generator=g)
    neg = torch.randint(0, 24, (O, K), generator=g)
    r, signed = 1e6, (-4.0, 4.0)
    xr = x.double().requires_grad_(True)
    ref = _reference_forward_f64(xr, pos, neg, vg, cur, (0.0, 4.0), r, signed)
    G = torch.randn(M, O, generator=g, dtype=torch.float64)
    ref.backward(G)
    s, c = measured.curve_tables(vg.numpy(), cur.numpy())
    v = measured.clamp_input(x.numpy(), 0.0, 4.0)
    seg = measured.segments_search(v, vg.numpy())
    out, pre = measured.forward(v, seg, pos.numpy(), neg.numpy(), s, c, 1.0, r, *signed)
    assert np.max(np.abs(out - ref.detach().numpy())) <= 1e-6 * np.max(np.abs(ref.detach().numpy()))
    assert np.any(np.abs(out) == 4.0)  # the clamp is exercised
    dx = measured.grad_x(x.numpy(), v, seg, pos.numpy(), neg.numpy(), s, G.numpy(), pre, 1.0, r, *signed, 0.0, 4.0)
    assert np.max(np.abs(dx - xr.grad.numpy())) <= 1e-6 * np.max(np.abs(xr.grad.numpy()))


def test_bins_mode_matches_reference_formulation():
    vg, cur = make_codebook(24, 61, seed=6)
    g = torch.Generator().manual_seed(7)
    M, K, O, bins = 5, 9, 6, 16
    x = torch.rand(M, K, generator=g) * 4.0
    pos = torch.randint(0, 24, (O, K), generator=g)
    neg = torch.randint(0, 24, (O, K), generator=g)
    ref = _reference_forward_f64(x, pos, neg, vg, cur, (0.0, 4.0), 1e5, (-4.0, 4.0), bins=bins)
    # the kernel's bins table: every state's current at every bin centre, zero slopes
    centers = torch.linspace(0.0, 4.0, bins)
    at = []
    for cen in centers:
        up = torch.searchsorted(vg, cen.clamp(vg[0], vg[-1]), right=True).clamp(1, vg.numel() - 1)
        lo = up - 1
        alpha = (cen - vg[lo]) / (vg[up] - vg[lo])
        at.append(cur[:, lo] + alpha * (cur[:, up] - cur[:, lo]))
    table_c = torch.stack(at, dim=1).numpy()
    v = measured.clamp_input(x.numpy(), 0.0, 4.0)
    seg = measured.segments_round(v, 0.0, (bins - 1) / 4.0, bins)
    out, _ = measured.forward(v, seg, pos.numpy(), neg.numpy(), np.zeros_like(table_c), table_c, 1.0, 1e5, -4.0, 4.0)
    assert np.max(np.abs(out - ref.numpy())) <= 1e-6 * max(np.max(np.abs(ref.numpy())), 1e-30)


def test_equal_ids_give_zero():
    vg, cur = make_codebook(8, 21, seed=8)
    s, c = measured.curve_tables(vg.numpy(), cur.numpy())
    ids = np.random.default_rng(2).integers(0, 8, (5, 6))
    v = np.random.default_rng(3).uniform(0, 4, (4, 6)).astype(np.float32)
    out, _ = measured.forward(v, measured.segments_search(v, vg.numpy()), ids, ids, s, c, 1.0, 1e5, -4.0, 4.0)
    assert np.all(out == 0.0)
