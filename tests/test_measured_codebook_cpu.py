"""Measured-codebook host logic on the CPU (no kernel runs): currents_at against numpy's
piecewise-linear interpolation of the measured curves, and install_fused_backend's shared
codebook (one copy of the codebook and its coefficient tables for all layers configured
from the same source tensors on one device, as fused_backend.py:37-131)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import flash_cfg, make_codebook


def _layer(K=12, O=10):
    from isa.measured_deployment.operator import DeploymentAwareCIMLinear

    return DeploymentAwareCIMLinear(K, O, flash_cfg(4096))


@pytest.mark.parametrize("uniform", [True, False])
def test_currents_at_matches_numpy_interp(uniform):
    vg, cur = make_codebook(24, 61, seed=4, uniform=uniform)
    layer = _layer()
    layer.configure_codebook(vg, cur)
    pts = np.concatenate([np.linspace(-0.5, 4.5, 97), vg.numpy()[::7]]).astype(np.float32)
    want = np.stack([np.interp(pts.astype(np.float64), vg.numpy().astype(np.float64), c.astype(np.float64))
                     for c in cur.numpy()])
    got = layer.currents_at(torch.from_numpy(pts)).numpy()
    assert got.shape == (24, pts.size)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    one = layer.currents_at(1.234).numpy()
    assert one.shape == (24,)
    assert np.allclose(one, [np.interp(1.234, vg.numpy(), c) for c in cur.numpy()], rtol=1e-5, atol=0)


def test_bins_table_holds_currents_at_bin_centres():
    vg, cur = make_codebook(24, 61, seed=5, uniform=False)
    layer = _layer()
    layer.configure_codebook(vg, cur, vin_lut_bins=16)
    centers = np.linspace(layer.lookup_min, layer.lookup_max, 16)
    want = np.stack([np.interp(centers, vg.numpy(), c) for c in cur.numpy()])
    assert torch.count_nonzero(layer.curve_slopes) == 0
    assert np.allclose(layer.curve_intercepts.numpy(), want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


def test_install_fused_backend_shares_one_codebook(monkeypatch):
    from isa.measured_deployment import operator
    from isa.measured_deployment.fused_backend import install_fused_backend

    from isa.measured_deployment import fused_backend

    monkeypatch.setattr(operator.DeploymentAwareCIMLinear, "_fg50_fused_backend_installed", False, raising=False)
    monkeypatch.setattr(fused_backend, "_SHARED_CODEBOOKS", {})
    vg, cur = make_codebook(24, 61, seed=6)
    a, b = _layer(), _layer()
    a.configure_codebook(vg, cur)
    b.configure_codebook(vg, cur)
    assert a.curve_slopes.data_ptr() != b.curve_slopes.data_ptr()  # not installed: tables per layer
    install_fused_backend()
    install_fused_backend()  # idempotent
    c, d, e = _layer(), _layer(), _layer()
    c.configure_codebook(vg, cur)
    d.configure_codebook(vg, cur)
    for name in ("measured_vg", "measured_currents", "curve_slopes", "curve_intercepts", "_segment_slopes"):
        assert getattr(c, name).data_ptr() == getattr(d, name).data_ptr(), name
    vg2, cur2 = make_codebook(24, 61, seed=7)
    e.configure_codebook(vg2, cur2)
    assert e.curve_slopes.data_ptr() != c.curve_slopes.data_ptr()
    assert torch.equal(c.curve_slopes, a.curve_slopes)  # same values as an unshared layer
    c.set_assignment(torch.randint(0, 24, (10, 12)), torch.randint(0, 24, (10, 12)))
    d.set_assignment(torch.zeros(10, 12, dtype=torch.long), torch.ones(10, 12, dtype=torch.long))
    assert not torch.equal(c.pos_idx, d.pos_idx)  # assignments stay per layer
    with pytest.raises(ValueError, match="outside the codebook"):
        d.set_assignment(torch.full((10, 12), 24), torch.zeros(10, 12, dtype=torch.long))


def test_shared_codebook_entry_follows_its_sources(monkeypatch):
    """The shared-codebook cache holds its sources weakly: freeing them frees their entry (the
    layers keep the device tables they were given), and an in-place edit of a source is a new
    codebook, not a stale hit."""
    import gc

    from isa.measured_deployment import fused_backend, operator
    from isa.measured_deployment.fused_backend import install_fused_backend

    monkeypatch.setattr(operator.DeploymentAwareCIMLinear, "_fg50_fused_backend_installed", False, raising=False)
    monkeypatch.setattr(fused_backend, "_SHARED_CODEBOOKS", {})
    monkeypatch.setattr(fused_backend, "_WATCHED_SOURCES", set())
    install_fused_backend()
    vg, cur = make_codebook(24, 61, seed=8)
    a, b = _layer(), _layer()
    a.configure_codebook(vg, cur)
    assert len(fused_backend._SHARED_CODEBOOKS) == 1
    before = a.curve_slopes.clone()
    cur.mul_(2.0)  # in place: the cached tables no longer describe this tensor
    b.configure_codebook(vg, cur)
    assert len(fused_backend._SHARED_CODEBOOKS) == 1
    assert torch.allclose(b.curve_slopes, 2.0 * before, rtol=1e-6, atol=0)
    assert torch.equal(a.curve_slopes, before)  # a keeps what it was configured with
    c = _layer()
    c.configure_codebook(vg, cur)
    assert c.curve_slopes.data_ptr() == b.curve_slopes.data_ptr()  # same version: shared
    book = next(iter(fused_backend._SHARED_CODEBOOKS.values()))
    assert book["sources"][0]() is vg and book["sources"][1]() is cur
    del vg, cur, book
    gc.collect()
    assert fused_backend._SHARED_CODEBOOKS == {}
    assert fused_backend._WATCHED_SOURCES == set()
    assert torch.allclose(b.curve_slopes, 2.0 * before, rtol=1e-6, atol=0)  # the layers' tables live on
