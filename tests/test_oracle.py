"""Pins the CPU oracle (CPU only, no GPU).

A restated formula checked against itself pins nothing, so every check here compares
the oracle with something independent of it: the closed form evaluated separately in
float64, the reference's own known-answer inputs and tolerances, torch autograd of the
exact formula, convergence of the LUT path to the exact formula as the table grows,
algebraic invariants, and a brute-force pure-Python loop on tiny inputs.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import exact, oracle
from tests.helpers import flash_cfg, make_inputs

# tests/test_flash_formula.py:19-25 of the reference (uA units, U_T = 0.026)
REF_TEST_CFG = {"I_S": 0.75875, "n": 4.1360, "U_T": 0.026, "V_D": 0.1, "V_sat": 8.2624}


def _closed_form_table(cfg, dmin, dmax, n):
    """float64 closed form, written independently of ekv_oracle.c."""
    j = np.arange(n, dtype=np.float64)
    d = dmin + j * (dmax - dmin) / (n - 1)
    k = 1.0 / (2.0 * cfg["n"] * cfg["U_T"])
    u1, u2 = d * k, (d - cfg["V_D"]) * k
    sp1, sp2 = np.logaddexp(0.0, u1), np.logaddexp(0.0, u2)
    sig1, sig2 = 1.0 / (1.0 + np.exp(-u1)), 1.0 / (1.0 + np.exp(-u2))
    ti = cfg["I_S"] * (sp1 ** 2 - sp2 ** 2)
    td = cfg["I_S"] * 2.0 * k * (sp1 * sig1 - sp2 * sig2)
    return ti, td


@pytest.mark.parametrize("size", [2, 257, 4096, 8192])
def test_table_matches_closed_form(size):
    cfg = flash_cfg(size)
    dmin, dmax, n = oracle.lut_range(cfg)
    assert (dmin, dmax) == (-9.0, 4.0)
    ti, td = oracle.lut_tables(cfg)
    ci, cd = _closed_form_table(cfg, dmin, dmax, n)
    # one rounding to fp32 (plus the softplus threshold at 20, a 2e-9 relative step)
    assert np.allclose(ti, ci, rtol=2e-7, atol=1e-30)
    assert np.allclose(td, cd, rtol=2e-7, atol=1e-30)
    assert np.all(np.diff(ti) >= 0) and np.all(td >= 0)  # I is monotone in dV, D = dI/ddV >= 0


def test_table_matches_reference_test_grid():
    """tests/test_flash_formula.py:56-84: grid (-1, 3, 257), rtol 8e-3, atol 3e-3."""
    ti, _ = oracle.lut_tables(dict(REF_TEST_CFG, **{"LUT_DELTA_SIZE": 257}), size=257, delta_min=-1.0, delta_max=3.0)
    delta = torch.linspace(-1.0, 3.0, 257, dtype=torch.float32)
    k = 1.0 / (2.0 * REF_TEST_CFG["n"] * REF_TEST_CFG["U_T"])
    expected = REF_TEST_CFG["I_S"] * (F.softplus(delta * k).square() - F.softplus((delta - REF_TEST_CFG["V_D"]) * k).square())
    assert torch.allclose(torch.from_numpy(ti), expected, rtol=8.0e-3, atol=3.0e-3)
    # and far tighter than the reference's bf16-absorbing tolerance
    assert torch.allclose(torch.from_numpy(ti), expected, rtol=1e-5, atol=1e-7)


def test_table_matches_torch_fp32_construction():
    """The reference builds the table with fp32 torch ops (delta_lut.py:25-34); ours rounds
    the fp64 value once. Norm-wise the two agree to fp32 evaluation error; elementwise the
    reference's derivative table loses its subthreshold end to the fp32 cancellation of
    1 - exp(-sp) (exactly zero below dV ~ -3.73 V, ~0.7% off at -2.5 V), which ours keeps."""
    cfg = flash_cfg(4096)
    dmin, dmax, n = oracle.lut_range(cfg)
    ri, rd, _, _ = oracle.reference_lut_tables(cfg)
    ti, td = oracle.lut_tables(cfg)
    assert oracle.normwise_error(ti, ri) < 1e-5
    assert oracle.normwise_error(td, rd) < 1e-5
    delta = dmin + np.arange(n) * (dmax - dmin) / (n - 1)
    assert np.all(rd[delta <= -3.8] == 0.0) and np.all(td[delta <= -3.8] > 0.0)
    near = (delta > -2.6) & (delta < -2.4)
    rel = np.abs(td[near].astype(np.float64) - rd[near]) / td[near]
    assert 1e-3 < rel.max() < 2e-2


def test_exact_formula_known_answers():
    """tests/test_flash_formula.py:16-31 inputs: exact current == restated softplus form."""
    vgs = torch.tensor([0.4, 1.2, 2.7], dtype=torch.float64)
    vth = torch.tensor([0.1, 0.8, 2.0], dtype=torch.float64)
    c = REF_TEST_CFG
    k = 1.0 / (2.0 * c["n"] * c["U_T"])
    expected = [c["I_S"] * (math.log1p(math.exp((v - t) * k)) ** 2 - math.log1p(math.exp((v - t - c["V_D"]) * k)) ** 2)
                / (1.0 + v / c["V_sat"]) for v, t in zip(vgs.tolist(), vth.tolist())]
    actual = exact.ekv_current(vgs, vth, c)
    assert torch.allclose(actual, torch.tensor(expected, dtype=torch.float64), rtol=1e-12, atol=1e-12)


def test_exact_analytic_gradients_match_autograd():
    """tests/test_flash_formula.py:33-53 inputs and tolerance."""
    vgs = torch.tensor([0.5, 1.4, 3.0], dtype=torch.float64, requires_grad=True)
    vth = torch.tensor([0.2, 0.9, 2.2], dtype=torch.float64, requires_grad=True)
    cur = exact.ekv_current(vgs, vth, REF_TEST_CFG)
    gv, gt = torch.autograd.grad(cur.sum(), (vgs, vth))
    assert torch.allclose(exact.ekv_current_grad_v(vgs, vth, REF_TEST_CFG), gv, rtol=1e-10, atol=1e-10)
    assert torch.allclose(exact.ekv_current_grad_vth(vgs, vth, REF_TEST_CFG), gt, rtol=1e-10, atol=1e-10)


def test_exact_products_brute_force_tiny():
    """diff_current_f64 (the exact-path checker) against a pure-Python triple loop with
    math.log1p/exp, including the softplus threshold (u > 20) and the sign of each term."""
    c = REF_TEST_CFG
    k = 1.0 / (2.0 * c["n"] * c["U_T"])

    def sp(u):
        return u if u > 20.0 else math.log1p(math.exp(u))

    def cur(v, t):
        return c["I_S"] * (sp((v - t) * k) ** 2 - sp((v - t - c["V_D"]) * k) ** 2) / (1.0 + v / c["V_sat"])

    g = torch.Generator().manual_seed(11)
    x = torch.rand(3, 5, generator=g, dtype=torch.float64) * 12.0 - 4.0  # reaches u > 20
    vp = torch.rand(4, 5, generator=g, dtype=torch.float64) * 5.0
    vn = torch.rand(4, 5, generator=g, dtype=torch.float64) * 5.0
    want = [[sum(cur(x[m, i].item(), vp[o, i].item()) - cur(x[m, i].item(), vn[o, i].item()) for i in range(5))
             for o in range(4)] for m in range(3)]
    got = exact.diff_current_f64(x, vp, vn, c, chunk=3)
    assert torch.allclose(got, torch.tensor(want, dtype=torch.float64), rtol=1e-12, atol=1e-12)


def test_exact_product_gradients_match_autograd():
    """diff_current_grads_f64 == torch autograd of sum(G * Idiff) of the closed form."""
    c = REF_TEST_CFG
    g = torch.Generator().manual_seed(12)
    x = (torch.rand(6, 7, generator=g, dtype=torch.float64) * 8.0 - 4.0).requires_grad_(True)
    vp = (torch.rand(9, 7, generator=g, dtype=torch.float64) * 5.0).requires_grad_(True)
    vn = (torch.rand(9, 7, generator=g, dtype=torch.float64) * 5.0).requires_grad_(True)
    G = torch.randn(6, 9, generator=g, dtype=torch.float64)
    cur = lambda v, t: exact.ekv_current(v, t, c)  # noqa: E731
    idiff = (cur(x.unsqueeze(1), vp.unsqueeze(0)) - cur(x.unsqueeze(1), vn.unsqueeze(0))).sum(-1)
    ax, ap, an = torch.autograd.grad((G * idiff).sum(), (x, vp, vn))
    dx, dp, dn = exact.diff_current_grads_f64(x.detach(), vp.detach(), vn.detach(), G, c, chunk=4)
    for a, b in ((dx, ax), (dp, ap), (dn, an)):
        assert torch.allclose(a, b, rtol=1e-10, atol=1e-12)


def test_lookup_boundaries():
    cfg = flash_cfg(4096)
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, td = oracle.lut_tables(cfg)
    h = (dmax - dmin) / (n - 1)
    assert oracle.lut_lookup(ti, dmin - 3.0, dmin, dmax) == ti[0]           # below: T[0]
    assert oracle.lut_lookup(ti, dmax + 3.0, dmin, dmax) == ti[-1]          # above: T[N-1]
    assert oracle.lut_lookup(td, dmax + 3.0, dmin, dmax) == td[-1]          # D is not zeroed outside
    assert oracle.lut_lookup(ti, float("nan"), dmin, dmax) == ti[0]         # NaN -> coordinate 0
    for j in (0, 1, 1000, 2047, 4094, 4095):                                # grid nodes (fp32 coordinates)
        v = oracle.lut_lookup(ti, np.float32(dmin + j * h), dmin, dmax)
        assert abs(v - ti[j]) <= 1e-3 * abs(ti[j] - ti[j - 1 if j else 1]) + 1e-30
    # halfway between nodes: the mean of the neighbours
    j = 3000
    v = oracle.lut_lookup(ti, np.float32(dmin + (j + 0.5) * h), dmin, dmax)
    assert abs(v - 0.5 * (ti[j] + ti[j + 1])) <= 2e-3 * abs(ti[j + 1] - ti[j])


def _brute_forward(x, wp, wn, ti, dmin, dmax, v_sat):
    """Pure-Python loops (tiny inputs), written from the reference equations directly."""
    n = len(ti)
    s = (n - 1) / (dmax - dmin)

    def L(d):
        c = min(max((d - dmin) * s, 0.0), n - 1.0)
        i0 = int(c)
        i1 = min(i0 + 1, n - 1)
        a = c - i0
        return float(ti[i0]) * (1 - a) + float(ti[i1]) * a

    M, K = x.shape
    O = wp.shape[0]
    out = np.zeros((M, O))
    for m in range(M):
        for o in range(O):
            out[m, o] = sum((L(float(x[m, k]) - float(wp[o, k])) - L(float(x[m, k]) - float(wn[o, k])))
                            / (1.0 + float(x[m, k]) / v_sat) for k in range(K))
    return out


def test_forward_brute_force_tiny():
    cfg = flash_cfg(512)
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, _ = oracle.lut_tables(cfg)
    x, vp, vn, _ = make_inputs(5, 7, 6, seed=1, x_mode="signed", vth_mode="full")
    got = oracle.forward(x.numpy(), vp.numpy(), vn.numpy(), ti, dmin, dmax, cfg["V_sat"], -1e9, 1e9)
    ref = _brute_forward(x.numpy(), vp.numpy(), vn.numpy(), ti, dmin, dmax, cfg["V_sat"])
    assert oracle.normwise_error(got, ref) < 1e-5


@pytest.mark.parametrize("x_mode", ["mapped", "signed"])
def test_lut_converges_to_exact_formula(x_mode):
    """The LUT oracle tends to the exact formula (and its analytic gradients, which are
    pinned by autograd above) as N grows, at second order in the grid step. A dropped
    term, a wrong sign or a transposed operand would leave an O(1) gap."""
    x, vp, vn, g = make_inputs(12, 40, 24, seed=4, x_mode=x_mode, vth_mode="full")
    cfg = flash_cfg(4096)
    xd, pd, nd, gd = (t.double() for t in (x, vp, vn, g))
    ex_out = exact.exact_forward(xd, pd, nd, cfg).numpy()
    ex_dx, ex_dp, ex_dn = (t.numpy() for t in exact.exact_backward(xd, pd, nd, gd, cfg))
    prev = None
    for size in (1024, 4096, 16384, 65536):
        ti, td = oracle.lut_tables(cfg, size=size)
        dmin, dmax, _ = oracle.lut_range(cfg)
        out = oracle.forward(x.numpy(), vp.numpy(), vn.numpy(), ti, dmin, dmax, cfg["V_sat"], -1e9, 1e9)
        dx, dp, dn = oracle.backward(x.numpy(), vp.numpy(), vn.numpy(), g.numpy(), ti, td, dmin, dmax, cfg["V_sat"])
        e = [oracle.normwise_error(out, ex_out), oracle.normwise_error(dx, ex_dx),
             oracle.normwise_error(dp, ex_dp), oracle.normwise_error(dn, ex_dn)]
        if prev is not None:
            for a, b in zip(e, prev):
                assert a < b / 3.0 or a < 5e-6   # ~4x per halving of the step until the fp32 floor
        prev = e
    assert max(prev) < 2e-5


def test_invariants():
    cfg = flash_cfg(4096)
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, td = oracle.lut_tables(cfg)
    x, vp, vn, g = make_inputs(9, 30, 11, seed=6, vth_mode="full")
    X, P, N, G = x.numpy(), vp.numpy(), vn.numpy(), g.numpy()
    big = 1e9
    # equal thresholds -> exactly zero current and dX, dVth+ == -dVth-
    assert np.count_nonzero(oracle.forward(X, P, P, ti, dmin, dmax, cfg["V_sat"], -big, big)) == 0
    dx, dp, dn = oracle.backward(X, P, P, G, ti, td, dmin, dmax, cfg["V_sat"])
    assert np.count_nonzero(dx) == 0 and np.array_equal(dp, -dn)
    # swapping the pair negates everything
    f1 = oracle.forward(X, P, N, ti, dmin, dmax, cfg["V_sat"], -big, big)
    f2 = oracle.forward(X, N, P, ti, dmin, dmax, cfg["V_sat"], -big, big)
    assert np.array_equal(f1, -f2)
    dx2, dp2, dn2 = oracle.backward(X, N, P, G, ti, td, dmin, dmax, cfg["V_sat"])
    dx1, dp1, dn1 = oracle.backward(X, P, N, G, ti, td, dmin, dmax, cfg["V_sat"])
    assert np.allclose(dx1, -dx2) and np.array_equal(dp1, -dn2) and np.array_equal(dn1, -dp2)
    # additivity over K
    a = oracle.forward(X[:, :13], P[:, :13], N[:, :13], ti, dmin, dmax, cfg["V_sat"], -big, big)
    b = oracle.forward(X[:, 13:], P[:, 13:], N[:, 13:], ti, dmin, dmax, cfg["V_sat"], -big, big)
    assert np.allclose(f1, a + b, rtol=1e-12, atol=1e-12 * np.abs(f1).max())
    # linearity in G
    dxa, dpa, dna = oracle.backward(X, P, N, 2.5 * G, ti, td, dmin, dmax, cfg["V_sat"])
    assert np.allclose(dxa, 2.5 * dx1, rtol=1e-6) and np.allclose(dpa, 2.5 * dp1, rtol=1e-6)
    # the output clamp (ekv_lut_triton.py:61)
    clamped = oracle.forward(X, P, N, ti, dmin, dmax, cfg["V_sat"], -1e-6, 1e-6)
    assert np.array_equal(clamped, np.clip(f1, -1e-6, 1e-6))


def test_nan_rules():
    """NaN x -> NaN cells (r is NaN) whose sum clamps to out_min (fmin/fmax); NaN vth reads T[0]."""
    cfg = flash_cfg(4096)
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, td = oracle.lut_tables(cfg)
    x, vp, vn, g = make_inputs(4, 6, 5, seed=7)
    X, P, N, G = x.numpy().copy(), vp.numpy().copy(), vn.numpy().copy(), g.numpy()
    X[1, 2] = np.nan
    P[3, 4] = np.nan
    out = oracle.forward(X, P, N, ti, dmin, dmax, cfg["V_sat"], -4.0, 4.0)
    assert np.all(out[1] == -4.0) and np.isfinite(out).all()
    dx, dp, dn = oracle.backward(X, P, N, G, ti, td, dmin, dmax, cfg["V_sat"])
    assert np.isnan(dx[1, 2]) and np.isnan(dp[:, 2]).all() and np.isfinite(dp[3, 4])
