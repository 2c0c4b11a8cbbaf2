"""Small-problem plans through the C ABI against the CPU oracle, at the library's default
options (no second table copy below 2^28 cells): the one-round token and K splits, and the
backward's grouped order whose blocks sum four token splits' dVth partials in LDS before
writing them (plan_info "dv_planes" = splits / 4). Gates as in test_gpu_parity.py: forward
<= 1e-4, dX and dVth+- <= 1e-3 norm-wise. Gradient subsets and a repeat run must be bitwise
equal to the full run."""

from __future__ import annotations

import pytest
import torch

from tests.helpers import errs, flash_cfg, make_inputs, oracle_all

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-4
BWD_TOL = 1e-3

# (M, K, O, x_mode, vth_mode): the ViT-S up-projection and its transpose (configs[0] shape),
# a ragged shape, and trained-like thresholds
SHAPES = [
    (520, 192, 768, "mapped", "init"),
    (520, 768, 192, "signed", "full"),
    (130, 96, 300, "mapped", "full"),
    (203, 40, 520, "signed", "init"),
]


def _run(x, vp, vn, g, cfg, dev, need_x=True, need_w=True):
    from isa.approximations.delta_lut import get_packed_tables, lut_range
    from isa.kernels.transformer_ffn import ops

    dmin, dmax, n = lut_range(cfg)
    fwd, bwd = get_packed_tables(cfg, dev)
    out = ops.lut_forward(x, vp, vn, fwd, n, dmin, dmax, cfg["V_sat"], -4.0, 4.0)
    gx, gp, gn = ops.lut_backward(x, vp, vn, g, bwd, n, dmin, dmax, cfg["V_sat"], need_x, need_w)
    torch.cuda.synchronize()
    return out, gx, gp, gn


@pytest.mark.parametrize("M,K,O,x_mode,vth_mode", SHAPES)
def test_small_plan_parity(cuda_device, M, K, O, x_mode, vth_mode):
    from isa.kernels.transformer_ffn import ops

    print(f"[case] small plan M={M} K={K} O={O} {x_mode}/{vth_mode}", flush=True)
    assert ops.copy_min_cells() == 1 << 28
    cfg = flash_cfg(4096)
    n = cfg["LUT_DELTA_SIZE"]
    pb = ops.plan_info("backward", M, K, O, n)
    pf = ops.plan_info("forward", M, K, O, n)
    print("plans", pf, pb, flush=True)
    assert pf["mode_offset"] == -1 and pb["mode_offset"] == -1  # one table copy below the threshold
    assert pb["blocks"] <= 2 * 256 and pf["blocks"] <= 2 * 256  # one round of blocks
    if (M, K, O) == (520, 192, 768):
        assert pb["dv_planes"] * 4 == pb["splits"]  # the grouped order
    x, vp, vn, g = make_inputs(M, K, O, seed=M + 7 * K, x_mode=x_mode, vth_mode=vth_mode)
    ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg)
    xd, pd, nd, gd = (t.to(cuda_device) for t in (x, vp, vn, g))
    out, gx, gp, gn = _run(xd, pd, nd, gd, cfg, cuda_device)
    e = [errs(out, ref_out)[0], errs(gx, ref_dx)[0], errs(gp, ref_gp)[0], errs(gn, ref_gn)[0]]
    print([f"{v:.2e}" for v in e], flush=True)
    assert e[0] <= FWD_TOL and max(e[1:]) <= BWD_TOL, e
    # dVth alone and dX alone: same plans for the shared parts, bitwise-equal results
    _, gx0, gp1, gn1 = _run(xd, pd, nd, gd, cfg, cuda_device, need_x=False)
    assert gx0 is None and torch.equal(gp1, gp) and torch.equal(gn1, gn)
    _, gx1, gp0, _ = _run(xd, pd, nd, gd, cfg, cuda_device, need_w=False)
    assert gp0 is None and torch.equal(gx1, gx)
    again = _run(xd, pd, nd, gd, cfg, cuda_device)
    for u, v in zip((out, gx, gp, gn), again):
        assert torch.equal(u, v)
