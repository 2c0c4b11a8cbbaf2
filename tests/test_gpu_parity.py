"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Gates (norm-wise max|d|/max|ref|, against the fp32-table LUT oracle): forward <= 1e-4,
dX and dVth+- <= 1e-3. Elementwise relative error (floor 1e-3 * max|ref|) is printed.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import errs, flash_cfg, make_inputs, oracle_all

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-4
BWD_TOL = 1e-3


@pytest.fixture(autouse=True)
def _small_calls_consider_table_copies():
    """The shapes here are far below the library's copy threshold (ISA_EKV_OPT_COPY_MIN_CELLS):
    let them take the second table copy as large calls do, so that its kernels are checked
    against the oracle."""
    from isa.kernels.transformer_ffn import ops

    prev = ops.copy_min_cells(0)
    yield
    ops.copy_min_cells(prev)


def _dev_run(x, vp, vn, grad, cfg, dev, need_x=True, need_w=True, out_min=-4.0, out_max=4.0, modes=None):
    """Forward and backward through the C ABI. modes: a dict that receives the table mode each
    main kernel ran in ("fwd", "bwd": 1 two copies, 0 one copy, 2 the ranked backward, None no
    second copy)."""
    from isa.approximations.delta_lut import get_packed_tables, lut_range
    from isa.kernels.transformer_ffn import ops

    dmin, dmax, n = lut_range(cfg)
    fwd, bwd = get_packed_tables(cfg, dev)
    xd, pd, nd, gd = (t.to(dev) for t in (x, vp, vn, grad))
    M, K = x.shape
    O = vp.shape[0]
    pf = ops.plan_info("forward", M, K, O, n)
    pb = ops.plan_info("backward", M, K, O, n, need_x, need_w)
    wsf = torch.empty(pf["workspace_bytes"], dtype=torch.uint8, device=dev)
    wsb = torch.empty(pb["workspace_bytes"], dtype=torch.uint8, device=dev)
    out = ops.lut_forward(xd, pd, nd, fwd, n, dmin, dmax, cfg["V_sat"], out_min, out_max, workspace=wsf)
    gx, gp, gn = ops.lut_backward(xd, pd, nd, gd, bwd, n, dmin, dmax, cfg["V_sat"], need_x, need_w, workspace=wsb)
    torch.cuda.synchronize()
    if modes is not None and M * O > 0:
        modes["fwd"] = ops.copy_mode(wsf, pf)
        modes["bwd"] = ops.copy_mode(wsb, pb)
    return out, gx, gp, gn


SHAPES = [
    (1, 1, 1),
    (17, 27, 13),      # reference GPU tile test shape (test_exact_direct_conv.py:137-140)
    (31, 67, 19),      # (test_exact_direct_conv.py:167-171)
    (5, 8, 256),
    (70, 129, 300),    # ragged in every dimension
    (40, 260, 300),    # forward K split into 7 ranges of 40 padded inputs, the last one short
    (1, 3000, 5),      # one token, one output block: eight K ranges of 376 inputs
    (3, 1000, 1000),
    (64, 192, 768),
    (520, 192, 768),   # config 1: ViT-S up-projection, full size
]


@pytest.mark.parametrize("M,K,O", SHAPES)
def test_forward_backward_parity(cuda_device, M, K, O):
    print(f"[case] parity M={M} K={K} O={O}", flush=True)
    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(M, K, O, seed=M * 7 + K)
    ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg)
    out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device)
    e = {"fwd": errs(out, ref_out), "dX": errs(gx, ref_dx), "dVth+": errs(gp, ref_gp), "dVth-": errs(gn, ref_gn)}
    print({k: f"{v[0]:.2e}/{v[1]:.2e}" for k, v in e.items()})
    assert e["fwd"][0] <= FWD_TOL
    assert e["dX"][0] <= BWD_TOL and e["dVth+"][0] <= BWD_TOL and e["dVth-"][0] <= BWD_TOL


def test_parity_random_shape_sweep(cuda_device):
    """Twenty seeded shapes up to 300 x 600 x 700 with mixed input ranges, so the forward plan
    visits every tokens-per-wave choice with and without K splits and the backward many
    token-split counts, each checked against the oracle."""
    rng = np.random.default_rng(20260808)
    cfg = flash_cfg(4096)
    modes = [("mapped", "init"), ("signed", "full"), ("mapped", "full"), ("wide", "wide")]
    for case in range(20):
        M, K, O = int(rng.integers(1, 301)), int(rng.integers(1, 601)), int(rng.integers(1, 701))
        x_mode, vth_mode = modes[case % len(modes)]
        print(f"[case] sweep {case}: M={M} K={K} O={O} {x_mode}/{vth_mode}", flush=True)
        x, vp, vn, g = make_inputs(M, K, O, seed=1000 + case, x_mode=x_mode, vth_mode=vth_mode)
        ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg)
        out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device)
        e = [errs(out, ref_out)[0], errs(gx, ref_dx)[0], errs(gp, ref_gp)[0], errs(gn, ref_gn)[0]]
        assert e[0] <= FWD_TOL and max(e[1:]) <= BWD_TOL, (M, K, O, x_mode, vth_mode, e)


@pytest.mark.parametrize("x_mode,vth_mode", [("signed", "full"), ("wide", "wide"), ("mapped", "full")])
def test_parity_input_ranges(cuda_device, x_mode, vth_mode):
    """fc2-like signed inputs, trained-like thresholds, and out-of-table coordinates (clamping loop)."""
    print(f"[case] ranges {x_mode}/{vth_mode}", flush=True)
    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(96, 160, 320, seed=3, x_mode=x_mode, vth_mode=vth_mode)
    ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg, -math.inf, math.inf)
    out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf)
    e = [errs(out, ref_out)[0], errs(gx, ref_dx)[0], errs(gp, ref_gp)[0], errs(gn, ref_gn)[0]]
    print([f"{v:.2e}" for v in e])
    assert e[0] <= FWD_TOL and max(e[1:]) <= BWD_TOL


@pytest.mark.parametrize("vth_mode", ["init", "full"])
def test_parity_grid_aligned_coordinates(cuda_device, vth_mode):
    """Inputs and thresholds on the table's grid (x = j h, vth = i h, h = (dmax - dmin)/(N - 1),
    rounded to fp32, and their fp32 neighbours), so that most coordinates fall on or within a few
    ulps of a record boundary: the ties of the forward's float-bits record address and the
    segment choice at every boundary, against the oracle. Thresholds near the initial spread
    (windowed forward copies, ranked backward) and over [0, 5] V."""
    from isa.approximations.delta_lut import lut_range

    cfg = flash_cfg(4096)
    dmin, dmax, n = lut_range(cfg)
    h = (dmax - dmin) / (n - 1)
    rng = np.random.default_rng(4242 if vth_mode == "init" else 4343)
    M, K, O = 64, 192, 512
    j = rng.integers(int(-4.0 / h), int(4.0 / h) + 1, size=(M, K))
    if vth_mode == "init":  # the initial thresholds' spread (about 69 records) around the middle
        lo_i, hi_i = int(2.4 / h), int(2.62 / h)
    else:
        lo_i, hi_i = 0, int(5.0 / h)
    ip = rng.integers(lo_i, hi_i + 1, size=(O, K))
    im = rng.integers(lo_i, hi_i + 1, size=(O, K))
    x = (j * h).astype(np.float32)
    nudge = rng.integers(-1, 2, size=x.shape)  # one ulp down, none, one ulp up
    x = np.where(nudge < 0, np.nextafter(x, np.float32(-np.inf)),
                 np.where(nudge > 0, np.nextafter(x, np.float32(np.inf)), x)).astype(np.float32)
    vp = (ip * h).astype(np.float32)
    vn = (im * h).astype(np.float32)
    g = rng.standard_normal((M, O)).astype(np.float32)
    x, vp, vn, g = (torch.from_numpy(np.ascontiguousarray(a)) for a in (x, vp, vn, g))
    print(f"[case] grid-aligned coordinates, thresholds {vth_mode}", flush=True)
    ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg, -math.inf, math.inf)
    modes = {}
    out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf, modes=modes)
    e = {"fwd": errs(out, ref_out), "dX": errs(gx, ref_dx), "dVth+": errs(gp, ref_gp), "dVth-": errs(gn, ref_gn)}
    print(modes, {k: f"{v[0]:.2e}/{v[1]:.2e}" for k, v in e.items()})
    assert e["fwd"][0] <= FWD_TOL
    assert e["dX"][0] <= BWD_TOL and e["dVth+"][0] <= BWD_TOL and e["dVth-"][0] <= BWD_TOL


@pytest.mark.parametrize("value", [0.0, 4.0])
def test_parity_constant_inputs(cuda_device, value):
    """Every input at one of the voltage mapping's clamps (0 V: negative activations; 4 V): all
    tokens share one coordinate, so the coordinate window is the thresholds' own (~70
    records), the forward takes the most windowed copies, and the lanes of a gather read a
    handful of records (broadcasts). Against the oracle, forward and backward."""
    cfg = flash_cfg(4096)
    M, K, O = 128, 256, 1024
    _, vp, vn, g = make_inputs(M, K, O, seed=77)
    x = torch.full((M, K), value, dtype=torch.float32)
    print(f"[case] constant inputs {value} V", flush=True)
    ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg)
    modes = {}
    out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, modes=modes)
    e = {"fwd": errs(out, ref_out), "dX": errs(gx, ref_dx), "dVth+": errs(gp, ref_gp), "dVth-": errs(gn, ref_gn)}
    print(modes, {k: f"{v[0]:.2e}/{v[1]:.2e}" for k, v in e.items()})
    assert 3 <= modes["fwd"] <= 32 and modes["bwd"] == 2, modes
    assert e["fwd"][0] <= FWD_TOL
    assert e["dX"][0] <= BWD_TOL and e["dVth+"][0] <= BWD_TOL and e["dVth-"][0] <= BWD_TOL


@pytest.mark.parametrize("size", [257, 1024, 8192])
def test_parity_table_sizes(cuda_device, size):
    print(f"[case] table size {size}", flush=True)
    cfg = flash_cfg(size)
    x, vp, vn, g = make_inputs(48, 96, 256, seed=size)
    ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg)
    out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device)
    assert errs(out, ref_out)[0] <= FWD_TOL
    assert max(errs(gx, ref_dx)[0], errs(gp, ref_gp)[0], errs(gn, ref_gn)[0]) <= BWD_TOL


@pytest.mark.parametrize("size", [12000, 16384, 32768])
def test_parity_global_memory_tables(cuda_device, size):
    """Tables past the LDS-resident limits (backward > 8192, forward > 16384 entries) are read
    from global memory by their own kernels: parity in the clamp-free loop and, with
    out-of-table coordinates, the clamping loop, plus a ragged K-split shape."""
    cfg = flash_cfg(size, CUDA_SHARED_BACKWARD=False)
    for (M, K, O), (x_mode, vth_mode) in (((48, 96, 300), ("mapped", "init")), ((33, 70, 130), ("wide", "wide")),
                                          ((5, 900, 257), ("signed", "full"))):
        print(f"[case] global-memory table {size}: M={M} K={K} O={O} {x_mode}/{vth_mode}", flush=True)
        x, vp, vn, g = make_inputs(M, K, O, seed=size + M, x_mode=x_mode, vth_mode=vth_mode)
        ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg, -math.inf, math.inf)
        out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf)
        e = [errs(out, ref_out)[0], errs(gx, ref_dx)[0], errs(gp, ref_gp)[0], errs(gn, ref_gn)[0]]
        assert e[0] <= FWD_TOL and max(e[1:]) <= BWD_TOL, (size, M, K, O, e)
        again = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf)
        for u, v in zip((out, gx, gp, gn), again):
            assert torch.equal(u, v)
    # gradient subsets through the same kernels
    x, vp, vn, g = make_inputs(24, 40, 256, seed=3)
    _, gx_all, gp_all, gn_all = _dev_run(x, vp, vn, g, cfg, cuda_device)
    _, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, need_x=True, need_w=False)
    assert gp is None and torch.equal(gx, gx_all)
    _, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, need_x=False, need_w=True)
    assert gx is None and torch.equal(gp, gp_all) and torch.equal(gn, gn_all)


@pytest.mark.parametrize("x_mode,vth_mode", [("mapped", "init"), ("signed", "init"), ("wide", "wide"),
                                             ("mapped", "full")])
def test_parity_8192_entries_table_modes(cuda_device, x_mode, vth_mode):
    """8192-entry tables: with mapped inputs the coordinates reach ~2700 of the 8224 records
    and the backward holds two bank-rotated copies of that window (the thresholds span ~135
    records); signed inputs reach too wide a window and wide thresholds need the clamping
    loop, so those run one interleaved copy; thresholds over [0, 5] V with mapped inputs reach
    too wide a window as well."""
    print(f"[case] 8192 entries {x_mode}/{vth_mode}", flush=True)
    cfg = flash_cfg(8192)
    # the windowed forward copies and the ranked backward are taken exactly when the
    # coordinates reach a window that fits (mapped inputs, initial thresholds); the other cases
    # must run one copy. The forward holds windowed copies (three or more, as many as fit its
    # LDS at the window these random inputs reach) or, when three do not fit, two
    fit = (x_mode, vth_mode) == ("mapped", "init")
    # (64, 203, 300): K % 8 != 0, so padded inputs k >= K run inside the windowed copies
    for M, K, O in ((64, 200, 300), (40, 768, 256), (64, 203, 300)):
        print(f"[case] 8192 entries {x_mode}/{vth_mode} M={M} K={K} O={O}", flush=True)
        x, vp, vn, g = make_inputs(M, K, O, seed=M + K, x_mode=x_mode, vth_mode=vth_mode)
        ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg, -math.inf, math.inf)
        modes = {}
        out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf,
                                   modes=modes)
        e = [errs(out, ref_out)[0], errs(gx, ref_dx)[0], errs(gp, ref_gp)[0], errs(gn, ref_gn)[0]]
        print(modes, [f"{v:.2e}" for v in e])
        if fit:
            assert modes["bwd"] == 2 and (modes["fwd"] in (1, 33) or 3 <= modes["fwd"] <= 16), modes
        else:
            assert modes == {"fwd": 0, "bwd": 0}, modes
        assert e[0] <= FWD_TOL and max(e[1:]) <= BWD_TOL, (M, K, O, e)
        _, gx2, gp2, gn2 = _dev_run(x, vp, vn, g, cfg, cuda_device, need_x=True, need_w=False)
        assert torch.equal(gx2, gx)


def test_forward_16384_entries(cuda_device):
    """The forward keeps the reference's fallback LUT size (delta_lut.py:48) resident in LDS."""
    cfg = flash_cfg(16384)
    x, vp, vn, g = make_inputs(40, 64, 256, seed=11)
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, _ = oracle.lut_tables(cfg)
    ref = oracle.forward(x.numpy(), vp.numpy(), vn.numpy(), ti, dmin, dmax, cfg["V_sat"])
    from isa.kernels.transformer_ffn.ekv_lut_triton import triton_lut_ekv_matmul

    out = triton_lut_ekv_matmul(x.to(cuda_device), vp.to(cuda_device), vn.to(cuda_device), cfg)
    assert errs(out, ref)[0] <= FWD_TOL


def test_gradient_subsets(cuda_device):
    """need_grad_x / need_grad_w alone give the same values as both together."""
    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(64, 72, 256, seed=5)
    _, gx_all, gp_all, gn_all = _dev_run(x, vp, vn, g, cfg, cuda_device)
    _, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, need_x=True, need_w=False)
    assert gp is None and gn is None
    assert torch.equal(gx, gx_all)
    _, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device, need_x=False, need_w=True)
    assert gx is None
    assert torch.equal(gp, gp_all) and torch.equal(gn, gn_all)


def test_bitwise_determinism(cuda_device):
    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(200, 192, 512, seed=9)
    a = _dev_run(x, vp, vn, g, cfg, cuda_device)
    b = _dev_run(x, vp, vn, g, cfg, cuda_device)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.mark.parametrize("ranked", [False, True])
def test_invariants_on_device(cuda_device, ranked):
    """vth_pos == vth_neg gives exactly zero Idiff, and dVth+ == -dVth- bitwise. dX is exactly
    zero where each cell forms L_D(+) - L_D(-) (the one-copy kernel); the ranked backward sums
    the + and - branches of an output in separate lanes and slots, so there dX vanishes to
    rounding: bounded by 1e-6 of the dX magnitude of the same inputs with distinct thresholds."""
    from isa.kernels.transformer_ffn import ops

    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(33, 50, 70, seed=2)
    prev = ops.ranked_backward(ranked)
    try:
        modes = {}
        out, gx, gp, gn = _dev_run(x, vp, vp.clone(), g, cfg, cuda_device, modes=modes)
        _, gx_ref, _, _ = _dev_run(x, vp, vn, g, cfg, cuda_device)
    finally:
        ops.ranked_backward(prev)
    # without the ranked backward at the initial thresholds' spread: the one-copy kernel
    assert modes["bwd"] == (2 if ranked else 0), modes
    assert torch.count_nonzero(out) == 0
    assert torch.equal(gp, -gn)
    if ranked:
        scale = float(gx_ref.abs().max())
        print(f"max |dX| {float(gx.abs().max()):.3e} of dX scale {scale:.3e}")
        assert float(gx.abs().max()) <= 1e-6 * scale
    else:
        assert torch.count_nonzero(gx) == 0


@pytest.mark.parametrize("M,K,O", [(70, 129, 300), (40, 203, 520), (1, 3000, 5), (96, 40, 768), (333, 768, 256)])
def test_ranked_matches_one_copy(cuda_device, M, K, O):
    """The ranked backward re-deals each input's branches to lanes in threshold rank but sums
    dVth+- from the same products in the same token order as the one-copy kernel: on the same
    plan (token splits) its dVth are bitwise those of the one-copy kernel (a dropped,
    repeated or mis-signed branch would show here), and its dX, summed in rank order, agrees
    to rounding. Both are checked against the oracle as well."""
    from isa.kernels.transformer_ffn import ops

    print(f"[case] ranked vs one copy M={M} K={K} O={O}", flush=True)
    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(M, K, O, seed=M + 3 * K)
    res = {}
    for ranked in (True, False):
        # without the ranked backward and without windowed copies: the one-copy kernel
        prev = ops.ranked_backward(ranked)
        prev_w = ops.window_copies(16 if ranked else 0)
        try:
            modes = {}
            res[ranked] = _dev_run(x, vp, vn, g, cfg, cuda_device, modes=modes)
        finally:
            ops.ranked_backward(prev)
            ops.window_copies(prev_w)
        assert modes["bwd"] == (2 if ranked else 0), (ranked, modes)
    (_, dx_r, gp_r, gn_r), (_, dx_1, gp_1, gn_1) = res[True], res[False]
    assert torch.equal(gp_r, gp_1) and torch.equal(gn_r, gn_1)
    e = errs(dx_r, dx_1.cpu().numpy())[0]
    print(f"dX ranked vs one copy {e:.2e}")
    assert e <= 1e-6
    _, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg)
    assert max(errs(dx_r, ref_dx)[0], errs(gp_r, ref_gp)[0], errs(gn_r, ref_gn)[0]) <= BWD_TOL


@pytest.mark.parametrize("max_copies", [3, 5, 8, 16, 32])
def test_windowed_window_copies(cuda_device, max_copies):
    """The forward's windowed table copies under each cap ISA_EKV_OPT_WINDOW_COPIES allows (the
    device takes as many as fit, up to the cap, and records their number): on ragged shapes
    whose coordinates reach a narrow window (mapped inputs, initial thresholds) the count is
    the cap; every case matches the oracle and the one-copy forward of the same inputs to
    rounding, and equal + and - thresholds still give exactly zero (the two signs' identical
    threshold sets get identical copy choices)."""
    from isa.approximations.delta_lut import get_packed_tables, lut_range
    from isa.kernels.transformer_ffn import ops

    cfg = flash_cfg(4096)
    dmin, dmax, n = lut_range(cfg)
    fwd, _ = get_packed_tables(cfg, cuda_device)
    # "narrow": inputs within a few hundredths of a volt of zero, as fc2's TIA outputs are
    cases = (((70, 129, 300), "narrow", "init"), ((5, 40, 1000), "narrow", "init"),
             ((64, 203, 520), "mapped", "init"), ((48, 200, 300), "mapped", "full"),
             ((33, 768, 256), "signed", "init"))
    prev = ops.window_copies()
    try:
        for (M, K, O), x_mode, vth_mode in cases:
            print(f"[case] windowed copies <= {max_copies}: M={M} K={K} O={O} {x_mode}/{vth_mode}", flush=True)
            x, vp, vn, g = make_inputs(M, K, O, seed=M + K + O, x_mode="signed" if x_mode == "narrow" else x_mode,
                                       vth_mode=vth_mode)
            if x_mode == "narrow":
                x = x * 0.01
            ref_out = oracle.forward(x.numpy(), vp.numpy(), vn.numpy(), oracle.lut_tables(cfg)[0], dmin, dmax,
                                     cfg["V_sat"], -4.0, 4.0)
            ops.window_copies(max_copies)
            modes = {}
            out, _, _, _ = _dev_run(x, vp, vn, g, cfg, cuda_device, modes=modes)
            xd, pd = x.to(cuda_device), vp.to(cuda_device)
            pf = ops.plan_info("forward", M, K, O, n)
            wsf = torch.empty(pf["workspace_bytes"], dtype=torch.uint8, device=cuda_device)
            zero = ops.lut_forward(xd, pd, pd.clone(), fwd, n, dmin, dmax, cfg["V_sat"], -4.0, 4.0, workspace=wsf)
            torch.cuda.synchronize()
            zmode = ops.copy_mode(wsf, pf)
            ops.window_copies(0)
            one, _, _, _ = _dev_run(x, vp, vn, g, cfg, cuda_device)
            e = errs(out, ref_out)[0]
            d = float((out - one).abs().max()) / max(float(one.abs().max()), 1e-30)
            print(modes, zmode, f"oracle {e:.2e}, vs one copy {d:.2e}")
            if x_mode == "narrow":  # a window of ~80 records: the cap
                assert modes["fwd"] == max_copies and zmode == max_copies, (modes, zmode)
            elif (x_mode, vth_mode) == ("mapped", "init"):  # ~1000-1400 records: fewer fit
                assert 3 <= modes["fwd"] <= max_copies, modes
            assert e <= FWD_TOL and d <= FWD_TOL
            assert torch.count_nonzero(zero) == 0
    finally:
        ops.window_copies(prev)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,O,x_mode", [(48, 200, 300, "signed"), (33, 203, 520, "signed"), (40, 129, 300, "mapped")])
def test_windowed_copies_wide_spread(cuda_device, M, K, O, x_mode):
    """Thresholds over [0, 5] V (1576 records: past the ranked backward's 420) against mapped
    inputs reach a ~2900-record window of the 4096-entry table: both directions hold three or
    more windowed copies. Inputs over [-4, 4] V reach ~4100 records: three copies fit neither
    the forward's 80 KB nor the backward's 3008-record halves, so both hold two (mode word 33;
    the backward's D halves a split table's length on). Every output and gradient matches the
    oracle and the one-copy kernels (window copies off) to rounding, with and without dVth."""
    from isa.kernels.transformer_ffn import ops

    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(M, K, O, seed=M * K, x_mode=x_mode, vth_mode="full")
    ref = oracle_all(x, vp, vn, g, cfg, -math.inf, math.inf)
    prev = ops.window_copies()
    try:
        modes, modes_x = {}, {}
        got = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf, modes=modes)
        got_x = _dev_run(x, vp, vn, g, cfg, cuda_device, need_w=False, out_min=-math.inf, out_max=math.inf,
                         modes=modes_x)
        ops.window_copies(0)
        one_modes = {}
        one = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf, modes=one_modes)
    finally:
        ops.window_copies(prev)
    e = [errs(got[i], ref[i])[0] for i in range(4)]
    d = [errs(got[i], one[i].detach().double().cpu().numpy())[0] for i in range(4)]
    ex = errs(got_x[1], ref[1])[0]
    print(modes, modes_x["bwd"], one_modes, [f"{v:.2e}" for v in e], [f"{v:.2e}" for v in d], f"{ex:.2e}")
    if x_mode == "signed":
        assert modes == {"fwd": 33, "bwd": 33} and modes_x["bwd"] == 33, (modes, modes_x)
    else:
        assert 3 <= modes["fwd"] <= 16 and 3 <= modes["bwd"] <= 16 and modes_x["bwd"] == modes["bwd"], (modes, modes_x)
    assert one_modes["fwd"] in (0, 1) and one_modes["bwd"] in (0, 1), one_modes
    assert e[0] <= FWD_TOL and max(e[1:]) <= BWD_TOL, e
    assert d[0] <= FWD_TOL and max(d[1:]) <= BWD_TOL, d
    assert ex <= BWD_TOL and got_x[2] is None and got_x[3] is None, ex


@pytest.mark.gpu
def _spread_inputs(M, K, O, spread_records, seed):
    """Mapped inputs and thresholds uniform over spread_records table records (4096 entries:
    315 records per volt) from 1 V."""
    x, _, _, g = make_inputs(M, K, O, seed=seed)
    gen = torch.Generator().manual_seed(seed + 1)
    span = spread_records * 13.0 / 4095.0  # volts
    vp = 1.0 + torch.rand(O, K, generator=gen) * span
    vn = 1.0 + torch.rand(O, K, generator=gen) * span
    return x, vp, vn, g


@pytest.mark.parametrize("spread_records,max_spread,greedy_min,expect", [
    (80, None, None, "ranked"), (380, None, None, "ranked"), (460, None, None, "copies"),
    (460, 4128, 100, "ranked"), (1500, 4128, 100, "ranked"), (1500, 4128, None, "ranked")])
def test_ranked_spread_limit(cuda_device, spread_records, max_spread, greedy_min, expect):
    """The ranked backward runs while the thresholds span at most ISA_EKV_OPT_RANK_MAX_SPREAD
    table records (default 420; raised here to take every spread whose window fits), dealt by
    rank, or past ISA_EKV_OPT_RANK_GREEDY_MIN records (off by default; 100 here) by the greedy
    bank-aware deal; past the limit the two-copy launch's windowed copies run. Every case
    matches the oracle."""
    from isa.kernels.transformer_ffn import ops

    cfg = flash_cfg(4096)
    M, K, O = 64, 96, 300
    x, vp, vn, g = _spread_inputs(M, K, O, spread_records, spread_records)
    ref = oracle_all(x, vp, vn, g, cfg, -math.inf, math.inf)
    modes = {}
    prev = ops.rank_max_spread(max_spread)
    prev_g = ops.rank_greedy_min(greedy_min)
    try:
        got = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf, modes=modes)
    finally:
        ops.rank_max_spread(prev)
        ops.rank_greedy_min(prev_g)
    e = [errs(got[i], ref[i])[0] for i in range(4)]
    print(spread_records, max_spread, greedy_min, modes, [f"{v:.2e}" for v in e])
    if expect == "ranked":
        assert modes["bwd"] == 2, modes
    else:
        assert 3 <= modes["bwd"] <= 16, modes
    assert e[0] <= FWD_TOL and max(e[1:]) <= BWD_TOL, e


@pytest.mark.parametrize("spread_records,M,K,O", [(135, 70, 129, 300), (460, 40, 203, 520), (1500, 96, 40, 768),
                                                  (1700, 333, 64, 256), (300, 1, 700, 5)])
def test_greedy_deal_matches_one_copy(cuda_device, spread_records, M, K, O):
    """The greedy bank-aware deal (spreads past ISA_EKV_OPT_RANK_GREEDY_MIN records) places every
    branch of an (input, output block) exactly once: a branch's dVth sum is the same products
    in the same token order wherever it is dealt, so the greedy deal's dVth+- are bitwise those
    of the rank deal on the same plan (with the greedy threshold raised past the spread; the
    rank deal is checked bitwise against the one-copy kernel in test_ranked_matches_one_copy):
    a dropped, repeated or mis-signed branch would show. dX, summed over an input's branches in
    another lane order, agrees to rounding, and both match the oracle."""
    from isa.kernels.transformer_ffn import ops

    print(f"[case] greedy deal spread {spread_records} M={M} K={K} O={O}", flush=True)
    cfg = flash_cfg(4096)
    x, vp, vn, g = _spread_inputs(M, K, O, spread_records, 7 * spread_records + M)
    res = {}
    for mode in ("greedy", "rank"):
        prev_g = ops.rank_greedy_min(100 if mode == "greedy" else 100000)
        prev = ops.rank_max_spread(4128)
        try:
            modes = {}
            res[mode] = _dev_run(x, vp, vn, g, cfg, cuda_device, out_min=-math.inf, out_max=math.inf, modes=modes)
        finally:
            ops.rank_greedy_min(prev_g)
            ops.rank_max_spread(prev)
        assert modes["bwd"] == 2, (mode, modes)
    (_, dx_g, gp_g, gn_g), (_, dx_r, gp_r, gn_r) = res["greedy"], res["rank"]
    assert torch.equal(gp_g, gp_r) and torch.equal(gn_g, gn_r)
    e = errs(dx_g, dx_r.cpu().numpy())[0]
    print(f"dX greedy vs rank deal {e:.2e}")
    assert e <= 1e-6
    _, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg, -math.inf, math.inf)
    assert max(errs(dx_g, ref_dx)[0], errs(gp_g, ref_gp)[0], errs(gn_g, ref_gn)[0]) <= BWD_TOL


def test_nan_semantics(cuda_device):
    """NaN x: r is NaN so its cells are NaN and the NaN row sum clamps to out_min (fminf/fmaxf);
    NaN vth reads table entry 0 like ekv_cuda.cu:19-21. Same rules as the oracle."""
    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(8, 16, 256, seed=4)
    x[3, 5] = float("nan")
    vp[7, 2] = float("nan")
    ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg)
    out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device)
    o = out.cpu().numpy()
    assert np.array_equal(np.isnan(o), np.isnan(ref_out))
    fin = np.isfinite(ref_out)
    assert np.allclose(o[fin], ref_out[fin], rtol=1e-4, atol=1e-4 * np.abs(ref_out[fin]).max())
    for a, r in ((gx, ref_dx), (gp, ref_gp), (gn, ref_gn)):
        a = a.cpu().numpy()
        assert np.array_equal(np.isnan(a), np.isnan(r))


def test_lut_build_matches_oracle(cuda_device):
    from isa.approximations.delta_lut import get_ekv_lut_tables

    for size in (257, 4096, 8192):
        cfg = flash_cfg(size)
        ti_d, td_d = get_ekv_lut_tables(cfg, cuda_device)
        ti, td = oracle.lut_tables(cfg)
        a_i, a_d = ti_d.cpu().numpy(), td_d.cpu().numpy()
        # both round the same fp64 value once; allow 1 ulp for libm differences
        assert np.all(np.abs(a_i.view(np.int32).astype(np.int64) - ti.view(np.int32)) <= 1)
        assert np.all(np.abs(a_d.view(np.int32).astype(np.int64) - td.view(np.int32)) <= 1)


@pytest.mark.parametrize("x_mode,M,K,O", [("mapped", 40, 64, 256), ("fc2init", 48, 1024, 256),
                                           ("fc2init", 64, 3072, 768)])
def test_bf16_table_mode(cuda_device, x_mode, M, K, O):
    """LUT_DTYPE=bfloat16 gives the reference's bf16 tables byte for byte (the fp32 torch
    construction of delta_lut.py:25-34 cast at :35) and the kernels compute with the widened
    values (cuda_backend.py:68-69), checked against the oracle fed those same tables. The
    fc2init cases (inputs within 0.3 V of zero, the initial thresholds: fc2 at
    initialisation) sit where the reference's fp32 construction loses the derivative table's
    subthreshold end: an fp64-accurate table rounded to bf16 is 4.6e-3 (dX) and 2.6e-3
    (dVth) away from the reference's there, past the gates."""
    from isa.approximations.delta_lut import get_ekv_lut_tables

    print(f"[case] bf16 tables {x_mode} M={M} K={K} O={O}", flush=True)
    cfg = flash_cfg(4096, LUT_DTYPE="bfloat16")
    ti_d, td_d = get_ekv_lut_tables(cfg, cuda_device)
    assert ti_d.dtype == torch.bfloat16 and td_d.dtype == torch.bfloat16
    _, _, ref_i, ref_d = oracle.reference_lut_tables(cfg)
    assert torch.equal(ti_d.cpu().view(torch.int16), ref_i.view(torch.int16))
    assert torch.equal(td_d.cpu().view(torch.int16), ref_d.view(torch.int16))
    x, vp, vn, g = make_inputs(M, K, O, seed=8, x_mode=x_mode)
    ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg)
    out, gx, gp, gn = _dev_run(x, vp, vn, g, cfg, cuda_device)
    e = [errs(out, ref_out)[0], errs(gx, ref_dx)[0], errs(gp, ref_gp)[0], errs(gn, ref_gn)[0]]
    print("bf16 tables:", [f"{v:.2e}" for v in e])
    assert e[0] <= FWD_TOL
    assert max(e[1:]) <= BWD_TOL


def test_lds_gather_probe(cuda_device):
    """The LDS roofline's probe runs and orders as bank conflicts predict: gathers whose
    lanes spread over a wide window cost at least as much as a 32-record window (one
    8-byte record per bank pair, conflict-free) and 16-byte records more than 8-byte ones."""
    from isa.kernels.transformer_ffn import ops

    print("[case] lds gather probe", flush=True)
    narrow = ops.probe_lds_gather(32, 8, iterations=256, device=cuda_device)
    wide = ops.probe_lds_gather(1024, 8, iterations=256, device=cuda_device)
    wide16 = ops.probe_lds_gather(1024, 16, iterations=256, device=cuda_device)
    assert 0.0 < narrow < 1e3
    assert wide >= 0.95 * narrow
    assert wide16 >= 0.95 * wide


def test_valu_issue_probe(cuda_device):
    """The measured VALU ceiling's replay runs every mix and reports rates a CU can issue:
    above a quarter of one wave-instruction per CU-cycle and below the four SIMDs' four, with
    a shader clock in the board's range."""
    from isa.kernels.transformer_ffn import ops

    for mix in ("fma", "forward", "ranked_backward", "forward_int_address"):
        print(f"[case] valu issue probe {mix}", flush=True)
        r = ops.probe_valu_issue(mix, iterations=256, device=cuda_device)
        print(f"  {r}", flush=True)
        assert 0.25 < r["instr_per_cu_cycle"] < 4.0, r
        assert 0.5 < r["ghz"] < 3.5, r
        # every CU held two blocks, and no CU issued faster than its busy interval allows
        assert r["blocks_per_cu"] == 2.0, r
        assert r["instr_per_cu_cycle_launch"] <= 1.05 * r["instr_per_cu_cycle"], r


def test_kernel_clock_sampling(cuda_device):
    """Under KernelTimer every block of the LUT main kernels adds its shader-clock span: a
    ranked backward and a forward large enough for the copy machinery report their blocks and
    a clock in the board's range, and a call outside the timer adds nothing."""
    from isa.kernels.transformer_ffn import _hip

    cfg = flash_cfg(4096)
    x, vp, vn, g = make_inputs(512, 256, 2048, seed=21)
    print("[case] kernel clock sampling", flush=True)
    with _hip.KernelTimer() as kt:
        modes = {}
        _dev_run(x, vp, vn, g, cfg, cuda_device, modes=modes)
    print(f"  modes {modes} clocks {kt.clocks}", flush=True)
    assert modes["bwd"] == 2
    assert kt.clocks["bwd_ranked_kernel"]["blocks"] > 0 and kt.clocks["fwd_kernel"]["blocks"] > 0
    for name in ("bwd_ranked_kernel", "fwd_kernel"):
        assert 0.5 < kt.clocks[name]["ghz"] < 3.5, (name, kt.clocks[name])
    _dev_run(x, vp, vn, g, cfg, cuda_device)
    with _hip.KernelTimer() as kt2:
        pass
    assert all(c["blocks"] == 0 for c in kt2.clocks.values()), kt2.clocks
