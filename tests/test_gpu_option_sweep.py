"""Seeded random sweep of the LUT forward and backward against the CPU oracle across the
library's planning options and table sizes: the copy threshold (ISA_EKV_OPT_COPY_MIN_CELLS
at its default or 0, so small calls take the copy modes), the ranked backward on or off, its
spread limit (420 or 4128 records) and greedy-deal threshold (never, past 100 records, always),
the windowed-copy cap (0, 3, 7, 16, 32), tables of 257 to 20000 entries (odd sizes, the
two-pass and global-memory backwards), every input and threshold range of the helpers,
gradient subsets and the output clamp on or off. Each case also runs twice and must repeat
bitwise. Gates as in test_gpu_parity.py: forward <= 1e-4, dX and dVth+- <= 1e-3 norm-wise."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from tests.helpers import errs, flash_cfg, make_inputs, oracle_all

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-4
BWD_TOL = 1e-3


@pytest.fixture
def restore_options():
    from isa.kernels.transformer_ffn import ops

    saved = (ops.copy_min_cells(), ops.ranked_backward(), ops.window_copies(), ops.rank_max_spread(),
             ops.rank_greedy_min())
    yield ops
    ops.copy_min_cells(saved[0])
    ops.ranked_backward(saved[1])
    ops.window_copies(saved[2])
    ops.rank_max_spread(saved[3])
    ops.rank_greedy_min(saved[4])


@pytest.mark.parametrize("seed", [20261202, 20261203])
def test_option_and_table_size_sweep(cuda_device, restore_options, seed):
    from isa.approximations.delta_lut import get_packed_tables, lut_range

    ops = restore_options
    default_min_cells = ops.copy_min_cells()
    rng = np.random.default_rng(seed)
    for case in range(40):
        size = int(rng.choice([257, 999, 2048, 4096, 8192, 12000, 16384, 20000]))
        x_mode = str(rng.choice(["mapped", "signed", "fc2init", "wide"]))
        vth_mode = str(rng.choice(["init", "full", "wide"]))
        cap = 1e7 if size <= 16384 else 2e6
        while True:
            M, K, O = int(rng.integers(1, 600)), int(rng.integers(1, 800)), int(rng.integers(1, 1000))
            if M * K * O <= cap:
                break
        min_cells = int(rng.choice([default_min_cells, 0]))
        ranked = bool(rng.integers(0, 2))
        copies = int(rng.choice([32, 16, 7, 3, 0]))
        max_spread = int(rng.choice([420, 4128]))
        greedy_min = int(rng.choice([4128, 100, 0]))
        need_x, need_w = [(True, True), (True, False), (False, True)][int(rng.integers(0, 3))]
        lim = float(rng.choice([4.0, math.inf]))
        print(f"[case] sweep {seed}/{case}: {size} entries M={M} K={K} O={O} {x_mode}/{vth_mode} "
              f"min_cells={min_cells} ranked={ranked} copies={copies} max_spread={max_spread} "
              f"greedy_min={greedy_min} need_x={need_x} need_w={need_w} clamp={lim}", flush=True)
        ops.copy_min_cells(min_cells)
        ops.ranked_backward(ranked)
        ops.window_copies(copies)
        ops.rank_max_spread(max_spread)
        ops.rank_greedy_min(greedy_min)
        cfg = flash_cfg(size)
        x, vp, vn, g = make_inputs(M, K, O, seed=seed % 1000 * 100 + case, x_mode=x_mode, vth_mode=vth_mode)
        dmin, dmax, n = lut_range(cfg)
        fwd, bwd = get_packed_tables(cfg, cuda_device)
        xd, pd, nd, gd = (t.to(cuda_device) for t in (x, vp, vn, g))

        def run():
            out = ops.lut_forward(xd, pd, nd, fwd, n, dmin, dmax, cfg["V_sat"], -lim, lim)
            grads = ops.lut_backward(xd, pd, nd, gd, bwd, n, dmin, dmax, cfg["V_sat"], need_x, need_w)
            torch.cuda.synchronize()
            return (out, *grads)

        first, again = run(), run()
        for a, b in zip(first, again):
            assert (a is None and b is None) or torch.equal(a, b)
        ref_out, ref_dx, ref_gp, ref_gn = oracle_all(x, vp, vn, g, cfg, -lim, lim)
        e = [errs(first[0], ref_out)[0]]
        e.append(errs(first[1], ref_dx)[0] if need_x else 0.0)
        e += [errs(first[2], ref_gp)[0], errs(first[3], ref_gn)[0]] if need_w else [0.0, 0.0]
        print("  ", [f"{v:.2e}" for v in e], flush=True)
        assert e[0] <= FWD_TOL and max(e[1:]) <= BWD_TOL, e
