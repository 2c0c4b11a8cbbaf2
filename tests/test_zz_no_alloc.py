"""isa_ekv_forward_noalloc (the forward without a workspace argument, for callers that
cannot allocate) against isa_ekv_forward, through the C ABI: the same kernels on the same
inputs, so outputs must be bitwise equal. Two calls in a row, the second smaller than the
first (the scratch array keeps the first call's contents), then calls in the windowed
table-copy regimes, the headline fc1 forward, and the size limit."""

from __future__ import annotations

import pytest
import torch

from tests.helpers import flash_cfg, make_inputs

pytestmark = pytest.mark.gpu


def _both(x, vp, vn, cfg, dev):
    """(workspace forward, no-allocation forward, the table-copy mode word of the workspace
    call) on the same inputs."""
    from isa.approximations.delta_lut import get_packed_tables, lut_range
    from isa.kernels.transformer_ffn import ops

    dmin, dmax, n = lut_range(cfg)
    fwd, _ = get_packed_tables(cfg, dev)
    xd, pd, nd = (t.to(dev).contiguous() for t in (x, vp, vn))
    M, K = x.shape
    plan = ops.plan_info("forward", M, K, vp.shape[0], n)
    ws = torch.empty(plan["workspace_bytes"], dtype=torch.uint8, device=dev)
    ref = ops.lut_forward(xd, pd, nd, fwd, n, dmin, dmax, cfg["V_sat"], -4.0, 4.0, workspace=ws)
    out = torch.full_like(ref, float("nan"))
    ops.lut_forward_noalloc(xd, pd, nd, fwd, n, dmin, dmax, cfg["V_sat"], -4.0, 4.0, out)
    torch.cuda.synchronize()
    return ref, out, ops.copy_mode(ws, plan)


def test_noalloc_forward_matches_workspace_forward(cuda_device):
    cfg = flash_cfg(4096)
    for M, K, O in ((300, 203, 500), (37, 64, 130)):  # second call smaller; K % 8 != 0 first
        print(f"[case] noalloc forward M={M} K={K} O={O}", flush=True)
        x, vp, vn, _ = make_inputs(M, K, O, seed=M + K + O)
        ref, out, _ = _both(x, vp, vn, cfg, cuda_device)
        assert torch.equal(out, ref)
        assert torch.count_nonzero(ref) > 0


def test_noalloc_forward_table_copies(cuda_device):
    """The windowed-copy forward, whose mode word, copy-assignment passes and reassigned
    threshold records live in the scratch array. These shapes are far below the library's
    copy threshold (ISA_EKV_OPT_COPY_MIN_CELLS), so the test lowers it to zero, as large
    calls run, and checks the mode the workspace call took: windowed copies (about three of
    the 8192-entry table's ~2800-record window of mapped inputs, up to 32 of the 4096-entry
    table's narrow window of fc2-like inputs)."""
    from isa.kernels.transformer_ffn import ops

    prev = ops.copy_min_cells(0)
    try:
        for size, x_mode in ((8192, "mapped"), (4096, "fc2init")):
            cfg = flash_cfg(size)
            for M, K, O in ((256, 400, 600), (64, 203, 300)):
                print(f"[case] noalloc forward {size} entries {x_mode} M={M} K={K} O={O}", flush=True)
                x, vp, vn, _ = make_inputs(M, K, O, seed=7 * M + K, x_mode=x_mode)
                ref, out, mode = _both(x, vp, vn, cfg, cuda_device)
                print(f"  mode {mode}", flush=True)
                assert mode is not None and 3 <= mode <= 33, mode
                assert torch.equal(out, ref)
    finally:
        ops.copy_min_cells(prev)


def test_noalloc_forward_headline_fc1(cuda_device):
    """The GPT-L fc1 forward (8192 x 768 -> 3072, 66 MiB of scratch): windowed table copies
    at the library's default options, as the headline runs it."""
    from isa.kernels.transformer_ffn import _hip, ops

    cfg = flash_cfg(4096)
    M, K, O = 8192, 768, 3072
    print(f"[case] noalloc forward headline fc1 M={M} K={K} O={O}", flush=True)
    assert ops.plan_info("forward", M, K, O, 4096)["workspace_bytes"] <= _hip.NOALLOC_MAX_BYTES
    x, vp, vn, _ = make_inputs(M, K, O, seed=11, x_mode="mapped")
    ref, out, mode = _both(x, vp, vn, cfg, cuda_device)
    print(f"  mode {mode}", flush=True)
    assert mode is not None and 3 <= mode <= 33, mode
    assert torch.equal(out, ref)


def test_noalloc_forward_rejects_oversized_shapes(cuda_device):
    from isa.approximations.delta_lut import get_packed_tables, lut_range
    from isa.kernels.transformer_ffn import _hip, ops

    cfg = flash_cfg(4096)
    M, K, O = 8192, 3072, 768  # headline fc2: 306 MiB of workspace (token records, K-split planes)
    assert ops.plan_info("forward", M, K, O, 4096)["workspace_bytes"] > _hip.NOALLOC_MAX_BYTES
    dmin, dmax, n = lut_range(cfg)
    fwd, _ = get_packed_tables(cfg, cuda_device)
    x = torch.zeros(M, K, device=cuda_device)
    w = torch.zeros(O, K, device=cuda_device)
    out = torch.full((M, O), 7.0, device=cuda_device)
    with pytest.raises(RuntimeError, match="maximum"):
        ops.lut_forward_noalloc(x, w, w, fwd, n, dmin, dmax, cfg["V_sat"], -4.0, 4.0, out)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was enqueued (a forward would have written zeros)
