"""The C ABI library loads on a host without a GPU and exports what include/isa_ekv.h
declares; argument validation that happens before any HIP call returns ISA_EKV_EINVAL
with a message (CPU only: no kernel is launched here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from isa.kernels.transformer_ffn import _hip

HEADER = Path(__file__).resolve().parents[1] / "include" / "isa_ekv.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(isa_ekv_\w+)\s*\(", text)))


def test_header_lists_the_python_exports():
    assert declared_functions() == sorted(_hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    raw = ctypes.CDLL(str(_hip.LIB_PATH))
    for name in declared_functions():
        assert hasattr(raw, name), name


def test_version_and_sizes():
    lib = _hip.load()
    assert lib.isa_ekv_abi_version() == _hip.ABI_VERSION
    pad = lib.isa_ekv_lut_pad()
    assert pad >= 2
    assert lib.isa_ekv_lut_bytes(4096, _hip.LUT_PLAIN_F32) == 4096 * 8
    assert lib.isa_ekv_lut_bytes(4096, _hip.LUT_PLAIN_BF16) == 4096 * 4
    assert lib.isa_ekv_lut_bytes(4096, _hip.LUT_FWD) == (4096 + 2 * pad) * 8
    assert lib.isa_ekv_lut_bytes(4096, _hip.LUT_BWD) == (4096 + 2 * pad) * 16
    assert lib.isa_ekv_lut_bytes(0, _hip.LUT_FWD) == 0
    assert lib.isa_ekv_lut_bytes(16, 99) == 0


def test_workspace_queries():
    lib = _hip.load()
    f = lib.isa_ekv_forward_workspace(8192, 768, 3072)
    # token records (8 B) and transposed thresholds (8 B) at least
    assert f >= 8192 * 768 * 8 + 768 * 3072 * 8
    b_all = lib.isa_ekv_backward_workspace(8192, 768, 3072, 4096, 1, 1)
    b_x = lib.isa_ekv_backward_workspace(8192, 768, 3072, 4096, 1, 0)
    b_w = lib.isa_ekv_backward_workspace(8192, 768, 3072, 4096, 0, 1)
    assert b_all > b_x and b_all > b_w
    assert lib.isa_ekv_forward_workspace(-1, 2, 3) == 0
    assert lib.isa_ekv_backward_workspace(1, 2, 3, 0, 1, 1) == 0


def _err(lib) -> str:
    return lib.isa_ekv_last_error().decode()


def test_lds_probe_rejects_bad_arguments_before_launch():
    lib = _hip.load()
    fake = ctypes.c_void_p(16)
    assert lib.isa_ekv_probe_lds_gather(64, 12, 1, fake, 1 << 20, None, None, None, None) == -1 and "record_bytes" in _err(lib)
    assert lib.isa_ekv_probe_lds_gather(0, 8, 1, fake, 1 << 20, None, None, None, None) == -1 and "window_records" in _err(lib)
    assert lib.isa_ekv_probe_lds_gather(4097, 16, 1, fake, 1 << 20, None, None, None, None) == -1 and "[1, 4096]" in _err(lib)
    assert lib.isa_ekv_probe_lds_gather(64, 8, 0, fake, 1 << 20, None, None, None, None) == -1 and "iterations" in _err(lib)


def test_forward_rejects_bad_arguments_before_launch():
    lib = _hip.load()
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    args = dict(M=4, K=4, O=4, n=4096, dmin=-9.0, dmax=4.0, vsat=8.26)

    def call(**over):
        a = dict(args, **over)
        return lib.isa_ekv_forward(fake, fake, fake, fake, a["M"], a["K"], a["O"], a["n"], a["dmin"], a["dmax"],
                                   a["vsat"], -4.0, 4.0, fake, fake, 0, None)

    assert call(M=-1) == -1 and "negative shape" in _err(lib)
    assert call(n=0) == -1 and "LUT_DELTA_SIZE" in _err(lib)
    assert call(n=(1 << 22) + 1) == -1 and "4194304" in _err(lib)
    assert call(dmax=-10.0) == -1 and "delta_max > delta_min" in _err(lib)
    assert call(vsat=0.0) == -1 and "V_sat" in _err(lib)
    assert call() == -1 and "workspace too small" in _err(lib)
    # empty outputs are a no-op
    assert call(M=0) == 0 and call(O=0) == 0


def test_backward_rejects_bad_arguments_before_launch():
    lib = _hip.load()
    fake = ctypes.c_void_p(16)

    def call(n=4096, gx=fake, gp=fake, gn=fake, ws_bytes=0):
        return lib.isa_ekv_backward(fake, fake, fake, fake, fake, 8, 8, 8, n, -9.0, 4.0, 8.26, gx, gp, gn,
                                    fake, ws_bytes, None)

    assert call(n=(1 << 22) + 1) == -1 and "4194304" in _err(lib)
    assert call(gp=None) == -1 and "both" in _err(lib)
    assert call() == -1 and "workspace too small" in _err(lib)
    assert call(gx=None, gp=None, gn=None) == 0  # nothing requested


def test_exact_entry_points_reject_bad_arguments_before_launch():
    lib = _hip.load()
    fake = ctypes.c_void_p(16)
    good = (ctypes.c_double * 4)(4.136, 0.0259, 7.5875e-7, 0.1)

    def fwd(params=good, M=4, vsat=8.26, ws_bytes=0):
        return lib.isa_ekv_exact_forward(fake, fake, fake, M, 4, 4, params, vsat, fake, fake, ws_bytes, None)

    assert fwd(params=None) == -1 and "params" in _err(lib)
    assert fwd(params=(ctypes.c_double * 4)(0.0, 0.0259, 1.0, 0.1)) == -1 and "U_T" in _err(lib)
    assert fwd(params=(ctypes.c_double * 4)(4.1, 0.0259, float("nan"), 0.1)) == -1 and "I_S" in _err(lib)
    assert fwd(vsat=0.0) == -1 and "V_sat" in _err(lib)
    assert fwd(M=-3) == -1 and "negative shape" in _err(lib)
    assert fwd() == -1 and "workspace too small" in _err(lib)
    assert fwd(M=0) == 0

    def bwd(gx=fake, gp=fake, gn=fake):
        return lib.isa_ekv_exact_backward(fake, fake, fake, fake, 8, 8, 8, good, 8.26, gx, gp, gn, fake, 0, None)

    assert bwd(gn=None) == -1 and "both" in _err(lib)
    assert bwd() == -1 and "workspace too small" in _err(lib)
    assert bwd(gx=None, gp=None, gn=None) == 0
    # the exact path keeps no table: its workspace adds the general-loop records instead
    assert lib.isa_ekv_exact_forward_workspace(64, 96, 256) > lib.isa_ekv_forward_workspace(64, 96, 256)
    assert lib.isa_ekv_exact_backward_workspace(64, 96, 256, 1, 1) > 0
    assert lib.isa_ekv_exact_backward_workspace(-1, 96, 256, 1, 1) == 0


def test_layer_entry_points_reject_bad_glue_before_launch():
    lib = _hip.load()
    fake = ctypes.c_void_p(16)

    def fwd(glue):
        return lib.isa_ekv_layer_forward(fake, fake, fake, fake, 4, 4, 4, 4096, -9.0, 4.0, 8.26, -4.0, 4.0,
                                         glue, fake, fake, fake, 0, None)

    assert fwd(None) == -1 and "glue is null" in _err(lib)
    g = _hip.Glue()
    g.adc_scale = 16
    assert fwd(ctypes.byref(g)) == -1 and "adc_shift" in _err(lib)
    g = _hip.Glue()
    g.r_tia, g.y_lo, g.y_hi = 16, 4.0, -4.0
    assert fwd(ctypes.byref(g)) == -1 and "y_hi" in _err(lib)
    g = _hip.Glue()
    g.r_log_scale, g.r_log_lo, g.r_log_hi = 16, -2.0, 2.0
    assert fwd(ctypes.byref(g)) == -1 and "needs r_tia" in _err(lib)
    g.r_tia, g.y_lo, g.y_hi = 16, -4.0, 4.0
    g.r_log_lo, g.r_log_hi = 2.0, -2.0
    assert fwd(ctypes.byref(g)) == -1 and "r_log_hi" in _err(lib)
    g = _hip.Glue()
    assert fwd(ctypes.byref(g)) == -1 and "workspace too small" in _err(lib)

    def bwd(glue, grads, gx=fake, idiff=fake):
        return lib.isa_ekv_layer_backward(fake, fake, fake, fake, idiff, fake, 8, 8, 8, 4096, -9.0, 4.0, 8.26,
                                          glue, gx, fake, fake, grads, fake, 0, None)

    g = _hip.Glue()
    gg = _hip.GlueGrads()
    gg.r_tia = 16
    assert bwd(ctypes.byref(g), ctypes.byref(gg)) == -1 and "r_tia gradient without r_tia" in _err(lib)
    g.r_tia, g.y_lo, g.y_hi = 16, -4.0, 4.0
    gg = _hip.GlueGrads()
    gg.r_log_scale = 16
    assert bwd(ctypes.byref(g), ctypes.byref(gg)) == -1 and "r_log_scale gradient without" in _err(lib)
    g = _hip.Glue()
    g.in_affine, g.in_lo, g.in_hi = 16, 0.0, 4.0
    gg = _hip.GlueGrads()
    gg.in_affine = 16
    assert bwd(ctypes.byref(g), ctypes.byref(gg), gx=None) == -1 and "needs grad_x" in _err(lib)
    assert bwd(ctypes.byref(g), ctypes.byref(gg), idiff=None) == -1 and "idiff is null" in _err(lib)
    assert bwd(ctypes.byref(g), ctypes.byref(gg)) == -1 and "workspace too small" in _err(lib)
    # the layer backward needs room for G_eff and the glue partials beyond the plain backward's
    assert lib.isa_ekv_layer_backward_workspace(64, 96, 256, 4096, 1, 1) > \
        lib.isa_ekv_backward_workspace(64, 96, 256, 4096, 1, 1)


def test_measured_entry_points_reject_bad_codebooks_before_launch():
    lib = _hip.load()
    fake = ctypes.c_void_p(16)

    def fwd(cb, r=fake, ids=fake):
        return lib.isa_ekv_measured_forward(fake, ids, None, 4, 4, 4, cb, 1.0, r, -4.0, 4.0, fake, fake, fake, 0,
                                            None)

    assert fwd(None) == -1 and "codebook is null" in _err(lib)
    cb = _hip.Codebook()
    assert fwd(ctypes.byref(cb)) == -1 and "n_seg" in _err(lib)
    cb.n_seg, cb.n_rows = 60, 24
    assert fwd(ctypes.byref(cb)) == -1 and "slopes" in _err(lib)
    cb.slopes = cb.intercepts = 16
    cb.seg_mode = 7
    assert fwd(ctypes.byref(cb)) == -1 and "segment mode" in _err(lib)
    cb.seg_mode = _hip.SEG_SEARCH
    assert fwd(ctypes.byref(cb)) == -1 and "vg" in _err(lib)
    cb.seg_mode, cb.lookup_min, cb.lookup_max = _hip.SEG_UNIFORM, 0.0, 4.0
    assert fwd(ctypes.byref(cb), ids=None) == -1 and "ids_a" in _err(lib)
    assert fwd(ctypes.byref(cb), r=None) == -1 and "r_tia" in _err(lib)
    assert fwd(ctypes.byref(cb)) == -1 and "workspace too small" in _err(lib)
    assert lib.isa_ekv_measured_forward_workspace(8, 8, 8, 60, 24) > lib.isa_ekv_forward_workspace(8, 8, 8)
    assert lib.isa_ekv_measured_backward_workspace(8, 8, 8, 0, 24) == 0
    rc = lib.isa_ekv_measured_backward(fake, fake, None, 4, 4, 4, ctypes.byref(cb), 1.0, fake, fake, fake, -4.0, 4.0,
                                       None, fake, 0, None)
    assert rc == 0  # no grad_x requested: nothing to do


def test_lut_build_and_pack_reject_bad_arguments():
    lib = _hip.load()
    params = (ctypes.c_double * 4)(4.136, 0.0259, 7.5875e-7, 0.1)
    fake = ctypes.c_void_p(16)
    assert lib.isa_ekv_lut_build(None, -9.0, 4.0, 16, _hip.LUT_FWD, fake, None) == -1
    assert lib.isa_ekv_lut_build(params, -9.0, 4.0, 16, 7, fake, None) == -1 and "layout" in _err(lib)
    assert lib.isa_ekv_lut_build(params, 4.0, 4.0, 16, _hip.LUT_FWD, fake, None) == -1
    bad = (ctypes.c_double * 4)(0.0, 0.0259, 7.5875e-7, 0.1)
    assert lib.isa_ekv_lut_build(bad, -9.0, 4.0, 16, _hip.LUT_FWD, fake, None) == -1
    assert lib.isa_ekv_lut_pack(fake, fake, 16, 0, _hip.LUT_PLAIN_F32, fake, None) == -1
    assert lib.isa_ekv_lut_pack(fake, None, 16, 0, _hip.LUT_BWD, fake, None) == -1
    assert lib.isa_ekv_lut_pack(fake, fake, 16, 5, _hip.LUT_FWD, fake, None) == -1


def test_profiler_round_trip_without_launches():
    with _hip.KernelTimer() as kt:
        pass
    assert kt.fwd_launches == 0 and kt.bwd_launches == 0 and kt.fwd_ms == 0.0


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_hip, "_lib", None)
    with pytest.raises(_hip.HipExtensionError, match="not found"):
        _hip.load(tmp_path / "absent.so")


def test_plan_info_reports_the_call_plans():
    """isa_ekv_plan_info (host-side planning only): workspace sizes agree with the workspace
    queries, and the table-copy mode word exists exactly where a second copy can be used."""
    from isa.kernels.transformer_ffn import ops

    lib = _hip.load()
    f = ops.plan_info("forward", 8192, 768, 3072, 4096)
    assert 0 < f["workspace_bytes"] <= lib.isa_ekv_forward_workspace(8192, 768, 3072)
    assert f["mode_offset"] >= 0 and f["mode_offset"] % 4 == 0
    assert f["splits"] == 1 and f["waves_per_block"] == 8
    b = ops.plan_info("backward", 8192, 768, 3072, 4096)
    assert b["workspace_bytes"] == lib.isa_ekv_backward_workspace(8192, 768, 3072, 4096, 1, 1)
    assert b["mode_offset"] >= 0 and b["splits"] >= 1 and b["waves_per_block"] == 16
    lb = ops.plan_info("layer_backward", 8192, 3072, 768, 4096)
    assert lb["workspace_bytes"] == lib.isa_ekv_layer_backward_workspace(8192, 3072, 768, 4096, 1, 1)
    # fc2 of the headline (O = 768, three output blocks) splits K to fill the chip
    assert ops.plan_info("forward", 8192, 3072, 768, 4096)["splits"] > 1
    # 8192 entries, 768 inputs per wave: both copies in one 16-wave block per CU
    f8 = ops.plan_info("forward", 8192, 768, 3072, 8192)
    assert f8["waves_per_block"] == 16 and f8["mode_offset"] >= 0
    # 16384 entries: one LDS copy in the forward (whose allocation may hold windowed copies
    # of a narrow enough coordinate window: a mode word), two half-table passes in the
    # backward (no mode word)
    f16 = ops.plan_info("forward", 8192, 768, 3072, 16384)
    assert f16["mode_offset"] >= 0 and f16["lds_bytes"] == (16384 + 2 * 16) * 8
    assert ops.plan_info("backward", 8192, 768, 3072, 16384)["mode_offset"] == -1
    # without windowed copies (ISA_EKV_OPT_WINDOW_COPIES < 4) the 16384-entry forward has no mode word
    prev = ops.window_copies(0)
    try:
        assert ops.plan_info("forward", 8192, 768, 3072, 16384)["mode_offset"] == -1
        assert ops.window_copies() == 0
    finally:
        ops.window_copies(prev)
    assert prev == 32
    # a dVth-only backward runs no copy pair
    assert ops.plan_info("backward", 512, 64, 256, 4096, need_grad_x=False)["mode_offset"] == -1
    info = (ctypes.c_int64 * 7)()
    assert lib.isa_ekv_plan_info(9, 1, 1, 1, 4096, 1, 1, info, 7) == -1 and "plan kind" in _err(lib)
    assert lib.isa_ekv_plan_info(0, 1, 1, 1, 0, 1, 1, info, 7) == -1 and "LUT_DELTA_SIZE" in _err(lib)


def test_small_calls_plan_one_table_copy_and_one_round():
    """Calls below ISA_EKV_OPT_COPY_MIN_CELLS (default 2^28 cells) plan no second table copy;
    isa_ekv_set_option moves the threshold. Small plans keep to one round of blocks."""
    from isa.kernels.transformer_ffn import ops

    lib = _hip.load()
    prev = ops.copy_min_cells()
    assert prev == 1 << 28
    shape = (520, 192, 768, 4096)  # the ViT-S up-projection: 7.7e7 cells
    assert ops.plan_info("forward", *shape)["mode_offset"] == -1
    assert ops.plan_info("layer_backward", *shape)["mode_offset"] == -1
    try:
        assert ops.copy_min_cells(0) == 1 << 28
        assert ops.plan_info("forward", *shape)["mode_offset"] >= 0
        assert ops.plan_info("backward", *shape)["mode_offset"] >= 0
    finally:
        ops.copy_min_cells(prev)
    assert ops.copy_min_cells() == prev
    for kind in ("forward", "backward", "layer_backward"):
        for m, k, o in ((520, 192, 768), (520, 768, 192), (64, 200, 300)):
            plan = ops.plan_info(kind, m, k, o, 4096)
            per_cu = 2 if plan["waves_per_block"] * 64 * 2 <= 2048 else 1
            assert plan["blocks"] <= per_cu * 256, (kind, m, k, o, plan)
    assert lib.isa_ekv_set_option(7, 0, None) == -1 and "option" in _err(lib)

