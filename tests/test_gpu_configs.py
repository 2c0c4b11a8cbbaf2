"""Parity at the BASELINE configurations through the path the benchmark times.

configs[1] Physical ViT-M FFN (PhysicalFFN 256 -> 1024 -> 256, X [128, 65, 256]) with the
4096-entry table and the vision default of 8192 entries; configs[2] Hybrid GPT-M FFN
(HybridFFN 384 -> 1536 with the digital Linear 1536 -> 384, X [16, 1024, 384]); configs[3]
the headline Physical GPT-L FFN (PhysicalFFN 768 -> 3072 -> 768, X [8, 1024, 768]). Each
runs the modules as bench.py does (fused layer glue, FusedCIMLayerFn, isa_ekv_layer_forward /
_backward) with N(0, 1) inputs and upstream gradient, and is checked layer by layer: a spy
around the two library calls captures what each layer received and produced on the GPU
(idiff, the layer output, the upstream gradient), and every layer is compared with the CPU
oracle on exact sub-problems fed with the GPU's own inputs (cim.py:217-280 composed with
ekv_lut_triton.py:52-61 and ekv_cuda.cu:224-250, :324-339):
  forward rows and dX rows depend only on their token (sampled rows); dVth columns only on
  their output, summed over every token (sampled columns); fc1's output after the TIA gain
  and clamp is fc2's input, and fc2's dX, masked by the clamp, is fc1's upstream gradient.
The glue (TIA gain and clamp, ADC affine, input mapping) is checked elementwise from the
GPU's own idiff, and the glue parameters' gradients against float64 sums of GPU
intermediates. The spy also reads each launch's table-copy mode word, so the regime the
bench runs is the regime tested. A second identical step must be bitwise equal.

Gates (norm-wise, against the fp32-table oracle): forward <= 1e-4, dX and dVth+- <= 1e-3.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import errs, flash_cfg, oracle_tables

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-4
BWD_TOL = 1e-3
SUM_TOL = 1e-4  # glue-parameter gradients: fp32 fixed-order sums vs float64


class LayerSpy:
    """Wraps ops.lut_layer_forward / lut_layer_backward (the calls FusedCIMLayerFn makes) to keep
    every call's inputs and results, run each with a workspace whose table-copy mode word is
    read back afterwards."""

    def __init__(self, monkeypatch):
        from isa.kernels.transformer_ffn import _hip, ops

        self.fwd, self.bwd = [], []
        lib = _hip.load()
        orig_f, orig_b = ops.lut_layer_forward, ops.lut_layer_backward

        def fwd(x, wpos, wneg, fwd_records, n_entries, *a, **k):
            M, K = x.shape
            O = wpos.shape[0]
            plan = ops.plan_info("forward", M, K, O, n_entries)
            nbytes = max(plan["workspace_bytes"], lib.isa_ekv_layer_forward_workspace(M, K, O))
            ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
            out, idiff = orig_f(x, wpos, wneg, fwd_records, n_entries, *a, workspace=ws, **k)
            self.fwd.append(dict(x=x, out=out, idiff=idiff, ws=ws, plan=plan))
            return out, idiff

        def bwd(x, wpos, wneg, grad_out, idiff, bwd_records, n_entries, *a, **k):
            M, K = x.shape
            O = wpos.shape[0]
            need_x = bool(k.get("need_grad_x")) or (bool(k.get("need_in_affine")) and k.get("in_affine") is not None)
            plan = ops.plan_info("layer_backward", M, K, O, n_entries, need_x, bool(k.get("need_grad_w")))
            ws = torch.empty(plan["workspace_bytes"], dtype=torch.uint8, device=x.device)
            res = orig_b(x, wpos, wneg, grad_out, idiff, bwd_records, n_entries, *a, workspace=ws, **k)
            self.bwd.append(dict(grad_out=grad_out, res=res, ws=ws, plan=plan))
            return res

        monkeypatch.setattr(ops, "lut_layer_forward", fwd)
        monkeypatch.setattr(ops, "lut_layer_backward", bwd)

    def modes(self):
        from isa.kernels.transformer_ffn import ops

        torch.cuda.synchronize()
        return ([ops.copy_mode(c["ws"], c["plan"]) for c in self.fwd],
                [ops.copy_mode(c["ws"], c["plan"]) for c in self.bwd])


def _np32(t):
    return t.detach().float().cpu().numpy()


def _f32(v):
    return np.float32(float(v.detach()) if isinstance(v, torch.Tensor) else float(v))


def _tables(cfg):
    dmin, dmax, _ = oracle.lut_range(cfg)
    ti, td = oracle_tables(cfg)
    return ti, td, dmin, dmax, float(cfg["V_sat"])


def _check(name, got, want, tol):
    e = errs(torch.as_tensor(got), want) if not isinstance(got, torch.Tensor) else errs(got, want)
    print(f"  {name}: norm {e[0]:.2e} elem {e[1]:.2e}")
    assert e[0] <= tol, (name, e)


def _check_sum(name, got, want):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    den = max(float(np.max(np.abs(want))), 1e-30)
    e = float(np.max(np.abs(got - want))) / den
    print(f"  {name}: {e:.2e}")
    assert e <= SUM_TOL, (name, e)


def _tia(idiff, r):
    """clamp(idiff * r_tia, -4, 4) in fp32 (cim.py:192-193) and its inclusive clamp mask."""
    y0 = idiff * r
    return np.clip(y0, np.float32(-4.0), np.float32(4.0)), (y0 >= -4.0) & (y0 <= 4.0)


def _check_cim_layer(tag, v, wp, wn, gpu_idiff, g_eff, gpu_dv, gpu_dwp, gpu_dwn, cfg, rows, cols):
    """One CIM projection on exact sub-problems: forward and dX rows from the GPU's input rows
    v[rows] and upstream gradient g_eff[rows]; dVth columns over every token."""
    ti, td, dmin, dmax, vsat = _tables(cfg)
    _check(f"{tag} forward rows", gpu_idiff[rows], oracle.forward(v[rows], wp, wn, ti, dmin, dmax, vsat), FWD_TOL)
    if gpu_dv is not None:
        _check(f"{tag} dX rows", gpu_dv[rows], oracle.grad_x(v[rows], wp, wn, g_eff[rows], ti, td, dmin, dmax, vsat),
               BWD_TOL)
    rgp, rgn = oracle.grad_w(v, wp[cols], wn[cols], np.ascontiguousarray(g_eff[:, cols]), td, dmin, dmax, vsat)
    _check(f"{tag} dVth+ cols", gpu_dwp[cols], rgp, BWD_TOL)
    _check(f"{tag} dVth- cols", gpu_dwn[cols], rgn, BWD_TOL)


def _step(model, x, g):
    model.zero_grad(set_to_none=True)
    xx = x.detach().clone().requires_grad_(True)
    out = model(xx)
    out.backward(g)
    torch.cuda.synchronize()
    return out, xx


def _grads(model, xx):
    return [xx.grad.clone()] + [p.grad.clone() for p in model.parameters() if p.grad is not None]


def _mapping(model, X):
    m = model.input_mapping
    s, b = _f32(m.scale), _f32(m.shift)
    pre = X * s + b  # two fp32 roundings, as the two tensor ops (cim.py:37-39)
    return s, b, pre, np.clip(pre, np.float32(0.0), np.float32(m.voltage_max))


def _inputs(B, T, D, seed):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(B, T, D, generator=gen)


# the forward's windowed table copies: their number depends on the coordinate window the
# inputs reach (3 up to ISA_EKV_OPT_WINDOW_COPIES, default 32)
WINDOWED = range(3, 33)


def _modes_match(got, want):
    """got: the mode words of a layer spy's calls; want: per call an int or a range of ints."""
    return len(got) == len(want) and all(g in w if isinstance(w, range) else g == w for g, w in zip(got, want))


def run_physical_ffn(monkeypatch, dev, D, F, B, T, size, expect_modes, n_rows=48, n_cols=24, seed=0, **cfg_over):
    from isa.device_models.config import make_flash_transistor_ekv_config
    from isa.operators.cim import PhysicalFFN

    cfg = make_flash_transistor_ekv_config(default_lut_size=size)
    cfg["LUT_DELTA_SIZE"] = size
    cfg.update(cfg_over)
    torch.manual_seed(seed)
    ffn = PhysicalFFN(D, F, cfg).to(dev)
    x = _inputs(B, T, D, seed + 1).to(dev)
    g = torch.randn(B, T, D, generator=torch.Generator().manual_seed(seed + 2)).to(dev)
    spy = LayerSpy(monkeypatch)
    out, xx = _step(ffn, x, g)
    fmodes, bmodes = spy.modes()
    print(f"[case] PhysicalFFN {D}->{F}->{D} x[{B},{T},{D}] LUT {size} {cfg.get('LUT_DTYPE', 'float32')}: "
          f"copy modes fwd {fmodes} bwd {bmodes}")
    assert len(spy.fwd) == 2 and len(spy.bwd) == 2, "the fused layer path must serve both projections"
    assert _modes_match(fmodes, expect_modes[0]) and _modes_match(bmodes, expect_modes[1]), (fmodes, bmodes)

    M = B * T
    rng = np.random.default_rng(seed + size)
    rows = np.sort(rng.choice(M, n_rows, replace=False))
    X = _np32(x).reshape(M, D)
    G = _np32(g).reshape(M, D)
    s, b, pre, v = _mapping(ffn, X)
    W1p, W1n, W2p, W2n = (_np32(t) for t in (ffn.fc1.vth_pos, ffn.fc1.vth_neg, ffn.fc2.vth_pos, ffn.fc2.vth_neg))
    r1, r2 = _f32(ffn.fc1.r_tia), _f32(ffn.fc2.r_tia)
    a, c = _np32(ffn.adc_affine_scale), _np32(ffn.adc_affine_shift)
    f1, f2 = spy.fwd
    i1, h = _np32(f1["idiff"]), _np32(f1["out"])
    i2, y_out = _np32(f2["idiff"]), _np32(f2["out"])
    assert np.array_equal(_np32(f1["x"]), X) and np.array_equal(_np32(f2["x"]), h)
    assert torch.equal(out.reshape(M, D), f2["out"])

    # glue, elementwise from the GPU's idiff (each op's own fp32 rounding)
    h_ref, mask1 = _tia(i1, r1)
    y2, mask2 = _tia(i2, r2)
    assert np.array_equal(h, h_ref), "fc1 TIA gain and clamp"
    assert np.array_equal(y_out, y2 * a + c), "fc2 TIA gain, clamp and ADC affine"
    sat = float(np.mean(np.abs(h) >= 4.0))
    print(f"  fc2 input saturation {sat:.3f}")

    # backward: fc2 first (autograd order), its dX is fc1's upstream gradient
    b2, b1 = spy.bwd
    assert torch.equal(b2["grad_out"], g.reshape(M, D))
    dh = _np32(b2["res"]["dx"])
    assert torch.equal(b1["grad_out"], b2["res"]["dx"])
    geff2 = (G * a) * r2 * mask2
    geff1 = dh * r1 * mask1
    cols2 = np.sort(rng.choice(D, min(n_cols, D), replace=False))
    cols1 = np.sort(rng.choice(F, n_cols, replace=False))
    _check_cim_layer("fc2", h, W2p, W2n, i2, geff2, dh, _np32(ffn.fc2.vth_pos.grad), _np32(ffn.fc2.vth_neg.grad),
                     cfg, rows, cols2)
    dv = None
    if s != 0.0:
        dv = _np32(xx.grad).reshape(M, D) / s * ((pre >= 0.0) & (pre <= 4.0))
    ti, td, dmin, dmax, vsat = _tables(cfg)
    ref_dv = oracle.grad_x(v[rows], W1p, W1n, geff1[rows], ti, td, dmin, dmax, vsat)
    ref_dx = ref_dv * float(s) * ((pre[rows] >= 0.0) & (pre[rows] <= 4.0))
    _check("fc1 dX rows (through the input mapping)", xx.grad.reshape(M, D)[torch.as_tensor(rows, device=dev)],
           ref_dx, BWD_TOL)
    _check_cim_layer("fc1", v, W1p, W1n, i1, geff1, None, _np32(ffn.fc1.vth_pos.grad), _np32(ffn.fc1.vth_neg.grad),
                     cfg, rows, cols1)

    # glue parameters' gradients from the GPU's intermediates, float64 sums
    G64 = G.astype(np.float64)
    _check_sum("adc_shift grad", _np32(ffn.adc_affine_shift.grad), G64.sum(0))
    _check_sum("adc_scale grad", _np32(ffn.adc_affine_scale.grad), (G64 * y2).sum(0))
    _check_sum("fc2 r_tia_log_scale grad", _np32(ffn.fc2.r_tia_log_scale.grad),
               ((G64 * a) * mask2 * i2).sum() * float(r2))
    _check_sum("fc1 r_tia_log_scale grad", _np32(ffn.fc1.r_tia_log_scale.grad),
               (dh.astype(np.float64) * mask1 * i1).sum() * float(r1))
    if dv is not None:
        _check_sum("mapping shift grad", _np32(ffn.input_mapping.shift.grad), dv.astype(np.float64).sum())
        _check_sum("mapping scale grad", _np32(ffn.input_mapping.scale.grad), (dv.astype(np.float64) * X).sum())

    # the same step again: bitwise equal outputs and gradients
    first = [out.detach().clone()] + _grads(ffn, xx)
    out2, xx2 = _step(ffn, x, g)
    again = [out2.detach()] + _grads(ffn, xx2)
    assert len(first) == len(again) and all(torch.equal(p, q) for p, q in zip(first, again))


def test_config1_vitm_physical_ffn_4096(cuda_device, monkeypatch):
    """configs[1] with the 4096-entry table: the initial thresholds span ~67 records; fc1's
    mapped inputs reach a coordinate window of ~1400 records (as many windowed forward copies
    as fit its LDS, about seven), fc2's TIA outputs a narrow one (the cap, 32); the backward runs
    ranked."""
    run_physical_ffn(monkeypatch, cuda_device, 256, 1024, 128, 65, 4096, ([WINDOWED, 32], [2, 2]))


def test_config1_vitm_physical_ffn_8192(cuda_device, monkeypatch):
    """configs[1] with the vision default of 8192 entries: the initial thresholds span ~135
    records and both layers' inputs reach a coordinate window that fits (fc1's mapped inputs in
    [0, 4] V, fc2's TIA outputs within a fraction of a volt of zero): fc1's forward holds three
    bank-rotated copies of its ~2800-record window (what fits its 80 KB), fc2's as many of its
    narrow one as fit (about two dozen: twice the records per volt of the 4096-entry table),
    and every backward runs ranked."""
    run_physical_ffn(monkeypatch, cuda_device, 256, 1024, 128, 65, 8192, ([WINDOWED, range(16, 33)], [2, 2]))


def test_config3_headline_physical_ffn(cuda_device, monkeypatch):
    """configs[3], the headline Physical GPT-L FFN at full size, exactly as bench.py runs it."""
    run_physical_ffn(monkeypatch, cuda_device, 768, 3072, 8, 1024, 4096, ([WINDOWED, 32], [2, 2]))


def test_config3_headline_physical_ffn_bf16_tables(cuda_device, monkeypatch):
    """The headline with LUT_DTYPE=bfloat16: the reference's own bf16 tables (delta_lut.py:35),
    checked against the oracle fed the same bytes. fc2's inputs are the TIA outputs of the
    initial model, within a fraction of a volt of zero, where the reference's fp32 table
    construction and an fp64-accurate one differ most after the bf16 cast."""
    run_physical_ffn(monkeypatch, cuda_device, 768, 3072, 8, 1024, 4096, ([WINDOWED, 32], [2, 2]),
                     LUT_DTYPE="bfloat16")


def test_config2_gptm_hybrid_ffn(cuda_device, monkeypatch):
    """configs[2] Hybrid GPT-M: the fused CIM up-projection (input mapping, TIA gain, clamp)
    and the digital nn.Linear down-projection on rocBLAS/hipBLASLt."""
    from isa.device_models.config import make_flash_transistor_ekv_config
    from isa.operators.cim import HybridFFN

    dev = cuda_device
    D, F, B, T, size = 384, 1536, 16, 1024, 4096
    cfg = make_flash_transistor_ekv_config(default_lut_size=size)
    cfg["LUT_DELTA_SIZE"] = size
    torch.manual_seed(3)
    ffn = HybridFFN(D, F, cfg).to(dev)
    x = _inputs(B, T, D, 4).to(dev)
    g = torch.randn(B, T, D, generator=torch.Generator().manual_seed(5)).to(dev)
    spy = LayerSpy(monkeypatch)
    out, xx = _step(ffn, x, g)
    fmodes, bmodes = spy.modes()
    print(f"[case] HybridFFN {D}->{F} + Linear x[{B},{T},{D}]: copy modes fwd {fmodes} bwd {bmodes}")
    assert len(spy.fwd) == 1 and len(spy.bwd) == 1
    assert _modes_match(fmodes, [WINDOWED]) and bmodes == [2], (fmodes, bmodes)

    M = B * T
    rng = np.random.default_rng(6)
    rows = np.sort(rng.choice(M, 48, replace=False))
    cols = np.sort(rng.choice(F, 24, replace=False))
    X, G = _np32(x).reshape(M, D), _np32(g).reshape(M, D)
    s, b, pre, v = _mapping(ffn, X)
    W1p, W1n = _np32(ffn.fc1.vth_pos), _np32(ffn.fc1.vth_neg)
    r1 = _f32(ffn.fc1.r_tia)
    f1, b1 = spy.fwd[0], spy.bwd[0]
    i1, h = _np32(f1["idiff"]), _np32(f1["out"])
    h_ref, mask1 = _tia(i1, r1)
    assert np.array_equal(h, h_ref), "fc1 TIA gain and clamp"
    # digital down-projection on sampled rows (fp32 GEMM vs float64)
    Wl, bl = _np32(ffn.fc2.weight).astype(np.float64), _np32(ffn.fc2.bias).astype(np.float64)
    _check("digital fc2 rows", out.reshape(M, D)[torch.as_tensor(rows, device=dev)], h[rows] @ Wl.T + bl, 1e-5)
    # its backward gives fc1's upstream gradient
    dh = _np32(b1["grad_out"])
    _check("digital fc2 dX rows", b1["grad_out"][torch.as_tensor(rows, device=dev)], G[rows] @ Wl, 1e-5)
    _check_sum("digital fc2 weight grad", _np32(ffn.fc2.weight.grad), G.astype(np.float64).T @ h)
    _check_sum("digital fc2 bias grad", _np32(ffn.fc2.bias.grad), G.astype(np.float64).sum(0))
    geff1 = dh * r1 * mask1
    ti, td, dmin, dmax, vsat = _tables(cfg)
    ref_dv = oracle.grad_x(v[rows], W1p, W1n, geff1[rows], ti, td, dmin, dmax, vsat)
    ref_dx = ref_dv * float(s) * ((pre[rows] >= 0.0) & (pre[rows] <= 4.0))
    _check("fc1 dX rows (through the input mapping)", xx.grad.reshape(M, D)[torch.as_tensor(rows, device=dev)],
           ref_dx, BWD_TOL)
    _check_cim_layer("fc1", v, W1p, W1n, i1, geff1, None, _np32(ffn.fc1.vth_pos.grad), _np32(ffn.fc1.vth_neg.grad),
                     cfg, rows, cols)
    _check_sum("fc1 r_tia_log_scale grad", _np32(ffn.fc1.r_tia_log_scale.grad),
               (dh.astype(np.float64) * mask1 * i1).sum() * float(r1))
    first = [out.detach().clone()] + _grads(ffn, xx)
    out2, xx2 = _step(ffn, x, g)
    again = [out2.detach()] + _grads(ffn, xx2)
    assert all(torch.equal(p, q) for p, q in zip(first, again))
