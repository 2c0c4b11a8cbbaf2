"""Drop-in surface on the GPU: CIMLinear / PhysicalFFN / HybridFFN autograd, estimate_idiff,
and the cuda_backend extension API, each against the CPU oracle composed by hand."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import errs, flash_cfg, make_inputs

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().double().cpu().numpy()


def _oracle_layer(x, wp, wn, cfg):
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, td = oracle.lut_tables(cfg)
    return oracle.forward(x, wp, wn, ti, dmin, dmax, cfg["V_sat"], -4.0, 4.0)


def _oracle_layer_bwd(x, wp, wn, g, cfg):
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, td = oracle.lut_tables(cfg)
    return oracle.backward(x, wp, wn, g, ti, td, dmin, dmax, cfg["V_sat"])


def test_physical_ffn_autograd(cuda_device):
    """VoltageMapping -> CIMLinear -> CIMLinear -> ADC affine (cim.py:217-247), all gradients."""
    from isa.operators.cim import PhysicalFFN

    cfg = flash_cfg(4096)
    torch.manual_seed(1)
    D, F, B, T = 48, 160, 2, 37
    ffn = PhysicalFFN(D, F, cfg).to(cuda_device)
    with torch.no_grad():
        ffn.input_mapping.set_affine(0.9, 0.4)
        ffn.fc1.r_tia_log_scale.fill_(0.3)
        ffn.adc_affine_scale.uniform_(0.5, 1.5)
        ffn.adc_affine_shift.uniform_(-0.1, 0.1)
    x = torch.randn(B, T, D, device=cuda_device, requires_grad=True)
    out = ffn(x)
    g = torch.randn_like(out)
    out.backward(g)
    torch.cuda.synchronize()

    # oracle composition on the CPU
    X = _np(x).reshape(-1, D)
    s, b = float(ffn.input_mapping.scale.detach()), float(ffn.input_mapping.shift.detach())
    pre0 = X * s + b
    v = np.clip(pre0, 0.0, 4.0)
    r1, r2 = float(ffn.fc1.r_tia.detach()), float(ffn.fc2.r_tia.detach())
    W1p, W1n, W2p, W2n = (_np(t) for t in (ffn.fc1.vth_pos, ffn.fc1.vth_neg, ffn.fc2.vth_pos, ffn.fc2.vth_neg))
    i1 = _oracle_layer(v.astype(np.float32), W1p, W1n, cfg)
    h = np.clip(i1 * r1, -4.0, 4.0)
    i2 = _oracle_layer(h.astype(np.float32), W2p, W2n, cfg)
    y = np.clip(i2 * r2, -4.0, 4.0)
    a, c = _np(ffn.adc_affine_scale), _np(ffn.adc_affine_shift)
    ref = y * a + c
    assert oracle.normwise_error(_np(out).reshape(-1, D), ref) <= 1e-4

    G = _np(g).reshape(-1, D)
    dy = G * a
    gi2 = dy * r2 * (np.abs(i2 * r2) < 4.0)
    dh, dW2p, dW2n = _oracle_layer_bwd(h.astype(np.float32), W2p, W2n, gi2.astype(np.float32), cfg)
    gi1 = dh * r1 * (np.abs(i1 * r1) < 4.0)
    dv, dW1p, dW1n = _oracle_layer_bwd(v.astype(np.float32), W1p, W1n, gi1.astype(np.float32), cfg)
    dx = dv * s * ((pre0 > 0.0) & (pre0 < 4.0))
    checks = {
        "dx": (x.grad, dx), "fc1.vth_pos": (ffn.fc1.vth_pos.grad, dW1p), "fc1.vth_neg": (ffn.fc1.vth_neg.grad, dW1n),
        "fc2.vth_pos": (ffn.fc2.vth_pos.grad, dW2p), "fc2.vth_neg": (ffn.fc2.vth_neg.grad, dW2n),
        "adc_scale": (ffn.adc_affine_scale.grad, (G * y).sum(0)), "adc_shift": (ffn.adc_affine_shift.grad, G.sum(0)),
    }
    for name, (got, want) in checks.items():
        e = oracle.normwise_error(_np(got).reshape(want.shape), want)
        print(name, f"{e:.2e}")
        assert e <= 1e-3, name
    # TIA log-scale gradient: d out / d s1 = Idiff1 * r1 inside the clamp
    want = float((dh * (np.abs(i1 * r1) < 4.0) * i1 * r1).sum())
    got = float(ffn.fc1.r_tia_log_scale.grad)
    assert abs(got - want) <= 1e-3 * max(abs(want), 1e-12)


def test_hybrid_ffn_autograd(cuda_device):
    from isa.operators.cim import HybridFFN

    cfg = flash_cfg(4096)
    torch.manual_seed(2)
    D, F = 40, 96
    ffn = HybridFFN(D, F, cfg).to(cuda_device)
    x = torch.randn(3, 11, D, device=cuda_device, requires_grad=True)
    out = ffn(x)
    g = torch.randn_like(out)
    out.backward(g)
    X = _np(x).reshape(-1, D)
    v = np.clip(X, 0.0, 4.0)
    r1 = float(ffn.fc1.r_tia.detach())
    W1p, W1n = _np(ffn.fc1.vth_pos), _np(ffn.fc1.vth_neg)
    i1 = _oracle_layer(v.astype(np.float32), W1p, W1n, cfg)
    h = np.clip(i1 * r1, -4.0, 4.0)
    Wl, bl = _np(ffn.fc2.weight), _np(ffn.fc2.bias)
    ref = h @ Wl.T + bl
    assert oracle.normwise_error(_np(out).reshape(-1, D), ref) <= 1e-4
    dh = _np(g).reshape(-1, D) @ Wl
    gi1 = dh * r1 * (np.abs(i1 * r1) < 4.0)
    dv, dWp, dWn = _oracle_layer_bwd(v.astype(np.float32), W1p, W1n, gi1.astype(np.float32), cfg)
    dx = dv * ((X > 0.0) & (X < 4.0))
    assert oracle.normwise_error(_np(x.grad).reshape(-1, D), dx) <= 1e-3
    assert oracle.normwise_error(_np(ffn.fc1.vth_pos.grad), dWp) <= 1e-3
    assert oracle.normwise_error(_np(ffn.fc1.vth_neg.grad), dWn) <= 1e-3


def test_cimlinear_dtypes_and_estimate_idiff(cuda_device):
    """bf16 activations compute in fp32 (out is fp32 Idiff x R_TIA); grads come back in the input dtype."""
    from isa.operators.cim import CIMLinear

    cfg = flash_cfg(4096)
    torch.manual_seed(3)
    layer = CIMLinear(64, 128, cfg).to(cuda_device)
    x = torch.rand(2, 20, 64, device=cuda_device).mul(4.0).to(torch.bfloat16).requires_grad_(True)
    out = layer(x)
    assert out.dtype == torch.float32
    out.sum().backward()
    assert x.grad.dtype == torch.bfloat16 and layer.vth_pos.grad.dtype == torch.float32
    est = layer.estimate_idiff(x.detach(), max_rows=25)
    assert est.shape == (25, 128)
    X = x.detach().float().reshape(-1, 64)[:25].cpu().numpy()
    ref = _oracle_layer(X, _np(layer.vth_pos), _np(layer.vth_neg), cfg)
    assert oracle.normwise_error(_np(est), ref) <= 1e-4


def test_cuda_backend_extension_api(cuda_device):
    """load_extension() ops and shared_backward keep the reference's tensor API
    (binding.cpp:56-62, cuda_backend.py:50-99), checked against the oracle."""
    from isa.approximations.delta_lut import get_ekv_lut_tables
    from isa.kernels.transformer_ffn import cuda_backend

    cfg = flash_cfg(4096)
    dmin, dmax, n = oracle.lut_range(cfg)
    ti_d, td_d = get_ekv_lut_tables(cfg, cuda_device)
    x, vp, vn, g = make_inputs(57, 70, 90, seed=21, x_mode="signed", vth_mode="full")
    xd, pd, nd, gd = (t.to(cuda_device) for t in (x, vp, vn, g))
    ext = cuda_backend.load_extension()
    ti, td = oracle.lut_tables(cfg)
    ref = oracle.forward(x.numpy(), vp.numpy(), vn.numpy(), ti, dmin, dmax, cfg["V_sat"], -np.inf, np.inf)
    assert errs(ext.forward(xd, pd, nd, ti_d, dmin, dmax, cfg["V_sat"]), ref)[0] <= 1e-4
    rdx, rgp, rgn = oracle.backward(x.numpy(), vp.numpy(), vn.numpy(), g.numpy(), ti, td, dmin, dmax, cfg["V_sat"])
    for fn in (ext.grad_x, ext.grad_x_shared):
        assert errs(fn(xd, pd, nd, gd, ti_d, td_d, dmin, dmax, cfg["V_sat"]), rdx)[0] <= 1e-3
    for fn in (ext.grad_w, ext.grad_w_shared):
        gp, gn = fn(xd, pd, nd, gd, td_d, dmin, dmax, cfg["V_sat"])
        assert errs(gp, rgp)[0] <= 1e-3 and errs(gn, rgn)[0] <= 1e-3
    gx, gp, gn = cuda_backend.shared_backward(xd.double(), pd, nd, gd, ti_d, td_d, dmin, dmax, cfg["V_sat"], True, True)
    assert gx.dtype == torch.float64
    assert errs(gx, rdx)[0] <= 1e-3 and errs(gp, rgp)[0] <= 1e-3 and errs(gn, rgn)[0] <= 1e-3
    gx, gp, gn = cuda_backend.shared_backward(xd, pd, nd, gd, ti_d, td_d, dmin, dmax, cfg["V_sat"], False, True)
    assert gx is None and gp is not None
    with pytest.raises(RuntimeError, match="x must be float32"):
        ext.grad_x_shared(xd.double(), pd, nd, gd, ti_d, td_d, dmin, dmax, cfg["V_sat"])
    big_i, big_d = get_ekv_lut_tables(flash_cfg(8193), cuda_device)
    with pytest.raises(RuntimeError, match="LUT_DELTA_SIZE <= 8192"):
        ext.grad_x_shared(xd, pd, nd, gd, big_i, big_d, dmin, dmax, cfg["V_sat"])


def test_backward_size_limit_message(cuda_device):
    from isa.kernels.transformer_ffn.ekv_lut_triton import triton_lut_ekv_matmul

    cfg = flash_cfg(12000)
    x, vp, vn, _ = make_inputs(8, 16, 32, seed=0)
    xd = x.to(cuda_device).requires_grad_(True)
    out = triton_lut_ekv_matmul(xd, vp.to(cuda_device), vn.to(cuda_device), cfg)
    with pytest.raises(RuntimeError, match="CUDA shared EKV backward requires LUT_DELTA_SIZE <= 8192"):
        out.sum().backward()


def test_backward_large_table_without_shared_backward(cuda_device):
    """With CUDA_SHARED_BACKWARD off the reference runs its Triton backward at any table size
    (ekv_lut_triton.py:193-218); here the global-memory table kernels serve it, through the
    autograd function and the fused CIMLinear layer alike."""
    from isa.kernels.transformer_ffn.ekv_lut_triton import triton_lut_ekv_matmul
    from isa.operators.cim import CIMLinear

    cfg = flash_cfg(12000, CUDA_SHARED_BACKWARD=False)
    x, vp, vn, g = make_inputs(8, 16, 32, seed=0)
    dmin, dmax, n = oracle.lut_range(cfg)
    ti, td = oracle.lut_tables(cfg)
    xd = x.to(cuda_device).requires_grad_(True)
    pd, nd = vp.to(cuda_device).requires_grad_(True), vn.to(cuda_device).requires_grad_(True)
    out = triton_lut_ekv_matmul(xd, pd, nd, cfg)
    out.backward(g.to(cuda_device))
    X, P, N, G = (t.numpy() for t in (x, vp, vn, g))
    assert errs(out.detach(), oracle.forward(X, P, N, ti, dmin, dmax, cfg["V_sat"]))[0] <= 1e-4
    assert errs(xd.grad, oracle.grad_x(X, P, N, G, ti, td, dmin, dmax, cfg["V_sat"]))[0] <= 1e-3
    rgp, rgn = oracle.grad_w(X, P, N, G, td, dmin, dmax, cfg["V_sat"])
    assert errs(pd.grad, rgp)[0] <= 1e-3 and errs(nd.grad, rgn)[0] <= 1e-3
    layer = CIMLinear(16, 32, cfg).to(cuda_device)
    xl = (torch.rand(3, 5, 16, device=cuda_device) * 4.0).requires_grad_(True)
    layer(xl).sum().backward()
    assert torch.isfinite(xl.grad).all() and layer.vth_pos.grad is not None


def test_prebuild(cuda_device, capsys):
    from isa.kernels.transformer_ffn import cuda_backend

    cuda_backend.prebuild()
    assert "[ekv-cuda] ready: isa_ekv_hip" in capsys.readouterr().out
