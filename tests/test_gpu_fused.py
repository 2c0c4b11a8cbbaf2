"""The fused layer glue (isa_ekv_layer_forward/backward) against the same modules with the
glue as separate PyTorch ops: forward outputs and the projections' gradients must be
bitwise equal (each fused op keeps the rounding of its tensor op), the glue parameters'
gradients equal up to summation order. The unfused composition itself is checked against
the CPU oracle in test_gpu_module.py."""

from __future__ import annotations

import pytest
import torch

from tests.helpers import flash_cfg

pytestmark = pytest.mark.gpu


def _run(model, x, g, fused: bool):
    from isa.operators import cim

    saved = cim.FUSE_GLUE
    cim.FUSE_GLUE = fused
    try:
        model.zero_grad(set_to_none=True)
        xi = x.detach().clone().requires_grad_(True)
        out = model(xi)
        out.backward(g)
        torch.cuda.synchronize()
        grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
        grads["x"] = xi.grad.detach().clone()
        return out.detach().clone(), grads
    finally:
        cim.FUSE_GLUE = saved


def _compare(a, b, exact_names):
    out_a, ga = a
    out_b, gb = b
    assert torch.equal(out_a, out_b)
    assert set(ga) == set(gb)
    for name in ga:
        if name in exact_names:
            assert torch.equal(ga[name], gb[name]), name
        else:
            # glue-parameter gradients are fp32 sums over M*K or M*O terms that cancel
            # (2.9e-10 from terms of either sign); the two paths sum in different orders.
            # Their float64 values are checked against the oracle in test_gpu_module.py.
            assert torch.allclose(ga[name], gb[name], rtol=1e-3, atol=1e-5 * float(gb[name].abs().max()) + 1e-30), name


@pytest.mark.parametrize("log_scale", [0.3, 1.6, 2.5])  # 1.6: many outputs in both clamps; 2.5: past the log-scale clamp
def test_physical_ffn_fused_equals_unfused(cuda_device, log_scale):
    from isa.operators.cim import PhysicalFFN

    print(f"[case] fused PhysicalFFN log_scale={log_scale}", flush=True)
    torch.manual_seed(11)
    D, F = 96, 260  # F not a multiple of 256: padded outputs in both layers
    ffn = PhysicalFFN(D, F, flash_cfg(4096)).to(cuda_device)
    with torch.no_grad():
        ffn.input_mapping.set_affine(1.1, 0.3)
        ffn.fc1.r_tia_log_scale.fill_(log_scale)
        ffn.fc2.r_tia_log_scale.fill_(-0.2)
        ffn.adc_affine_scale.uniform_(0.5, 1.5)
        ffn.adc_affine_shift.uniform_(-0.1, 0.1)
    x = torch.randn(3, 41, D, device=cuda_device) * 2.0  # reaches both ends of the [0, 4] mapping
    g = torch.randn(3, 41, D, device=cuda_device)
    fused = _run(ffn, x, g, True)
    plain = _run(ffn, x, g, False)
    exact = {"x", "fc1.vth_pos", "fc1.vth_neg", "fc2.vth_pos", "fc2.vth_neg"}
    _compare(fused, plain, exact)
    # every glue parameter received a gradient
    for name in ("input_mapping.scale", "input_mapping.shift", "fc1.r_tia_log_scale", "fc2.r_tia_log_scale",
                 "adc_affine_scale", "adc_affine_shift"):
        assert name in fused[1], name
    if log_scale > 2.0:  # past R_TIA_LOG_SCALE_MAX: the clamp passes no gradient
        assert float(fused[1]["fc1.r_tia_log_scale"]) == 0.0
    else:
        assert float(fused[1]["fc1.r_tia_log_scale"]) != 0.0


def test_hybrid_ffn_and_cimlinear_fused_equal_unfused(cuda_device):
    from isa.operators.cim import CIMLinear, HybridFFN

    torch.manual_seed(12)
    cfg = flash_cfg(4096)
    ffn = HybridFFN(64, 300, cfg).to(cuda_device)
    x = torch.randn(2, 33, 64, device=cuda_device)
    g = torch.randn(2, 33, 64, device=cuda_device)
    _compare(_run(ffn, x, g, True), _run(ffn, x, g, False), {"x", "fc1.vth_pos", "fc1.vth_neg"})

    layer = CIMLinear(70, 130, cfg).to(cuda_device)
    with torch.no_grad():
        layer.r_tia_log_scale.fill_(1.2)
    x = torch.rand(2, 19, 70, device=cuda_device) * 4.0
    g = torch.randn(2, 19, 130, device=cuda_device)
    _compare(_run(layer, x, g, True), _run(layer, x, g, False), {"x", "vth_pos", "vth_neg"})


def test_fused_layer_bf16_input_and_frozen_parameters(cuda_device):
    """bf16 activations take the unfused voltage mapping (its output is rounded to bf16) and
    the fused CIM layers; parameters without requires_grad get no gradient."""
    from isa.operators.cim import PhysicalFFN

    torch.manual_seed(13)
    ffn = PhysicalFFN(48, 96, flash_cfg(4096)).to(cuda_device)
    ffn.adc_affine_scale.requires_grad_(False)
    ffn.fc2.r_tia_log_scale.requires_grad_(False)
    x = torch.randn(2, 9, 48, device=cuda_device).to(torch.bfloat16)
    g = torch.randn(2, 9, 48, device=cuda_device)
    fused = _run(ffn, x, g, True)
    plain = _run(ffn, x, g, False)
    assert "adc_affine_scale" not in fused[1] and "fc2.r_tia_log_scale" not in fused[1]
    _compare(fused, plain, {"x", "fc1.vth_pos", "fc1.vth_neg", "fc2.vth_pos", "fc2.vth_neg"})


def test_fused_layer_direct_call_and_degenerate_k(cuda_device):
    """fused_cim_layer with every glue piece, and K = 0 (empty sums: idiff = 0, the glue
    still acts and its parameters still get gradients)."""
    from isa.kernels.transformer_ffn.fused_layer import fused_cim_layer

    cfg = flash_cfg(4096)
    dev = cuda_device
    M, O = 5, 7
    x = torch.empty(M, 0, device=dev, requires_grad=True)
    wp = torch.empty(O, 0, device=dev, requires_grad=True)
    wn = torch.empty(O, 0, device=dev, requires_grad=True)
    r = torch.tensor([2.0], device=dev, requires_grad=True)
    a = torch.rand(O, device=dev, requires_grad=True)
    c = torch.rand(O, device=dev, requires_grad=True)
    aff = torch.tensor([1.0, 0.5], device=dev, requires_grad=True)
    out = fused_cim_layer(x, wp, wn, cfg, in_affine=aff, r_tia=r, adc_scale=a, adc_shift=c)
    assert torch.equal(out, c.detach().expand(M, O))  # idiff = 0 -> y = 0 -> out = shift
    gz = torch.randn(M, O, device=dev)
    out.backward(gz)
    assert torch.allclose(c.grad, gz.sum(0)) and float(a.grad.abs().max()) == 0.0
    assert float(r.grad.abs().max()) == 0.0 and float(aff.grad.abs().max()) == 0.0


def test_output_stats_fused_equal_unfused(cuda_device):
    """Output-statistics tracking (cim.py:194-198) in the fused epilogue: after two forwards
    the counts and running max |y| equal the separate-op path's; a larger running max is
    kept; NaN outputs (a NaN TIA gain) make the max NaN as torch.maximum does."""
    import math

    from isa.operators.cim import PhysicalFFN

    print("[case] fused output statistics", flush=True)
    torch.manual_seed(14)
    ffn = PhysicalFFN(64, 200, flash_cfg(4096)).to(cuda_device)
    with torch.no_grad():
        ffn.fc1.r_tia_base.fill_(4e6)  # |idiff| reaches ~2e-6 A: some outputs clamp at +-4
    xs = [torch.randn(2, 37, 64, device=cuda_device) * 2.0, torch.randn(1, 23, 64, device=cuda_device)]
    gain = float(ffn.fc2.r_tia_base)

    def stats(fused, preset=0.0, nan_gain=False):
        from isa.operators import cim

        saved = cim.FUSE_GLUE
        cim.FUSE_GLUE = fused
        try:
            for layer in (ffn.fc1, ffn.fc2):
                layer.set_output_stats_tracking(True, reset=True)
                layer._stat_abs_max.fill_(preset)
            with torch.no_grad():
                ffn.fc2.r_tia_base.fill_(float("nan") if nan_gain else gain)
                for x in xs:
                    ffn(x)
            torch.cuda.synchronize()
            return [layer.output_stats() for layer in (ffn.fc1, ffn.fc2)]
        finally:
            cim.FUSE_GLUE = saved
            with torch.no_grad():
                ffn.fc2.r_tia_base.fill_(gain)
            for layer in (ffn.fc1, ffn.fc2):
                layer.set_output_stats_tracking(False)

    fused, plain = stats(True), stats(False)
    assert fused == plain, (fused, plain)
    assert fused[0]["total"] == (2 * 37 + 23) * 200 and fused[1]["total"] == (2 * 37 + 23) * 64
    assert fused[0]["preclamp_abs_max"] == 4.0  # clamped outputs reached the bound
    assert stats(True, preset=100.0) == stats(False, preset=100.0)
    assert stats(True, preset=100.0)[1]["preclamp_abs_max"] == 100.0
    nan_fused, nan_plain = stats(True, nan_gain=True), stats(False, nan_gain=True)
    assert nan_fused[0] == nan_plain[0] == fused[0]
    assert math.isnan(nan_fused[1]["preclamp_abs_max"]) and math.isnan(nan_plain[1]["preclamp_abs_max"])
    assert nan_fused[1]["total"] == nan_plain[1]["total"]
