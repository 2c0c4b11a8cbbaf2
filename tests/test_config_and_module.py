"""Configuration and module surface of the drop-in package (CPU only)."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "flash_transistor_ekv.json"


def test_runtime_parameters_match_device_file():
    """Restates the reference's tests/test_device_parameters.py:12-27 against the committed values."""
    from isa.device_models.config import FLASH_TRANSISTOR_PARAMETERS as P

    payload = json.loads(GOLDEN.read_text())
    for k in ("I_S", "n", "U_T", "V_D", "V_sat", "R_TIA"):
        assert payload["parameters"][k] == pytest.approx(P[k])
    assert payload["ranges"]["Vth"] == [P["V_TH_MIN"], P["V_TH_MAX"]]
    assert payload["ranges"]["input_voltage"] == [P["V_min"], P["V_max"]]
    assert payload["ranges"]["signed_output_voltage"] == [P["V_signed_min"], P["V_signed_max"]]


def test_config_factory_and_env(monkeypatch):
    from isa.device_models import config as c

    cfg = c.make_flash_transistor_ekv_config(default_lut_size=4096)
    assert cfg["LUT_DELTA_SIZE"] == 4096 and cfg["use_triton"] and cfg["ekv_approx"] == "lut"
    assert cfg["CUDA_SHARED_BACKWARD"] is True and cfg["FORWARD_CHUNK_SIZE"] == 64
    assert c.FLASH_TRANSISTOR_EKV_CONFIG["LUT_DELTA_SIZE"] in (8192, int(__import__("os").environ.get("EKV_LUT_SIZE", 8192)))
    monkeypatch.setenv("EKV_LUT_SIZE", "2048")
    monkeypatch.setenv("EKV_CUDA_SHARED_BACKWARD", "0")
    cfg = c.make_flash_transistor_ekv_config(default_lut_size=4096)
    assert cfg["LUT_DELTA_SIZE"] == 2048 and cfg["CUDA_SHARED_BACKWARD"] is False


def test_lut_range_resolution():
    from isa.approximations.delta_lut import lut_range, lut_is_bf16
    from isa.device_models.config import make_flash_transistor_ekv_config

    cfg = make_flash_transistor_ekv_config(4096)
    assert lut_range(cfg) == (-9.0, 4.0, 4096)          # V_signed_min - V_TH_MAX, V_signed_max - V_TH_MIN
    assert lut_range({"LUT_DELTA_MIN": -1.0, "LUT_DELTA_MAX": 3.0}) == (-1.0, 3.0, 16384)
    assert not lut_is_bf16(cfg) and lut_is_bf16({"LUT_DTYPE": "bfloat16"})
    with pytest.raises(ValueError):
        lut_is_bf16({"LUT_DTYPE": "fp8"})


def test_cimlinear_parameters_and_init():
    """Names, shapes and the centered_random init of cim.py:49-71, :113-138 (same RNG order)."""
    from isa.device_models.config import make_flash_transistor_ekv_config
    from isa.operators.cim import CIMLinear

    cfg = make_flash_transistor_ekv_config(4096)
    torch.manual_seed(0)
    layer = CIMLinear(24, 40, cfg)
    sd = layer.state_dict()
    assert set(sd) == {"vth_pos", "vth_neg", "r_tia_base", "r_tia_log_scale"}
    assert layer.vth_pos.shape == (40, 24) and layer.vth_neg.shape == (40, 24)
    assert float(layer.r_tia.detach()) == pytest.approx(1e5)
    eps = 0.5 * 2.0 * cfg["n"] * cfg["U_T"]
    torch.manual_seed(0)
    ref_p = torch.empty(40, 24).uniform_(-eps, eps).add_(2.5)
    ref_n = torch.empty(40, 24).uniform_(-eps, eps).add_(2.5)
    assert torch.equal(layer.vth_pos.data, ref_p) and torch.equal(layer.vth_neg.data, ref_n)
    with torch.no_grad():
        layer.vth_pos.fill_(7.0)
        layer.r_tia_log_scale.fill_(5.0)
    layer.clamp_vth()
    assert float(layer.vth_pos.max()) == 5.0
    assert float(layer.r_tia.detach()) == pytest.approx(1e5 * torch.exp(torch.tensor(2.0)).item(), rel=1e-6)
    layer.set_r_tia(3e4)
    assert float(layer.r_tia.detach()) == pytest.approx(3e4)
    layer.reset_vth(center=1.0, eps_k=0.5, symmetric=True, mode="centered_symmetric")
    assert torch.allclose(layer.vth_pos + layer.vth_neg, torch.full_like(layer.vth_pos, 2.0), atol=1e-6)


def test_ffn_module_layout():
    from isa.operators.cim import HybridFFN, PhysicalFFN

    p = PhysicalFFN(16, 64)
    assert {n for n, _ in p.named_parameters()} >= {"input_mapping.scale", "input_mapping.shift",
                                                     "fc1.vth_pos", "fc1.vth_neg", "fc2.vth_pos",
                                                     "adc_affine_scale", "adc_affine_shift"}
    h = HybridFFN(16, 64)
    assert isinstance(h.fc2, torch.nn.Linear) and h.fc1.vth_pos.shape == (64, 16)


def test_cpu_input_raises_instead_of_falling_back():
    from isa.operators.cim import CIMLinear, VoltageMapping

    layer = CIMLinear(8, 8)
    x = torch.rand(1, 3, 8)
    with pytest.raises(RuntimeError, match="ROCm device"):
        layer(x)
    with pytest.raises(RuntimeError, match="ROCm device"):
        layer.estimate_idiff(x)
    v = VoltageMapping()
    assert torch.equal(v(torch.tensor([-1.0, 2.0, 9.0])), torch.tensor([0.0, 2.0, 4.0]))


def test_ops_reject_cpu_tensors():
    from isa.kernels.transformer_ffn import cuda_backend, ops

    x = torch.rand(4, 8)
    w = torch.rand(5, 8)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        ops.lut_forward(x, w, w, torch.empty(1), 4096, -9.0, 4.0, 8.26, -4.0, 4.0)
    ext = cuda_backend.load_extension()
    assert ext.__name__ == "isa_ekv_hip"
    with pytest.raises(RuntimeError, match="x must be a CUDA tensor"):
        ext.grad_x_shared(x, w, w, torch.rand(4, 5), torch.rand(16), torch.rand(16), -9.0, 4.0, 8.26)
