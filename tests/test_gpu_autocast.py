"""The drop-in under the reference trainers' mixed precision: torch.autocast(bfloat16) as
language/train.py:729 runs the model, and fp16 autocast with a GradScaler-scaled loss as
vision/train.py:190-206 does. The CIM projections compute in fp32 inside their autograd
Functions (the reference's LUTTritonEKVMatmulFn also returns fp32), so a PhysicalFFN fed the
fp32 output of a LayerNorm gives the fp32 eager results exactly under autocast; a GradScaler
scales the upstream gradient by a power of two, which every linear-in-G backward carries
exactly, so the unscaled gradients equal the unscaled run's."""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from tests.helpers import flash_cfg

pytestmark = pytest.mark.gpu


class Block(nn.Module):
    """LayerNorm -> FFN with a residual, the FFN half of a transformer block."""

    def __init__(self, ffn, d):
        super().__init__()
        self.ln = nn.LayerNorm(d)
        self.ffn = ffn

    def forward(self, x):
        return x + self.ffn(self.ln(x))


def _run(model, x, g, autocast_dtype=None, scaler=None):
    model.zero_grad(set_to_none=True)
    xx = x.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=autocast_dtype or torch.float32, enabled=autocast_dtype is not None):
        out = model(xx)
        loss = (out.float() * g).sum()
    if scaler is not None:
        scaler.scale(loss).backward()
    else:
        loss.backward()
    torch.cuda.synchronize()
    return out.detach(), [xx.grad.detach().clone()] + [p.grad.detach().clone() for p in model.parameters()]


def _physical_block(dev, seed=0):
    from isa.operators.cim import PhysicalFFN

    torch.manual_seed(seed)
    d, f = 96, 384
    return Block(PhysicalFFN(d, f, flash_cfg(4096)), d).to(dev), d


def test_physical_ffn_under_bf16_autocast(cuda_device):
    model, d = _physical_block(cuda_device)
    x = torch.randn(4, 50, d, device=cuda_device)
    g = torch.randn(4, 50, d, device=cuda_device)
    out32, grads32 = _run(model, x, g)
    out_ac, grads_ac = _run(model, x, g, torch.bfloat16)
    assert out_ac.dtype == torch.float32
    assert torch.equal(out_ac, out32)
    assert all(torch.equal(a, b) for a, b in zip(grads_ac, grads32))


def test_cimlinear_under_bf16_autocast(cuda_device):
    from isa.operators.cim import CIMLinear

    torch.manual_seed(1)
    layer = CIMLinear(64, 256, flash_cfg(4096)).to(cuda_device)
    x = torch.randn(3, 40, 64, device=cuda_device).clamp(0.0, 4.0)
    g = torch.randn(3, 40, 256, device=cuda_device)
    out32, grads32 = _run(layer, x, g)
    out_ac, grads_ac = _run(layer, x, g, torch.bfloat16)
    assert torch.equal(out_ac, out32)
    assert all(torch.equal(a, b) for a, b in zip(grads_ac, grads32))


def test_hybrid_ffn_under_bf16_autocast(cuda_device):
    """The digital Linear down-projection runs in bf16 under autocast (so does the
    reference's); outputs and gradients stay within bf16 rounding of the fp32 run."""
    from isa.operators.cim import HybridFFN

    torch.manual_seed(2)
    d, f = 96, 384
    model = Block(HybridFFN(d, f, flash_cfg(4096)), d).to(cuda_device)
    x = torch.randn(4, 50, d, device=cuda_device)
    g = torch.randn(4, 50, d, device=cuda_device)
    out32, grads32 = _run(model, x, g)
    out_ac, grads_ac = _run(model, x, g, torch.bfloat16)
    den = out32.abs().max()
    assert float((out_ac.float() - out32).abs().max() / den) <= 2e-2
    for (name, _), a, b in zip([("x", None)] + list(model.named_parameters()), grads_ac, grads32):
        e = float((a.float() - b).abs().max() / b.abs().max().clamp_min(1e-30))
        print(f"{name}: {e:.2e}")
        assert e <= 5e-2, name


def test_physical_ffn_fp16_autocast_with_grad_scaler(cuda_device):
    model, d = _physical_block(cuda_device, seed=3)
    x = torch.randn(4, 50, d, device=cuda_device)
    g = torch.randn(4, 50, d, device=cuda_device)
    out32, grads32 = _run(model, x, g)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 16)
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    out16, _ = _run(model, x, g, torch.float16, scaler=scaler)
    assert torch.equal(out16, out32)
    scaler.unscale_(opt)
    grads = [p.grad.detach().clone() for p in model.parameters()]
    for (name, _), a, b in zip(model.named_parameters(), grads, grads32[1:]):
        assert torch.allclose(a, b, rtol=1e-6, atol=0.0), name
    scale = scaler.get_scale()
    scaler.step(opt)
    scaler.update()
    assert scaler.get_scale() == scale  # no inf/NaN gradient was found
