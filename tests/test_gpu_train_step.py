"""the full Physical GPT-L training step on one GPU (bench.py's harness:
12 layers, d=768, 12 heads, Physical FFN 3072 on the CIM kernels, SDPA attention, vocab
50304, 8 x 1024 tokens, AdamW, then clamp_vth as the reference's language trainer does,
language/train.py:740-760). Two steps must give finite losses and keep every threshold in
[V_TH_MIN, V_TH_MAX]; two models built from the same seed must give bitwise-equal losses and
gradients on their first step (the attention runs on the math SDPA backend here so that the
non-CIM ops are deterministic too; the CIM kernels are deterministic on any backend)."""

from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _first_step(dev):
    import bench

    model, _, step = bench.make_gpt_train(4096, dev, seed=0)
    loss = step()
    torch.cuda.synchronize()
    # AdamW has stepped; keep the gradients of that step
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
    return model, step, float(loss.detach()), grads


def test_gpt_training_step_full_size(cuda_device):
    from torch.nn.attention import SDPBackend, sdpa_kernel

    print("[case] GPT-L training step, 12 layers, 8x1024 tokens", flush=True)
    with sdpa_kernel(SDPBackend.MATH):
        model, step, loss0, grads0 = _first_step(cuda_device)
        before = {n: p.detach().clone() for n, p in model.named_parameters() if "ffn" in n}
        loss1 = float(step().detach())
        torch.cuda.synchronize()
    print(f"losses {loss0:.4f} {loss1:.4f}")
    assert math.isfinite(loss0) and math.isfinite(loss1)
    n_cim = 0
    for name, p in model.named_parameters():
        if "vth" in name:
            # at the random initialisation fc2's inputs sit deep below threshold, so the threshold
            # gradients are ~1e-12: nonzero and finite, though AdamW's eps keeps their update
            # below an fp32 ulp of the thresholds
            n_cim += 1
            assert float(p.min()) >= 0.0 and float(p.max()) <= 5.0, name
            assert torch.isfinite(grads0[name]).all(), name
            assert int(torch.count_nonzero(grads0[name])) > 0, name
        if "adc_affine_shift" in name:  # O(0.1) gradients: the optimizer visibly steps the FFNs
            assert not torch.equal(p.detach(), before[name]), f"{name} did not move"
    assert n_cim == 12 * 2 * 2  # fc1/fc2 x vth_pos/vth_neg x 12 blocks
    del model
    torch.cuda.empty_cache()
    with sdpa_kernel(SDPBackend.MATH):
        model2, _, loss0b, grads0b = _first_step(cuda_device)
    assert loss0b == loss0
    assert grads0.keys() == grads0b.keys()
    differ = [n for n in grads0 if not torch.equal(grads0[n], grads0b[n])]
    assert not differ, differ[:8]
