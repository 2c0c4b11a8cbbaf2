"""GPU parity of the measured-codebook kernels (isa_ekv_measured_forward/backward) and the
DeploymentAwareCIMLinear / fused_measured_forward drop-ins against oracle/measured.py
(per-cell fp32 terms, float64 sums; pinned against the reference's masked-GEMM
formulation in test_oracle_measured.py). Gates: forward <= 1e-4, dX <= 1e-3 norm-wise."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import measured, oracle
from tests.helpers import flash_cfg, make_codebook

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-4
BWD_TOL = 1e-3


def _err(got, want):
    return oracle.normwise_error(got.detach().double().cpu().numpy(), want)


def _case(M, K, O, n_states, n_points, seed, uniform, pair=False, x_lo=-0.3, x_hi=4.3):
    vg, cur = make_codebook(n_states, n_points, seed=seed, uniform=uniform)
    g = torch.Generator().manual_seed(seed + 100)
    x = torch.rand(M, K, generator=g) * (x_hi - x_lo) + x_lo
    ids_a = torch.randint(0, n_states * n_states if pair else n_states, (O, K), generator=g).to(torch.int16)
    ids_b = None if pair else torch.randint(0, n_states, (O, K), generator=g).to(torch.int16)
    grad = torch.randn(M, O, generator=g)
    return vg, cur, x, ids_a, ids_b, grad


def _run(dev, x, ids_a, ids_b, slopes, intercepts, seg_mode, vg=None, vmin=0.0, inv=1.0, lookup=(0.0, 4.0),
         scale=1.0, r=1e6, grad=None):
    from isa.kernels.transformer_ffn import ops

    rt = torch.full((1,), float(r), device=dev)
    kw = dict(seg_mode=seg_mode, vg=None if vg is None else vg.to(dev), voltage_min=vmin, inverse_step=inv,
              lookup_min=lookup[0], lookup_max=lookup[1], current_scale=scale, r_tia=rt)
    xd = x.to(dev)
    a = ids_a.to(dev)
    b = None if ids_b is None else ids_b.to(dev)
    out, pre = ops.measured_forward(xd, a, b, slopes.to(dev), intercepts.to(dev), **kw)
    gx = None
    if grad is not None:
        gx = ops.measured_backward(xd, a, b, slopes.to(dev), intercepts.to(dev), grad.to(dev), pre, **kw)
    torch.cuda.synchronize()
    return out, pre, gx


CASES = [
    # M, K, O, states, points, uniform grid, segment mode
    (1, 1, 1, 24, 61, True, "search"),
    (17, 27, 13, 24, 61, False, "search"),
    (70, 129, 300, 24, 61, True, "uniform"),
    (64, 192, 768, 24, 61, False, "search"),
    (33, 96, 260, 3000, 61, True, "search"),  # 1.4 MB codebook: global-memory gathers
]


@pytest.mark.parametrize("M,K,O,S,V,uniform,mode", CASES)
def test_measured_member_parity(cuda_device, M, K, O, S, V, uniform, mode):
    from isa.kernels.transformer_ffn import _hip

    print(f"[case] measured M={M} K={K} O={O} states={S} points={V} uniform={uniform} mode={mode}", flush=True)
    vg, cur, x, ids_a, ids_b, grad = _case(M, K, O, S, V, seed=M + K, uniform=uniform)
    s, c = measured.curve_tables(vg.numpy(), cur.numpy())
    v = measured.clamp_input(x.numpy(), 0.0, 4.0)
    if mode == "search":
        seg = measured.segments_search(v, vg.numpy())
        kw = dict(seg_mode=_hip.SEG_SEARCH, vg=vg)
    else:
        inv = 1.0 / float(vg[1] - vg[0])
        seg = measured.segments_uniform(v, float(vg[0]), inv, V - 1)
        kw = dict(seg_mode=_hip.SEG_UNIFORM, vmin=float(vg[0]), inv=inv)
    out, pre, gx = _run(cuda_device, x, ids_a, ids_b, torch.from_numpy(s), torch.from_numpy(c), grad=grad, **kw)
    ref_out, ref_pre = measured.forward(v, seg, ids_a.numpy(), ids_b.numpy(), s, c, 1.0, 1e6, -4.0, 4.0)
    ref_dx = measured.grad_x(x.numpy(), v, seg, ids_a.numpy(), ids_b.numpy(), s, grad.numpy(), ref_pre, 1.0, 1e6,
                             -4.0, 4.0, 0.0, 4.0)
    e = (_err(out, ref_out), _err(pre, ref_pre), _err(gx, ref_dx))
    print(f"fwd {e[0]:.2e} pre {e[1]:.2e} dX {e[2]:.2e}")
    assert e[0] <= FWD_TOL and e[1] <= FWD_TOL and e[2] <= BWD_TOL


def test_fused_measured_forward_pair_and_member(cuda_device):
    """fused_measured_forward (measured_lut_triton.py:159-267): pair mode over the 24x24
    difference curves (as fused_backend.py builds them) equals member mode, and both match
    the oracle; tensor and float r_tia agree."""
    from isa.measured_deployment.kernels.measured_lut_triton import fused_measured_forward

    vg, cur = make_codebook(24, 61, seed=9)
    s, c = measured.curve_tables(vg.numpy(), cur.numpy())
    st, ct = torch.from_numpy(s), torch.from_numpy(c)
    pair_s = (st[:, None, :] - st[None, :, :]).reshape(24 * 24, -1).contiguous()
    pair_c = (ct[:, None, :] - ct[None, :, :]).reshape(24 * 24, -1).contiguous()
    g = torch.Generator().manual_seed(10)
    B, N, K, O = 2, 9, 40, 70
    x = torch.rand(B, N, K, generator=g) * 4.4 - 0.2
    pos = torch.randint(0, 24, (O, K), generator=g)
    neg = torch.randint(0, 24, (O, K), generator=g)
    dev = cuda_device
    kw = dict(lookup_min=0.0, lookup_max=4.0, current_scale=1.0, signed_min=-4.0, signed_max=4.0)
    member = fused_measured_forward(x.to(dev), pos.to(torch.int16).to(dev), st.to(dev), ct.to(dev), vg.to(dev),
                                    assignment_b=neg.to(torch.int16).to(dev), pair_mode=False, r_tia=1e6, **kw)
    pair_ids = (pos * 24 + neg).to(torch.int16)
    pair = fused_measured_forward(x.to(dev), pair_ids.to(dev), pair_s.to(dev), pair_c.to(dev), vg.to(dev),
                                  pair_mode=True, r_tia=torch.tensor(1e6, device=dev), **kw)
    assert member.shape == (B, N, O)
    assert torch.allclose(member, pair, rtol=0, atol=1e-6 * float(member.abs().max()))
    v = measured.clamp_input(x.reshape(-1, K).numpy(), 0.0, 4.0)
    seg = measured.segments_uniform(v, float(vg[0]), 1.0 / float(vg[1] - vg[0]), 60)
    ref, _ = measured.forward(v, seg, pos.numpy(), neg.numpy(), s, c, 1.0, 1e6, -4.0, 4.0)
    assert _err(member.reshape(-1, O), ref) <= FWD_TOL
    with pytest.raises(ValueError, match="uniform voltage grid"):
        vgn, curn = make_codebook(24, 61, seed=9, uniform=False)
        fused_measured_forward(x.to(dev), pos.to(torch.int16).to(dev), st.to(dev), ct.to(dev), vgn.to(dev),
                               assignment_b=neg.to(torch.int16).to(dev), pair_mode=False, **kw)


def _deployment_layer(dev, K, O, bins=0, seed=11):
    from isa.measured_deployment.operator import DeploymentAwareCIMLinear

    torch.manual_seed(seed)
    layer = DeploymentAwareCIMLinear(K, O, flash_cfg(4096)).to(dev)
    vg, cur = make_codebook(24, 61, seed=seed, uniform=False)
    layer.configure_codebook(vg, cur, vin_lut_bins=bins)
    g = torch.Generator().manual_seed(seed)
    pos = torch.randint(0, 24, (O, K), generator=g)
    neg = torch.randint(0, 24, (O, K), generator=g)
    layer.set_assignment(pos, neg)
    with torch.no_grad():
        layer.r_tia_log_scale.fill_(1.5)  # R_TIA ~ 4.5e5: part of the outputs clamp
    return layer, vg, cur, pos, neg


def test_deployment_layer_measured_mode_forward_backward(cuda_device):
    layer, vg, cur, pos, neg = _deployment_layer(cuda_device, 96, 200)
    layer.set_forward_mode("measured")
    x = (torch.rand(3, 21, 96, device=cuda_device) * 4.6 - 0.3).requires_grad_(True)
    out = layer(x)
    g = torch.randn_like(out)
    out.backward(g)
    r = float(layer.r_tia.detach())
    s, c = layer.curve_slopes.cpu().numpy(), layer.curve_intercepts.cpu().numpy()
    X = x.detach().cpu().numpy().reshape(-1, 96)
    v = measured.clamp_input(X, layer.lookup_min, layer.lookup_max)
    seg = measured.segments_search(v, vg.numpy())
    ref, pre = measured.forward(v, seg, pos.numpy(), neg.numpy(), s, c, 1.0, r, -4.0, 4.0)
    assert np.any(np.abs(ref) == 4.0) and np.any(np.abs(ref) < 4.0)
    assert _err(out.reshape(-1, 200), ref) <= FWD_TOL
    dx = measured.grad_x(X, v, seg, pos.numpy(), neg.numpy(), s, g.cpu().numpy().reshape(-1, 200), pre, 1.0, r,
                         -4.0, 4.0, layer.lookup_min, layer.lookup_max)
    assert _err(x.grad.reshape(-1, 96), dx) <= BWD_TOL
    assert layer.vth_pos.grad is None  # the measured path does not reach the thresholds


def test_deployment_layer_bins_mode(cuda_device):
    layer, vg, cur, pos, neg = _deployment_layer(cuda_device, 48, 64, bins=16, seed=12)
    layer.set_forward_mode("measured")
    x = torch.rand(2, 15, 48, device=cuda_device) * 4.0
    out = layer(x)
    r = float(layer.r_tia.detach())
    X = x.cpu().numpy().reshape(-1, 48)
    v = measured.clamp_input(X, layer.lookup_min, layer.lookup_max)
    seg = measured.segments_round(v, layer.lookup_min, 15 / (layer.lookup_max - layer.lookup_min), 16)
    table_c = layer.curve_intercepts.cpu().numpy()
    ref, _ = measured.forward(v, seg, pos.numpy(), neg.numpy(), np.zeros_like(table_c), table_c, 1.0, r, -4.0, 4.0)
    assert _err(out.reshape(-1, 64), ref) <= FWD_TOL


def test_deployment_layer_modes(cuda_device):
    """continuous == CIMLinear; STE forward == measured, STE backward == continuous."""
    from isa.operators.cim import CIMLinear

    layer, *_ = _deployment_layer(cuda_device, 40, 72, seed=13)
    x = torch.rand(2, 11, 40, device=cuda_device) * 4.0
    plain = CIMLinear(40, 72, layer.cfg).to(cuda_device)
    plain.load_state_dict(layer.state_dict())
    assert torch.equal(layer(x), plain(x))
    layer.set_forward_mode("measured")
    measured_out = layer(x)
    layer.set_forward_mode("ste")
    xs = x.clone().requires_grad_(True)
    ste = layer(xs)
    assert torch.allclose(ste, measured_out, rtol=0, atol=1e-6 * float(measured_out.abs().max()))
    g = torch.randn_like(ste)
    ste.backward(g)
    xc = x.clone().requires_grad_(True)
    plain(xc).backward(g)
    assert torch.equal(xs.grad, xc.grad)
    with pytest.raises(ValueError, match="Unsupported"):
        layer.set_forward_mode("bogus")


def test_nan_input_propagates(cuda_device):
    from isa.kernels.transformer_ffn import _hip

    vg, cur, x, ids_a, ids_b, grad = _case(6, 10, 20, 24, 61, seed=3, uniform=True)
    x[2, 4] = float("nan")
    s, c = measured.curve_tables(vg.numpy(), cur.numpy())
    out, _, _ = _run(cuda_device, x, ids_a, ids_b, torch.from_numpy(s), torch.from_numpy(c), _hip.SEG_SEARCH, vg=vg)
    out = out.cpu()
    assert torch.isnan(out[2]).all() and torch.isfinite(torch.cat([out[:2], out[3:]])).all()
