"""The fused layer's forward and backward captured in a HIP graph (torch.cuda.CUDAGraph) and
replayed: every replay must equal the eager computation on the same inputs, bitwise. The
library decides nothing on the host from tensor values (the table-copy mode is a word the
device computes from the thresholds each call), allocates nothing and clears its
workspaces with fill kernels, so one captured graph serves any thresholds: the replays
below switch between the initial thresholds (one table copy) and thresholds spread over
U[V_TH_MIN, V_TH_MAX] (two copies) in place, with eager work and synchronisations between
replays."""

from __future__ import annotations

import pytest
import torch

from tests.helpers import flash_cfg

pytestmark = pytest.mark.gpu


def _grads(model, x):
    out = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
    out["x"] = x.grad.detach().clone()
    return out


def _eager(model, x, g):
    model.zero_grad(set_to_none=True)
    xi = x.detach().clone().requires_grad_(True)
    out = model(xi)
    out.backward(g)
    torch.cuda.synchronize()
    return out.detach().clone(), _grads(model, xi)


def _set_thresholds(model, cfg, spread: str, seed: int):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("vth_pos") or name.endswith("vth_neg"):
                if spread == "full":
                    v = torch.empty(p.shape).uniform_(float(cfg["V_TH_MIN"]), float(cfg["V_TH_MAX"]), generator=gen)
                else:
                    v = 2.5 + 0.1 * (torch.rand(p.shape, generator=gen) * 2 - 1)
                p.copy_(v.to(p.device))


def _inputs(shape, d_in, scale, gen):
    if scale is None:
        return torch.rand(*shape, d_in, generator=gen) * 4.0
    return torch.randn(*shape, d_in, generator=gen) * scale


def _capture(model, static_x, static_g):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):  # warm-up: tables built and cached, plans settled
            model.zero_grad(set_to_none=True)
            model(static_x.detach().clone().requires_grad_(True)).backward(static_g)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    model.zero_grad(set_to_none=True)
    static_x.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = model(static_x)
        static_out.backward(static_g)
    grads = {n: p.grad for n, p in model.named_parameters() if p.grad is not None}
    grads["x"] = static_x.grad
    return graph, static_out, grads


# torch notes that the parameters' gradient accumulators, created during the warm-up on the
# side stream, now receive gradients on the capture stream; that costs a stream wait only
@pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream does not match")
@pytest.mark.parametrize("kind", ["physical_ffn", "cimlinear"])
def test_graph_replays_equal_eager(cuda_device, kind):
    from isa.operators import cim
    from isa.operators.cim import CIMLinear, PhysicalFFN

    print(f"[case] graph capture {kind}", flush=True)
    assert cim.FUSE_GLUE
    torch.manual_seed(31)
    cfg = flash_cfg(4096)
    if kind == "physical_ffn":
        D, F, shape = 192, 768, (4, 65)
        model = PhysicalFFN(D, F, cfg).to(cuda_device)
        with torch.no_grad():
            model.input_mapping.set_affine(1.1, 0.3)
            model.fc1.r_tia_log_scale.fill_(0.4)
            model.adc_affine_scale.uniform_(0.5, 1.5)
        d_in, d_out = D, D
    else:
        d_in, d_out, shape = 200, 520, (3, 97)
        model = CIMLinear(d_in, d_out, cfg).to(cuda_device)
    # PhysicalFFN maps any activation into [0, 4] V; CIMLinear takes voltages: inputs inside
    # the table's range take the kernels' fast path, where the table copies apply
    scale = 2.0 if kind == "physical_ffn" else None
    x0 = _inputs(shape, d_in, scale, torch.Generator(device="cpu").manual_seed(7)).to(cuda_device).requires_grad_(True)
    g0 = torch.randn(*shape, d_out, device=cuda_device)
    _set_thresholds(model, cfg, "init", 0)
    graph, static_out, static_grads = _capture(model, x0, g0)

    cases = [("init", 1), ("full", 2), ("init", 3), ("full", 4), ("full", 5)]
    for i, (spread, seed) in enumerate(cases):
        _set_thresholds(model, cfg, spread, seed)
        gen = torch.Generator(device="cpu").manual_seed(100 + seed)
        x = _inputs(shape, d_in, scale, gen).to(cuda_device)
        g = torch.randn(*shape, d_out, generator=gen).to(cuda_device)
        want_out, want_grads = _eager(model, x, g)
        with torch.no_grad():
            x0.copy_(x)
            g0.copy_(g)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, want_out), (i, spread)
        assert set(static_grads) == set(want_grads)
        for name, t in static_grads.items():
            assert torch.equal(t, want_grads[name]), (i, spread, name)
        # eager work on the same stream between replays
        _eager(model, x * 0.5, g)
