"""Benchmark: Flash-EKV LUT CIMLinear cell-evals/s, fwd+bwd, Physical GPT-L FFN, 1 GPU.

A step is one forward and backward pass of the drop-in `PhysicalFFN` (VoltageMapping ->
CIMLinear 768->3072 -> CIMLinear 3072->768 -> ADC affine) over one batch X[8, 1024, 768]
~ N(0, 1) with an N(0, 1) upstream gradient, fp32, 4096-entry LUT, random-init
thresholds U(2.5 +- 0.5*2nU_T) (the reference's CIMLinear initialisation). Inputs and
parameters are resident in HBM before timing starts.

value = cell-evals per second over the timed steps, counting M*K*O cells per CIM layer
in the forward and again in the backward; the timed steps carry no instrumentation.
`roofline` reports the dominant kernel (the backward main kernel) against the VALU
lane-instruction peak, from HIP events the library records around each launch on its own
stream in a second pass of the same steps; `cpu_baseline` times the reference's
PyTorch CPU path (exact formula, chunked over 64 outputs, analytic backward) restated in
oracle/exact.py, on a bounded token sample of fc1.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT / "isa-_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

# gfx950 VALU issue peak: 256 CUs x 64 lanes x 2.4 GHz (lane-instructions per second)
VALU_PEAK = 256 * 64 * 2.4e9
# lane-instructions per cell-eval (forward, backward). LUT path: the algorithmic count of
# the interpolated lookup formulation. Exact path: the issued count of the exact kernels'
# range-checked inner loops (4 log2 per cell forward; 4 log2 + 4 rcp backward, each with
# the rounding correction of log2(1 + e)), so its fraction measures issue efficiency.
INSTR_PER_CELL = {"lut": (12, 16), "exact": (32, 52)}
# measured-codebook path (member mode): issued lane-instructions per cell of the forward
# and dX inner loops (forward: two id-offset adds, the slope and intercept differences, fma,
# accumulate; dX: slope gathers only)
MEASURED_INSTR_PER_CELL = (6, 8)

CONFIGS = {
    # name: (batch, tokens, d_model, d_ffn, physical fc2)
    "gptl_ffn": (8, 1024, 768, 3072, True),     # configs[3], the headline
    "vitm_ffn": (128, 65, 256, 1024, True),     # configs[1]
    "gptm_hybrid": (16, 1024, 384, 1536, False),  # configs[2]
    "vits_up": (8, 65, 192, 768, None),          # configs[0]: one CIMLinear
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_info() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                fields[k.strip()] = v.strip()
        return f"{fields.get('Model name', platform.processor())}; sockets {fields.get('Socket(s)', '?')}, " \
               f"cores/socket {fields.get('Core(s) per socket', '?')}"
    except Exception:
        return platform.processor() or "unknown"


CPU_BATCH_TOKENS = 128


def cpu_baseline(layers, target_s: float) -> dict:
    """The reference's PyTorch CPU path (exact formula, cim.py:201-214 + flash_transistor.py:95-131),
    restated in oracle/exact.py, fwd+bwd on a token sample of every CIM layer of the workload
    (K -> O pairs; about target_s / len(layers) seconds each). fc1 takes mapped inputs
    clamp(N(0,1), 0, 4), a later layer signed TIA outputs clamp(N(0,1), -4, 4)."""
    import torch

    from oracle import exact, oracle

    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    torch.set_num_threads(threads)
    cfg = dict(oracle.FLASH_PARAMS)
    g = torch.Generator().manual_seed(0)
    lo, hi = 2.5 - 0.5 * 2 * cfg["n"] * cfg["U_T"], 2.5 + 0.5 * 2 * cfg["n"] * cfg["U_T"]
    total_cells, total_s, parts = 0.0, 0.0, []
    for idx, (k_in, o_out) in enumerate(layers):
        vp = torch.empty(o_out, k_in).uniform_(lo, hi, generator=g).requires_grad_(True)
        vn = torch.empty(o_out, k_in).uniform_(lo, hi, generator=g).requires_grad_(True)
        x_lo = 0.0 if idx == 0 else -4.0

        def run(tokens: int) -> float:
            x = torch.randn(1, tokens, k_in, generator=g).clamp(x_lo, 4.0).requires_grad_(True)
            gr = torch.randn(1, tokens, o_out, generator=g)
            t0 = time.perf_counter()
            out = exact.cim_idiff_cpu(x, vp, vn, cfg)
            out.backward(gr)
            return time.perf_counter() - t0

        run(2)  # warm-up
        # 128-token batches until this layer's share of the CPU time budget is spent (at least
        # one): the reference path's per-token cost grows with its batch's temporaries (~6x
        # from 32 to 736 tokens at fc1), so the batch is fixed and the count bounded by time
        want, dt = 0, 0.0
        while want == 0 or dt < target_s / len(layers):
            dt += run(CPU_BATCH_TOKENS)
            want += CPU_BATCH_TOKENS
        cells = 2.0 * want * k_in * o_out
        total_cells += cells
        total_s += dt
        parts.append(f"{k_in}->{o_out} on {want} tokens in batches of {CPU_BATCH_TOKENS} ({cells:.3e} "
                     f"cell-evals, {dt:.1f} s, {cells / dt:.3e}/s)")
    return {
        "value": total_cells / total_s,
        "unit": "cell-evals/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": "reference CPU path (exact EKV formula, chunked over 64 outputs, analytic backward) restated "
                  "in oracle/exact.py, fwd+bwd, every CIM layer on a token sample: " + "; ".join(parts)
                  + f"; total {total_cells:.3e} cell-evals in {total_s:.1f} s; host {cpu_info()}, "
                  f"os.cpu_count()={os.cpu_count()}",
    }


def cpu_lut_oracle(d_model: int, d_ffn: int, target_s: float) -> dict:
    """For information: the CPU LUT oracle (oracle/ekv_oracle.c: OpenMP over rows, fp32 cells
    with double sums) timed on fc1 fwd+bwd over a token sample sized to about target_s seconds."""
    import numpy as np

    from oracle import oracle

    cfg = dict(oracle.FLASH_PARAMS)
    cfg["LUT_DELTA_SIZE"] = 4096
    dmin, dmax, _ = oracle.lut_range(cfg)
    ti, td = oracle.lut_tables(cfg)
    rng = np.random.default_rng(0)
    lo, hi = 2.5 - 0.5 * 2 * cfg["n"] * cfg["U_T"], 2.5 + 0.5 * 2 * cfg["n"] * cfg["U_T"]
    vp = rng.uniform(lo, hi, (d_ffn, d_model)).astype(np.float32)
    vn = rng.uniform(lo, hi, (d_ffn, d_model)).astype(np.float32)

    def run(tokens: int) -> float:
        x = np.clip(rng.standard_normal((tokens, d_model)), 0.0, 4.0).astype(np.float32)
        g = rng.standard_normal((tokens, d_ffn)).astype(np.float32)
        t0 = time.perf_counter()
        oracle.forward(x, vp, vn, ti, dmin, dmax, cfg["V_sat"])
        oracle.backward(x, vp, vn, g, ti, td, dmin, dmax, cfg["V_sat"])
        return time.perf_counter() - t0

    run(1)  # warm-up
    dt = run(8)
    want = max(1, min(1024, int(8 * target_s / max(dt, 1e-4))))
    dt = run(want)
    cells = 2.0 * want * d_model * d_ffn
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": cells / dt, "unit": "cell-evals/s", "cores": threads, "kind": "oracle (LUT, C, OpenMP)",
            "sample": f"oracle/ekv_oracle.c LUT forward + dX + dVth, fc1 {d_model}->{d_ffn} on {want} tokens "
                      f"({cells:.3e} cell-evals, {dt:.1f} s)"}


def measured_traffic(config: str):
    """(HBM bytes per backward main-kernel launch, source, per-layer measured and algorithmic
    bytes) from the committed rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, calibrated on
    a plain copy kernel), or (None, None, None): the counters need a rocprofv3 --pmc run of
    their own, so this run does not measure them."""
    path = ROOT / "profiles" / f"bwd_kernel_{config}_hbm_traffic.txt"
    total, fields = None, {}
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                total = float(line.split(":", 1)[1])
            elif line.startswith(("traffic_fc", "algorithmic_fc")):
                key, val = line.split(":", 1)
                fields[key.strip()] = float(val)
    except OSError:
        return None, None, None
    layers = {}
    for layer in ("fc1", "fc2"):
        t, a = fields.get(f"traffic_{layer}_bytes"), fields.get(f"algorithmic_{layer}_bytes")
        if t and a:
            layers[layer] = {"measured_bytes": t, "algorithmic_bytes": a, "ratio": round(t / a, 2)}
    src = f"profiles/{path.name} (rocprofv3 --pmc, not this run)" if total else None
    return total, src, layers or None


def issued_valu_per_cell() -> dict:
    """Issued VALU lane-instructions per cell-eval of each LUT main kernel, from the committed
    rocprofv3 SQ_INSTS_VALU summary (lines "valu_per_cell <kernel>: <value>"): the counters
    need a rocprofv3 --pmc run of their own, so this run does not measure them."""
    path = ROOT / "profiles" / "counters_gptl_ffn_bench.md"
    out = {}
    try:
        for line in path.read_text().splitlines():
            if line.startswith("valu_per_cell "):
                name, val = line[len("valu_per_cell "):].split(":", 1)
                out[name.strip()] = float(val)
    except OSError:
        pass
    return out


def measured_ceiling(kt, cells_launch: float, fwd_ms: float, bwd_ms: float, dev) -> dict:
    """Each LUT main kernel against the VALU issue rate it can reach on this GPU: the issued
    VALU wave-instructions of one launch (committed SQ_INSTS_VALU per cell x cells / 64) over
    (the register-only replay's wave-instructions per CU-cycle for the kernel's mix x CUs x the
    shader clock the kernel's own blocks ran at during the timed steps, clock64 / wall_clock64)
    gives the launch time if VALU issue were its only limit; frac = that / the measured launch
    time, at most 1. The replay (isa_ekv_probe_valu_issue) runs after the timed steps."""
    import torch

    from isa.kernels.transformer_ffn import ops

    per_cell = issued_valu_per_cell()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    probes = {mix: ops.probe_valu_issue(mix, device=dev) for mix in ("fma", "forward", "ranked_backward")}
    bwd_name = max(("bwd_kernel", "bwd_two_copies_kernel", "bwd_ranked_kernel"),
                   key=lambda n: kt.clocks[n]["block_seconds"])

    def one(name: str, avg_ms: float, mix: str) -> dict:
        clk = kt.clocks[name]
        ghz, n = clk["ghz"], per_cell.get(name)
        res = {"kernel": name, "kernel_ghz": round(ghz, 4) if ghz else None, "issued_valu_per_cell": n,
               "replay_mix": mix, "replay_instr_per_cu_cycle": round(probes[mix]["instr_per_cu_cycle"], 4),
               "avg_launch_ms": round(avg_ms, 4),
               # a block's first wave from entry to exit, averaged over every block of the timed
               # launches: against avg_launch_ms it shows how much of a one-round launch (small
               # calls) lies outside its blocks, in the dispatch of their start and the drain
               "mean_block_lifetime_ms": round(clk["block_seconds"] / clk["blocks"] * 1e3, 5)
               if clk["blocks"] else None}
        if ghz and n and avg_ms:
            wave_instr = n * cells_launch / 64.0
            ceiling_ms = wave_instr / (probes[mix]["instr_per_cu_cycle"] * cus * ghz * 1e9) * 1e3
            res.update(ceiling_ms=round(ceiling_ms, 4), frac=round(ceiling_ms / avg_ms, 4),
                       issue_rate_instr_per_cu_cycle=round(wave_instr / (cus * ghz * 1e9 * avg_ms * 1e-3), 4))
        return res

    return {
        "bound": "valu issue, measured",
        "backward": one(bwd_name, bwd_ms, "ranked_backward"),
        "forward": one("fwd_kernel", fwd_ms, "forward"),
        "fma_issue_instr_per_cu_cycle": round(probes["fma"]["instr_per_cu_cycle"], 4),
        "replay_ghz": {m: round(p.get("ghz", 0.0), 4) for m, p in probes.items()},
        "source": "issued_valu_per_cell: profiles/counters_gptl_ffn_bench.md (rocprofv3 SQ_INSTS_VALU, not this "
                  "run); kernel_ghz: clock64 / wall_clock64 of every block of the kernel during the timed steps "
                  "(isa_ekv_profile_clock), mean_block_lifetime_ms: the same blocks' wall time each; replay: isa_ekv_probe_valu_issue after the timed steps (the kernel's "
                  "VALU mix on registers only, at its occupancy; the one- and two-copy backwards are priced "
                  "with the ranked backward's mix)",
    }


def measured_fc1_step(args) -> int:
    """The measured-codebook deployment of a Physical ViT-S fc1 (192 -> 768, measured
    mode, forward and dX) over X[128, 65, 192] with a synthetic 24-state, 61-point codebook
    (the FG50 centre-codebook shape). A step is one forward and backward; cell-evals count
    M*K*O per pass as for the LUT path. Reports the measured kernels' HIP-event times."""
    import torch

    from isa.device_models.config import make_flash_transistor_ekv_config
    from isa.kernels.transformer_ffn import _hip
    from isa.measured_deployment.operator import DeploymentAwareCIMLinear

    dev = torch.device("cuda", 0)
    B, T, D, F = 128, 65, 192, 768
    M = B * T
    cfg = make_flash_transistor_ekv_config(default_lut_size=args.lut_size)
    torch.manual_seed(0)
    layer = DeploymentAwareCIMLinear(D, F, cfg).to(dev)
    vg = torch.linspace(0.0, 4.0, 61)
    vt = torch.linspace(0.4, 3.6, 24)
    sp = torch.nn.functional.softplus((vg[None, :] - vt[:, None]) / 0.1)
    layer.configure_codebook(vg, 2e-9 * sp * sp + 4e-10)
    layer.set_assignment(torch.randint(0, 24, (F, D)), torch.randint(0, 24, (F, D)))
    layer.set_forward_mode("measured")
    x = (torch.randn(B, T, D, device=dev).clamp(0.0, 4.0)).requires_grad_(True)
    g = torch.randn(B, T, F, device=dev)

    def step():
        x.grad = None
        layer(x).backward(g)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()  # the value: uninstrumented steps
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    with _hip.KernelTimer() as kt:  # per-kernel launch times: the same steps, instrumented
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    cells = float(M * D * F)
    value = 2.0 * cells / (ms * 1e-3)
    fwd_avg = kt.fwd_ms / max(kt.fwd_launches, 1)
    bwd_avg = kt.bwd_ms / max(kt.bwd_launches, 1)
    instr_f, instr_b = MEASURED_INSTR_PER_CELL
    result = {
        "metric": "measured-codebook CIM cell-evals/sec fwd+dX, ViT-S fc1, 1 GPU",
        "value": value,
        "unit": "cell-evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (24-state 61-point codebook, random assignment)",
        "config": {"workload": "DeploymentAwareCIMLinear 192->768 measured mode, X[128,65,192], fwd+dX",
                   "tokens": M, "parallelism": "single GPU"},
        "roofline": {
            "bound": "valu", "unit": "TOP/s", "peak": round(VALU_PEAK / 1e12, 3),
            "kernel": "bwd_measured_kernel (dX)", "avg_launch_ms": round(bwd_avg, 4),
            "achieved": round(cells * instr_b / (bwd_avg * 1e-3) / 1e12, 3),
            "frac": round(cells * instr_b / (bwd_avg * 1e-3) / VALU_PEAK, 4),
            "work": f"{instr_b} VALU lane-instr per cell x {cells:.4e} cells per launch",
            "forward_kernel": {"kernel": "fwd_measured_kernel", "avg_launch_ms": round(fwd_avg, 4),
                               "frac": round(cells * instr_f / (fwd_avg * 1e-3) / VALU_PEAK, 4)},
            "traffic": None,
        },
        "cpu_baseline": None,
    }
    log(f"[bench] measured fc1: {ms:.3f} ms/step, fwd {fwd_avg:.3f} ms, dX {bwd_avg:.3f} ms")
    print(json.dumps(result), flush=True)
    return 0


GPT_SHAPE = dict(n_layer=12, n_head=12, d=768, d_ffn=3072, vocab=50304, B=8, T=1024)


def make_gpt_train(lut_size: int, dev, seed: int = 0):
    """configs[4]'s model and step: a GPT (12 layers, d=768, 12 heads, Physical FFN 3072 on the
    HIP kernels, causal SDPA attention, vocab 50304 tied embeddings) on 8 x 1024 uniform random
    token ids, AdamW, then the thresholds clamped to [V_TH_MIN, V_TH_MAX] as the reference's
    language trainer does. Returns (model, optimizer, step); step() runs one training step and
    returns the loss tensor."""
    import torch
    import torch.nn as nn
    import torch.nn.functional as F

    from isa.device_models.config import make_flash_transistor_ekv_config
    from isa.operators.cim import PhysicalFFN

    n_layer, n_head, d, d_ffn, vocab, B, T = (GPT_SHAPE[k] for k in ("n_layer", "n_head", "d", "d_ffn", "vocab",
                                                                     "B", "T"))
    cfg = make_flash_transistor_ekv_config(default_lut_size=lut_size)
    cfg["LUT_DELTA_SIZE"] = lut_size

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.ln1 = nn.LayerNorm(d)
            self.qkv = nn.Linear(d, 3 * d)
            self.proj = nn.Linear(d, d)
            self.ln2 = nn.LayerNorm(d)
            self.ffn = PhysicalFFN(d, d_ffn, cfg)

        def forward(self, x):
            b, t, _ = x.shape
            q, k, v = self.qkv(self.ln1(x)).view(b, t, 3, n_head, d // n_head).unbind(dim=2)
            a = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                               is_causal=True)
            x = x + self.proj(a.transpose(1, 2).reshape(b, t, d))
            return x + self.ffn(self.ln2(x))

    class GPT(nn.Module):
        def __init__(self):
            super().__init__()
            self.tok = nn.Embedding(vocab, d)
            self.pos = nn.Embedding(T, d)
            self.blocks = nn.ModuleList(Block() for _ in range(n_layer))
            self.ln_f = nn.LayerNorm(d)
            self.head = nn.Linear(d, vocab, bias=False)
            self.head.weight = self.tok.weight

        def forward(self, ids):
            x = self.tok(ids) + self.pos(torch.arange(ids.shape[1], device=ids.device))[None]
            for blk in self.blocks:
                x = blk(x)
            return self.head(self.ln_f(x))

    torch.manual_seed(seed)
    model = GPT().to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, weight_decay=0.0)
    ids = torch.randint(0, vocab, (B, T + 1), device=dev)
    inp, tgt = ids[:, :-1].contiguous(), ids[:, 1:].contiguous()
    ffns = [blk.ffn for blk in model.blocks]

    def step():
        opt.zero_grad(set_to_none=True)
        logits = model(inp)
        loss = F.cross_entropy(logits.view(-1, vocab), tgt.view(-1))
        loss.backward()
        opt.step()
        for f in ffns:
            f.clamp_vth()
        return loss

    return model, opt, step


def gpt_train_step(args) -> int:
    """GPT training steps on make_gpt_train's model. Reports tokens/s and the share
    of step time spent in the CIM library calls."""
    import torch

    from isa.kernels.transformer_ffn import _hip

    dev = torch.device("cuda", 0)
    n_layer, d, d_ffn, vocab, B, T = (GPT_SHAPE[k] for k in ("n_layer", "d", "d_ffn", "vocab", "B", "T"))
    model, opt, step = make_gpt_train(args.lut_size, dev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()  # the value: uninstrumented steps
    for _ in range(args.steps):
        loss = step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    with _hip.KernelTimer() as kt:  # the library calls' share: the same steps, instrumented
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    cim_ms = (kt.fwd_call_ms + kt.bwd_call_ms) / args.steps
    main_ms = (kt.fwd_ms + kt.bwd_ms) / args.steps
    cells = 2.0 * n_layer * 2 * (B * T) * d * d_ffn
    result = {
        "metric": "GPT-L training step tokens/s, 1 GPU (Physical FFN on the CIM kernels); FFN share of step time",
        "value": B * T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "GPT 12 layers, d=768, 12 heads, Physical FFN 3072, vocab 50304, 8x1024 tokens, AdamW",
                   "lut_entries": args.lut_size, "parallelism": "single GPU"},
        "ffn": {"cim_call_ms_per_step": cim_ms, "cim_main_kernels_ms_per_step": main_ms,
                "cim_share_of_step": cim_ms / ms, "cell_evals_per_step": cells,
                "cim_cell_evals_per_s": cells / (cim_ms * 1e-3), "final_loss": float(loss.detach())},
    }
    print(json.dumps(result), flush=True)
    return 0


def _smi_snapshot() -> dict:
    """The board's firmware counters from `rocm-smi -a --json`: energy accumulator, its clock,
    and the power-limit (PPT) and thermal residency counters."""
    out = subprocess.run(["rocm-smi", "-a", "--json"], capture_output=True, text=True, timeout=30).stdout
    card = json.loads(out)["card0"]
    num = lambda key: float(card[key])
    return {"energy_j": num("energy_accumulator (15.259uJ (2^-16))") * 15.259e-6,
            "ns": num("system_clock_counter (ns)"), "ppt": num("ppt_residency_acc (Count)"),
            "thm": num("socket_thm_residency_acc (Count)"), "acc": num("accumulation_counter (Count)"),
            "cap_w": card.get("Max Graphics Package Power (W)"), "gfxclk_mhz": card.get("current_gfxclks (MHz)")}


def board_power(step, seconds: float) -> dict:
    """Mean board power and power-limit residency while `step` runs back to back for `seconds`:
    two snapshots of the firmware counters taken from a second thread 1 s into the loop and
    0.5 s before its end, so that both fall inside the run."""
    import threading

    import torch

    snaps, errors = [], []

    def take():
        try:
            time.sleep(1.0)
            snaps.append(_smi_snapshot())
            time.sleep(max(0.5, seconds - 2.0))
            # the firmware refreshes its counters periodically: read again (a few times at most)
            # until its clock has moved on by half a second
            for _ in range(8):
                last = _smi_snapshot()
                if last["ns"] - snaps[0]["ns"] >= 0.5e9:
                    break
                time.sleep(0.5)
            snaps.append(last)
        except Exception as e:  # rocm-smi absent or its output without these fields
            errors.append(repr(e))

    th = threading.Thread(target=take, daemon=True)
    th.start()
    t0 = time.perf_counter()
    steps = 0
    while time.perf_counter() - t0 < seconds or th.is_alive():
        step()
        steps += 1
        if steps % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    th.join()
    if errors or len(snaps) != 2:
        return {"error": errors[0] if errors else "no snapshots"}
    a, b = snaps
    dt = (b["ns"] - a["ns"]) * 1e-9
    if dt <= 0.0:
        return {"error": "the firmware counters did not advance between the snapshots"}
    ticks = max(1.0, b["acc"] - a["acc"])
    return {"watts": round((b["energy_j"] - a["energy_j"]) / dt, 1), "interval_s": round(dt, 3),
            "ppt_residency": round((b["ppt"] - a["ppt"]) / ticks, 4),
            "thermal_residency": round((b["thm"] - a["thm"]) / ticks, 4),
            "cap_watts": b["cap_w"], "gfxclk_mhz_per_xcd": b["gfxclk_mhz"], "steps": steps,
            "source": "rocm-smi -a --json energy accumulator and PPT residency counters, two snapshots inside a "
                      f"{seconds:.0f} s loop of the step after the timed region"}


def power_phases(cfg: dict, d_model: int, d_ffn: int, tokens: int, dev, seconds: float) -> dict:
    """board_power for one kernel family at a time: the first CIM layer's table backward and
    table forward through the library's ops (the workload's fc1 shapes, mapped inputs
    clamp(N(0,1), 0, 4), the reference's initial thresholds), the register-only VALU replay of
    independent fmas, and the LDS gather probe at the thresholds' window; then the idle board."""
    import torch

    from isa.approximations.delta_lut import get_packed_tables, lut_range
    from isa.kernels.transformer_ffn import ops

    dmin, dmax, n = lut_range(cfg)
    fwd_t, bwd_t = get_packed_tables(cfg, dev)
    g = torch.Generator().manual_seed(0)
    lo = 2.5 - 0.5 * 2 * cfg["n"] * cfg["U_T"]
    hi = 2.5 + 0.5 * 2 * cfg["n"] * cfg["U_T"]
    x = torch.randn(tokens, d_model, generator=g).clamp(0.0, 4.0).to(dev)
    vp = torch.empty(d_ffn, d_model).uniform_(lo, hi, generator=g).to(dev)
    vn = torch.empty(d_ffn, d_model).uniform_(lo, hi, generator=g).to(dev)
    grad = torch.randn(tokens, d_ffn, generator=g).to(dev)
    pf = ops.plan_info("forward", tokens, d_model, d_ffn, n)
    pb = ops.plan_info("backward", tokens, d_model, d_ffn, n, True, True)
    wsf = torch.empty(pf["workspace_bytes"], dtype=torch.uint8, device=dev)
    wsb = torch.empty(pb["workspace_bytes"], dtype=torch.uint8, device=dev)
    phases = {
        "table_backward": lambda: ops.lut_backward(x, vp, vn, grad, bwd_t, n, dmin, dmax, cfg["V_sat"], True, True,
                                                   workspace=wsb),
        "table_forward": lambda: ops.lut_forward(x, vp, vn, fwd_t, n, dmin, dmax, cfg["V_sat"], -4.0, 4.0,
                                                 workspace=wsf),
        "valu_replay_fma": lambda: ops.probe_valu_issue("fma", iterations=16384, device=dev, repeats=1),
        "lds_gather_probe": lambda: ops.probe_lds_gather(69, 8, iterations=8192, device=dev, repeats=1),
        "idle": lambda: time.sleep(0.05),
    }
    out = {"workload": f"fc1 {tokens} x {d_model} -> {d_ffn}, mapped inputs, initial thresholds"}
    for name, fn in phases.items():
        fn()
        torch.cuda.synchronize()
        out[name] = board_power(fn, seconds)
        log(f"[bench] board power, {name}: {out[name]}")
    return out


def lds_roofline(model, cfg: dict, cells_launch: float, fwd_ms: float, bwd_ms: float, dev) -> dict:
    """The table kernels' second bound: their LDS gathers. Each cell-eval gathers 2 records
    (forward: the + and - branch, ds_read_b64) or 4 (backward: the I and D halves of both
    branches, ds_read_b64 each); the 64 lanes of a gather share the token and input, so
    their indices spread over the window the thresholds of the wave's outputs span,
    (max - min of vth) / LUT step records. isa_ekv_probe_lds_gather measures the time per
    random b64 gather at that window on this GPU (bank conflicts included), which gives
    the LDS-bound launch times of a kernel that reads one table copy with the lanes in
    output order. The kernels beat that rate where they spread a gather over the banks (the
    forward's windowed table copies, the ranked backward), so those fractions can pass 1;
    the conflict-free rate (one record per bank pair) bounds both."""
    import math

    import torch

    from isa.approximations.delta_lut import lut_range
    from isa.kernels.transformer_ffn import ops

    dmin, dmax, n = lut_range(cfg)
    step = (dmax - dmin) / (n - 1)
    spans = []
    for name, p in model.named_parameters():
        if name.endswith("vth_pos") or name.endswith("vth_neg"):
            spans.append(float(p.detach().max() - p.detach().min()))
    window = max(1, min(8192, int(math.ceil(max(spans) / step)) + 1))
    clock = {}
    ns = ops.probe_lds_gather(window, 8, device=dev, clock=clock)
    ns_free = ops.probe_lds_gather(32, 8, device=dev)  # one record per bank pair: no conflicts
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    waves_per_launch = cells_launch / 64.0
    fwd_roof = 2 * waves_per_launch * ns / cus * 1e-6  # ms
    bwd_roof = 4 * waves_per_launch * ns / cus * 1e-6
    fwd_free = 2 * waves_per_launch * ns_free / cus * 1e-6
    bwd_free = 4 * waves_per_launch * ns_free / cus * 1e-6
    return {
        "bound": "lds",
        "window_records": window,
        "ns_per_gather_per_cu": round(ns, 4),
        "forward_roof_ms": round(fwd_roof, 4),
        "forward_frac": round(fwd_roof / fwd_ms, 4) if fwd_ms else None,
        "backward_roof_ms": round(bwd_roof, 4),
        "backward_frac": round(bwd_roof / bwd_ms, 4) if bwd_ms else None,
        "conflict_free_ns_per_gather_per_cu": round(ns_free, 4),
        "conflict_free_frac": {"forward": round(fwd_free / fwd_ms, 4) if fwd_ms else None,
                               "backward": round(bwd_free / bwd_ms, 4) if bwd_ms else None},
        "work": "forward 2, backward 4 random ds_read_b64 gathers per cell-eval (wave-level: per 64 cells); "
                "forward/backward_frac price them at the one-copy random rate of the window (the windowed "
                "forward copies and the ranked backward conflict less, so these can pass 1); "
                "conflict_free_frac prices them at the probe's W = 32 rate (one record per bank pair)",
        "_clock": clock,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="gptl_ffn", choices=sorted(CONFIGS) + ["gptl_train", "measured_fc1"])
    ap.add_argument("--lut-size", type=int, default=4096)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ekv-approx", default="lut", choices=["lut", "exact"],
                    help="CIMLinear projection: the LUT kernels (headline) or the exact-formula kernels")
    ap.add_argument("--lut-dtype", default=None, choices=["float32", "bfloat16"],
                    help="LUT table precision (default: the config's, float32); bfloat16 reproduces the "
                         "reference's bf16 tables")
    ap.add_argument("--vth-spread", default="init", choices=["init", "full"],
                    help="thresholds: the reference's initialisation U(2.5 +- 0.5*2nU_T) (headline), or "
                         "U[V_TH_MIN, V_TH_MAX] as a stand-in for trained thresholds (wider table windows)")
    ap.add_argument("--graph", action="store_true",
                    help="time the step as replays of one captured HIP graph (torch.cuda.CUDAGraph): "
                         "no host launch cost; the per-kernel figures come from an eager pass after")
    ap.add_argument("--calling-thread", action="store_true",
                    help="run the backward on the calling thread (torch.autograd.set_multithreading_enabled"
                         "(False)) instead of torch's autograd device thread (its default); the handoff "
                         "between the two threads costs ~40-85 us per eager step")
    ap.add_argument("--no-ranked", action="store_true",
                    help="plan the table backwards without the ranked kernel (isa_ekv_set_option "
                         "ISA_EKV_OPT_RANKED = 0): the one- or two-copy kernel runs instead")
    ap.add_argument("--copy-min-cells", type=int, default=None,
                    help="calls of fewer cells M*K*O plan one table copy and no ranked backward "
                         "(isa_ekv_set_option ISA_EKV_OPT_COPY_MIN_CELLS, default 2^28)")
    ap.add_argument("--window-copies", type=int, default=None,
                    help="the most windowed table copies a LUT forward or the two-copy backward may hold "
                         "(isa_ekv_set_option "
                         "ISA_EKV_OPT_WINDOW_COPIES: 3 to 32, default 32; 0 none)")
    ap.add_argument("--rank-max-spread", type=int, default=None,
                    help="the widest threshold spread (table records) the ranked backward takes "
                         "(isa_ekv_set_option ISA_EKV_OPT_RANK_MAX_SPREAD, default 420)")
    ap.add_argument("--rank-greedy-min", type=int, default=None,
                    help="threshold spreads (table records) past which the ranked backward deals its branches "
                         "greedily by LDS bank instead of by rank (ISA_EKV_OPT_RANK_GREEDY_MIN, default 4128: never)")
    ap.add_argument("--rank-xcd-order", type=int, default=None, choices=[0, 1],
                    help="1: each XCD runs a contiguous range of the ranked backward's blocks "
                         "(ISA_EKV_OPT_RANK_XCD_ORDER); 0: the hardware's round-robin order")
    ap.add_argument("--power-seconds", type=float, default=6.0,
                    help="after timing, run the step back to back this long and report the board's mean power "
                         "and power-limit residency from its firmware counters (board_power; rocm-smi); 0 skips")
    ap.add_argument("--power-phases", type=float, default=0.0,
                    help="after the run, board_power for one kernel family at a time, this many seconds each "
                         "(board_power_phases: table backward, table forward, VALU replay, LDS probe, idle)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="after timing, run one plain device-to-device copy of this many MiB (a reference "
                         "kernel of known HBM traffic for counter runs)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the operator would shard "
              "over tokens with one all-reduce of dVth per layer). Run with --gpus 1.", file=sys.stderr)
        return 2

    if args.calling_thread:
        # The steps run their backward on the calling thread (a documented torch setting that
        # changes no result): for small layers the wake-up of torch's per-device autograd thread
        # and the wait for it cost more host time than the library's launches. By default the
        # value is timed under torch's default threading, and the CIM configs' JSON reports
        # the eager step on the calling thread beside it (host.eager_ms_calling_thread).
        import torch

        torch.autograd.set_multithreading_enabled(False)
    if args.no_ranked:
        from isa.kernels.transformer_ffn import ops

        ops.ranked_backward(False)
    if args.window_copies is not None:
        from isa.kernels.transformer_ffn import ops

        ops.window_copies(args.window_copies)
    if args.copy_min_cells is not None:
        from isa.kernels.transformer_ffn import ops

        ops.copy_min_cells(args.copy_min_cells)
    if args.rank_max_spread is not None:
        from isa.kernels.transformer_ffn import ops

        ops.rank_max_spread(args.rank_max_spread)
    if args.rank_greedy_min is not None:
        from isa.kernels.transformer_ffn import ops

        ops.rank_greedy_min(args.rank_greedy_min)
    if args.rank_xcd_order is not None:
        from isa.kernels.transformer_ffn import ops

        ops.rank_xcd_order(bool(args.rank_xcd_order))
    if args.config == "gptl_train":
        return gpt_train_step(args)
    if args.config == "measured_fc1":
        return measured_fc1_step(args)

    import torch
    import torch.nn as nn

    from isa.device_models.config import make_flash_transistor_ekv_config
    from isa.kernels.transformer_ffn import _hip
    from isa.operators.cim import CIMLinear, HybridFFN, PhysicalFFN

    assert torch.cuda.is_available(), "bench.py needs a ROCm device"
    dev = torch.device("cuda", 0)
    B, T, D, F, physical = CONFIGS[args.config]
    M = B * T
    cfg = make_flash_transistor_ekv_config(default_lut_size=args.lut_size)
    cfg["LUT_DELTA_SIZE"] = args.lut_size
    cfg["ekv_approx"] = args.ekv_approx
    if args.lut_dtype:
        cfg["LUT_DTYPE"] = args.lut_dtype
    fwd_instr, bwd_instr = INSTR_PER_CELL[args.ekv_approx]

    torch.manual_seed(0)
    if physical is True:
        model: nn.Module = PhysicalFFN(D, F, cfg)
        layers = [(M, D, F), (M, F, D)]
    elif physical is False:
        model = HybridFFN(D, F, cfg)
        layers = [(M, D, F)]
    else:
        model = CIMLinear(D, F, cfg)
        layers = [(M, D, F)]
    model = model.to(dev)
    if args.vth_spread == "full":
        with torch.no_grad():
            for name, p in model.named_parameters():
                if name.endswith(("vth_pos", "vth_neg")):
                    p.uniform_(float(cfg["V_TH_MIN"]), float(cfg["V_TH_MAX"]))
    x = torch.randn(B, T, D, device=dev)
    if physical is None:
        x = x.clamp(0.0, 4.0)  # VoltageMapping defaults, applied once up front
    x.requires_grad_(True)
    with torch.no_grad():
        g = torch.randn_like(model(x))
    cells_fwd = float(sum(m * k * o for m, k, o in layers))
    cells_step = 2.0 * cells_fwd

    def step():
        model.zero_grad(set_to_none=True)
        x.grad = None
        out = model(x)
        out.backward(g)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    graph = None
    if args.graph:
        # the step captured once; each replay recomputes the outputs and gradients in the
        # graph's own buffers (the library reads nothing back to the host and allocates nothing)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        model.zero_grad(set_to_none=True)
        x.grad = None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            model(x).backward(g)
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    step_ms = []

    def timed(run):
        """Mean ms per step over the timed region (the whole-job rate), wall seconds; the
        per-step durations from HIP events between steps go to step_ms (for the median)."""
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        for i in range(args.steps):
            marks[i].record()
            run()
        marks[-1].record()
        e1.record()
        torch.cuda.synchronize()
        step_ms[:] = [marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps)]
        return e0.elapsed_time(e1) / args.steps, time.perf_counter() - t0

    if graph is None:
        # the value comes from uninstrumented steps: the library's per-call HIP events (the
        # KernelTimer's) add a stream marker around each launch, ~40 us per step at configs[0]
        ms, wall = timed(step)
        value_step_ms = list(step_ms)
        with _hip.KernelTimer() as kt:  # per-kernel launch times and clocks: the same steps, instrumented
            timed(step)
        step_ms[:] = value_step_ms
    else:
        ms, wall = timed(graph.replay)
        with _hip.KernelTimer() as kt:  # per-kernel launch times: the same kernels, eager
            eager_ms, _ = timed(step)
        log(f"[bench] {args.config}: eager step {eager_ms:.3f} ms (host launches included)")
    value = cells_step / (ms * 1e-3)
    median_ms = statistics.median(step_ms) if step_ms else ms
    host = {"autograd_thread": "calling" if args.calling_thread else "engine (torch default)"}
    if graph is None:
        # the same eager step with the other autograd threading, for comparison (not the value)
        torch.autograd.set_multithreading_enabled(args.calling_thread)
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        other = 1e3 * (time.perf_counter() - t0) / args.steps
        torch.autograd.set_multithreading_enabled(not args.calling_thread)
        host["eager_ms_engine_thread" if args.calling_thread else "eager_ms_calling_thread"] = round(other, 4)
        log(f"[bench] eager step with the {'engine' if args.calling_thread else 'calling'} thread: {other:.3f} ms")
    log(f"[bench] {args.config}: {ms:.3f} ms/step mean, {median_ms:.3f} median"
        f"{' (graph replay)' if graph is not None else ''} "
        f"(wall {1e3 * wall / args.steps:.3f}), {value:.4e} cell-evals/s")

    power = None
    if args.power_seconds > 0:
        power = board_power(graph.replay if graph is not None else step, args.power_seconds)
        if "watts" in power:  # the board's energy per cell-eval at the timed rate
            power["nj_per_cell_eval"] = round(power["watts"] / value * 1e9, 4)
        log(f"[bench] board power over the step loop: {power}")

    phases = None
    if args.power_phases > 0 and args.ekv_approx == "lut":
        phases = power_phases(cfg, layers[0][1], layers[0][2], layers[0][0], dev, args.power_phases)

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.empty(n, device=dev).uniform_()
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 1.0, out=dst)  # an elementwise kernel (a hipMemcpy may use the DMA engines)
        torch.cuda.synchronize()
        del src, dst

    fwd_avg = kt.fwd_ms / max(kt.fwd_launches, 1)
    bwd_avg = kt.bwd_ms / max(kt.bwd_launches, 1)
    cells_launch = cells_fwd / len(layers)  # per-launch cells (equal for fc1 and fc2)
    fwd_cells_s = cells_fwd * args.steps / (kt.fwd_ms * 1e-3) if kt.fwd_ms else 0.0
    bwd_cells_s = cells_fwd * args.steps / (kt.bwd_ms * 1e-3) if kt.bwd_ms else 0.0
    achieved = bwd_cells_s * bwd_instr / 1e12
    peak = VALU_PEAK / 1e12
    exact = args.ekv_approx == "exact"
    roofline = {
        "bound": "valu",
        "achieved": round(achieved, 3),
        "peak": round(peak, 3),
        "unit": "TOP/s",
        "frac": round(achieved / peak, 4),
        "model": f"the contract model: {bwd_instr} (backward) / {fwd_instr} (forward) VALU lane-instr per cell-eval "
                 "at 256 CU x 64 lanes x 2.4 GHz; the kernels issue other counts and gfx950 issues more than one "
                 "VALU instruction per CU-cycle, so these fractions are not utilisation (measured_ceiling is)",
        "traffic": None if exact else measured_traffic(args.config)[0],
        "traffic_source": None if exact else measured_traffic(args.config)[1],
        "traffic_per_layer": None if exact else measured_traffic(args.config)[2],
        "kernel": ("bwd_exact_kernel<true,true> (backward main kernel, dominant)" if exact else
                   "table backward main kernel, dominant: bwd_ranked_kernel<true> where the ranked mode applies "
                   "(the initial thresholds), else bwd_kernel / bwd_two_copies_kernel"),
        "work": f"{bwd_instr} VALU lane-instr per cell-eval x {cells_launch:.4e} cells per launch",
        "avg_launch_ms": round(bwd_avg, 4),
        "forward_kernel": {
            "kernel": ("fwd_exact_kernel" if exact else "fwd_kernel (windowed table copies where they fit)")
                      + " (with split_reduce_kernel where the plan splits K)",
            "avg_launch_ms": round(fwd_avg, 4),
            "achieved": round(fwd_cells_s * fwd_instr / 1e12, 3),
            "frac": round(fwd_cells_s * fwd_instr / VALU_PEAK, 4),
        },
        "step_frac_of_cell_roofline": round(value / (2.0 / (fwd_instr / VALU_PEAK + bwd_instr / VALU_PEAK)), 4),
    }
    log(f"[bench] fwd kernel {fwd_avg:.3f} ms/launch ({roofline['forward_kernel']['frac']:.3f} of VALU peak), "
        f"bwd kernel {bwd_avg:.3f} ms/launch ({roofline['frac']:.3f})")
    if not exact:
        roofline["lds"] = lds_roofline(model, cfg, cells_launch, fwd_avg, bwd_avg, dev)
        clock = roofline["lds"].pop("_clock")
        log(f"[bench] LDS gather roofline (window {roofline['lds']['window_records']} records, "
            f"{roofline['lds']['ns_per_gather_per_cu']:.3f} ns per gather per CU): fwd "
            f"{roofline['lds']['forward_frac']:.3f}, bwd {roofline['lds']['backward_frac']:.3f}; "
            f"conflict-free {roofline['lds']['conflict_free_frac']}")
        roofline["lds"]["probe_ghz"] = round(clock["ghz"], 4) if clock.get("ghz") else None
        mc = measured_ceiling(kt, cells_launch, fwd_avg, bwd_avg, dev)
        roofline["measured_ceiling"] = mc
        for side in ("backward", "forward"):
            r = mc[side]
            log(f"[bench] measured VALU ceiling, {r['kernel']}: {r.get('kernel_ghz')} GHz during the steps, "
                f"{r['issued_valu_per_cell']} VALU/cell, replay {r['replay_instr_per_cu_cycle']} instr/CU-cycle "
                f"-> ceiling {r.get('ceiling_ms')} ms vs {r['avg_launch_ms']} ms: frac {r.get('frac')}")

    cpu = None
    lut_cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU baseline ...")
        cpu = cpu_baseline([(k, o) for _, k, o in layers], args.cpu_seconds)
        log(f"[bench] cpu {cpu['value']:.4e} cell-evals/s on {cpu['cores']} threads")
        lut_cpu = cpu_lut_oracle(D, F, 4.0)
        log(f"[bench] cpu LUT oracle {lut_cpu['value']:.4e} cell-evals/s on {lut_cpu['cores']} threads")

    result = {
        "metric": "CIM cell-evals/sec fwd+bwd, Physical GPT-L FFN, 1 GPU; % of VALU roofline",
        "value": value,
        "unit": "cell-evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "ms_per_step_median": median_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": {
                "gptl_ffn": "Physical GPT-L FFN: CIMLinear 768->3072->768, X[8,1024,768] fp32, fwd+bwd",
                "vitm_ffn": "Physical ViT-M FFN: CIMLinear 256->1024->256, X[128,65,256] fp32, fwd+bwd",
                "gptm_hybrid": "Hybrid GPT-M FFN: CIMLinear 384->1536 + Linear 1536->384, X[16,1024,384], fwd+bwd",
                "vits_up": "ViT-S up-projection: CIMLinear 192->768, X[8,65,192] fp32, fwd+bwd",
            }[args.config] + (" (exact-formula kernels, ekv_approx='exact')" if exact else "")
              + (f" (LUT_DTYPE={cfg['LUT_DTYPE']})" if args.lut_dtype else "")
              + (" (thresholds U[V_TH_MIN, V_TH_MAX])" if args.vth_spread == "full" else "")
              + (" (step replayed from one captured HIP graph)" if graph is not None else ""),
            "tokens": M,
            "lut_entries": args.lut_size,
            "cell_evals_per_step": cells_step,
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_lut_oracle": lut_cpu,
        "host": host,
        "board_power": power,
        "board_power_phases": phases,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
