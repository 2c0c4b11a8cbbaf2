"""bench.py keeps the driver's contract: one JSON line with the required keys, and a clear
refusal for more than one GPU (this build measures one)."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

REQUIRED = {"metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"}


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and proc.stdout == ""


@pytest.mark.gpu
def test_bench_json_line(cuda_device, capsys, monkeypatch):
    import bench

    print("[case] bench.py --config vits_up --steps 2 --warmup 1 --no-cpu-baseline --power-seconds 2", flush=True)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--config", "vits_up", "--steps", "2", "--warmup", "1",
                                      "--no-cpu-baseline", "--power-seconds", "2"])
    assert bench.main() == 0
    lines = [ln for ln in capsys.readouterr().out.splitlines() if ln.startswith("{")]
    assert len(lines) == 1
    rec = json.loads(lines[0])
    assert REQUIRED <= set(rec)
    assert rec["n_gpus"] == 1 and rec["steps"] == 2 and rec["warmup"] == 1
    assert rec["value"] > 0 and rec["ms_per_step"] > 0 and rec["higher_is_better"] is True
    assert "workload" in rec["config"]
    # the board power leg: the firmware counters' reading, or why there is none
    bp = rec["board_power"]
    assert ("watts" in bp and bp["watts"] > 0 and 0.0 <= bp["ppt_residency"] <= 1.0 and bp["nj_per_cell_eval"] > 0) \
        or "error" in bp, bp
    roof = rec["roofline"]
    assert {"bound", "achieved", "peak", "unit", "frac", "traffic"} <= set(roof)
    assert 0 < roof["frac"] < 2 and roof["achieved"] > 0
    lds = roof["lds"]
    assert lds["window_records"] >= 1 and lds["ns_per_gather_per_cu"] > 0
    assert 0 < lds["conflict_free_ns_per_gather_per_cu"] <= 1.05 * lds["ns_per_gather_per_cu"]
    assert lds["conflict_free_frac"]["forward"] > 0 and lds["conflict_free_frac"]["backward"] > 0
    assert rec["ms_per_step_median"] > 0
    assert 0.5 < lds["probe_ghz"] < 3.5, lds  # the shader clock, in GHz
    mc = roof["measured_ceiling"]
    for side in ("backward", "forward"):
        r = mc[side]
        assert 0.5 < r["kernel_ghz"] < 3.5, r  # the clock the kernel's own blocks ran at
        assert r["issued_valu_per_cell"] > 0 and r["replay_instr_per_cu_cycle"] > 0.25, r
        assert 0 < r["frac"] <= 1.05, r  # a ceiling: the kernel cannot issue faster than its replay
        # its blocks live within the launch (one round of blocks at config 1's size)
        assert 0 < r["mean_block_lifetime_ms"] <= r["avg_launch_ms"], r
    assert mc["backward"]["kernel"] == "bwd_kernel"  # config 1 is below the copy threshold: one copy
    assert mc["fma_issue_instr_per_cu_cycle"] > 0.25


def _smi_json(energy_ticks: float, ns: float, ppt: float, acc: float) -> str:
    card = {"energy_accumulator (15.259uJ (2^-16))": str(energy_ticks), "system_clock_counter (ns)": str(ns),
            "ppt_residency_acc (Count)": str(ppt), "socket_thm_residency_acc (Count)": "0",
            "accumulation_counter (Count)": str(acc), "Max Graphics Package Power (W)": "1400.0",
            "current_gfxclks (MHz)": "[2100, 2100]"}
    return json.dumps({"card0": card, "system": {}})


def test_board_power_from_firmware_counters(monkeypatch):
    """bench.board_power: mean power = energy accumulator delta (15.259 uJ ticks) over the
    firmware clock delta, power-limit residency = PPT count delta over the accumulation count
    delta, from two rocm-smi snapshots taken while the step loop runs; an absent tool gives an
    error entry, not a failed bench."""
    import torch

    import bench

    snaps = iter([_smi_json(1e9, 1e9, 100.0, 1000.0), _smi_json(1e9 + 2.0e8, 3e9, 400.0, 2000.0)])

    class Done:
        def __init__(self, out):
            self.stdout = out

    monkeypatch.setattr(bench.subprocess, "run", lambda *a, **k: Done(next(snaps)))
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    calls = []
    res = bench.board_power(lambda: calls.append(1), 0.5)
    assert calls, "the step ran while the snapshots were taken"
    # 2e8 ticks x 15.259 uJ = 3051.8 J over 2 s
    assert res["watts"] == pytest.approx(2.0e8 * 15.259e-6 / 2.0, rel=1e-6)
    assert res["ppt_residency"] == pytest.approx(0.3) and res["thermal_residency"] == 0.0
    assert res["cap_watts"] == "1400.0" and res["interval_s"] == pytest.approx(2.0)

    def missing(*a, **k):
        raise FileNotFoundError("rocm-smi")

    monkeypatch.setattr(bench.subprocess, "run", missing)
    res = bench.board_power(lambda: None, 0.5)
    assert "error" in res and "rocm-smi" in res["error"]

    # a firmware sample that has not moved on is read again, and one that never does gives an
    # error entry, not a division by zero
    stale = iter([_smi_json(1e9, 1e9, 0.0, 1000.0)] * 3 + [_smi_json(1e9 + 1e8, 2e9, 0.0, 1500.0)])
    monkeypatch.setattr(bench.subprocess, "run", lambda *a, **k: Done(next(stale)))
    monkeypatch.setattr(bench.time, "sleep", lambda s: None)
    res = bench.board_power(lambda: None, 0.5)
    assert res["interval_s"] == pytest.approx(1.0) and res["watts"] == pytest.approx(1e8 * 15.259e-6)
    monkeypatch.setattr(bench.subprocess, "run", lambda *a, **k: Done(_smi_json(1e9, 1e9, 0.0, 1000.0)))
    res = bench.board_power(lambda: None, 0.5)
    assert "did not advance" in res["error"]
