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

    print("[case] bench.py --config vits_up --steps 2 --warmup 1 --no-cpu-baseline", flush=True)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--config", "vits_up", "--steps", "2", "--warmup", "1",
                                      "--no-cpu-baseline"])
    assert bench.main() == 0
    lines = [ln for ln in capsys.readouterr().out.splitlines() if ln.startswith("{")]
    assert len(lines) == 1
    rec = json.loads(lines[0])
    assert REQUIRED <= set(rec)
    assert rec["n_gpus"] == 1 and rec["steps"] == 2 and rec["warmup"] == 1
    assert rec["value"] > 0 and rec["ms_per_step"] > 0 and rec["higher_is_better"] is True
    assert "workload" in rec["config"]
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
    assert mc["backward"]["kernel"] == "bwd_kernel"  # config 1 is below the copy threshold: one copy
    assert mc["fma_issue_instr_per_cu_cycle"] > 0.25
