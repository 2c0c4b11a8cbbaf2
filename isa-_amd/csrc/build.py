"""Build libisa_ekv_hip.so (gfx950) in-tree with hipcc.

Usage: ``python isa-_amd/csrc/build.py`` (also called by ``__graft_entry__.build()``).
The library lands next to its ctypes loader in ``isa/kernels/transformer_ffn/``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG_ROOT = CSRC.parent
REPO = PKG_ROOT.parent
SOURCES = [CSRC / "ekv_lut.hip"]
INCLUDE = REPO / "include"
OUT = PKG_ROOT / "isa" / "kernels" / "transformer_ffn" / "libisa_ekv_hip.so"
ARCH = os.environ.get("ISA_EKV_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed FP32 ops stay off on this pool; hipcc -O3 would otherwise form them
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def build(verbose: bool = False) -> Path:
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", "-o", str(tmp), *map(str, SOURCES)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    path = build(verbose=True)
    print(f"built {path}")
    sys.exit(0)
