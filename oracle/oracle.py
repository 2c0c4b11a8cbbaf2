"""CPU oracle for the Flash-EKV LUT CIMLinear (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this module, and only as the checker; the product package never does.

Wraps ``oracle/ekv_oracle.c`` (the reference LUT algorithm restated with an fp32 table,
per-cell fp32 arithmetic and double sums) through ctypes, plus the reference's
configuration restated from ``src/isa/device_models/config.py:9-43`` and
``src/isa/approximations/delta_lut.py:41-48``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Optional, Tuple

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libekv_oracle.so"

# device_models/config.py:9-22 (and configs/devices/flash_transistor_ekv.yaml:6-16)
FLASH_PARAMS = {
    "n": 4.1360,
    "V_sat": 8.2624,
    "I_S": 7.5875e-7,
    "U_T": 0.0259,
    "V_D": 0.1,
    "R_TIA": 1e5,
    "V_TH_MIN": 0.0,
    "V_TH_MAX": 5.0,
    "V_min": 0.0,
    "V_max": 4.0,
    "V_signed_min": -4.0,
    "V_signed_max": 4.0,
}


def lut_range(cfg: dict) -> Tuple[float, float, int]:
    """delta_lut.py:42-48 / ekv_lut_triton.py:138-144."""
    v_min = float(cfg.get("LUT_V_MIN", cfg.get("V_signed_min", -4.0)))
    v_max = float(cfg.get("LUT_V_MAX", cfg.get("V_signed_max", 4.0)))
    vth_min = float(cfg.get("LUT_VTH_MIN", cfg.get("V_TH_MIN", 0.0)))
    vth_max = float(cfg.get("LUT_VTH_MAX", cfg.get("V_TH_MAX", 5.0)))
    delta_min = float(cfg.get("LUT_DELTA_MIN", v_min - vth_max))
    delta_max = float(cfg.get("LUT_DELTA_MAX", v_max - vth_min))
    size = int(cfg.get("LUT_DELTA_SIZE", 16384))
    return delta_min, delta_max, size


def build(force: bool = False) -> Path:
    """Compile ekv_oracle.c with the committed Makefile."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (HERE / "ekv_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        f64p = ctypes.POINTER(ctypes.c_double)
        i64 = ctypes.c_int64
        d = ctypes.c_double
        L.oracle_lut_build.argtypes = [d, d, d, d, d, d, ctypes.c_int, f32p, f32p]
        L.oracle_lut_build.restype = None
        L.oracle_forward.argtypes = [f32p, f32p, f32p, f32p, i64, i64, i64, ctypes.c_int, d, d,
                                     ctypes.c_float, d, d, f64p]
        L.oracle_forward.restype = None
        L.oracle_grad_x.argtypes = [f32p, f32p, f32p, f32p, f32p, f32p, i64, i64, i64, ctypes.c_int, d, d,
                                    ctypes.c_float, f64p]
        L.oracle_grad_x.restype = None
        L.oracle_grad_w.argtypes = [f32p, f32p, f32p, f32p, f32p, i64, i64, i64, ctypes.c_int, d, d,
                                    ctypes.c_float, f64p, f64p]
        L.oracle_grad_w.restype = None
        L.oracle_lut_lookup.argtypes = [f32p, ctypes.c_float, d, d, ctypes.c_int]
        L.oracle_lut_lookup.restype = ctypes.c_float
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _p32(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _p64(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def lut_tables(cfg: Optional[dict] = None, size: Optional[int] = None,
               delta_min: Optional[float] = None, delta_max: Optional[float] = None) -> Tuple[np.ndarray, np.ndarray]:
    """fp32 (table_i, table_ddelta), delta_lut.py:25-34 evaluated in fp64."""
    cfg = dict(FLASH_PARAMS if cfg is None else cfg)
    dmin, dmax, n = lut_range(cfg)
    if size is not None:
        n = size
    if delta_min is not None:
        dmin = delta_min
    if delta_max is not None:
        dmax = delta_max
    ti = np.empty(n, np.float32)
    td = np.empty(n, np.float32)
    lib().oracle_lut_build(float(cfg["n"]), float(cfg["U_T"]), float(cfg["I_S"]), float(cfg["V_D"]),
                           dmin, dmax, n, _p32(ti), _p32(td))
    return ti, td


def reference_lut_tables(cfg: Optional[dict] = None, size: Optional[int] = None,
                         delta_min: Optional[float] = None, delta_max: Optional[float] = None):
    """The reference's own table pair, restated statement by statement from
    `src/isa/approximations/delta_lut.py:25-35` in torch fp32 (its third-party arithmetic:
    torch's CPU `linspace`, `softplus` and `exp`, whose roundings the bytes depend on).

    Returns (fp32 table_i, fp32 table_ddelta, bf16 table_i, bf16 table_ddelta): the fp32
    intermediate of `:31`/`:34` as numpy float32, and the `:35` cast as torch bfloat16.
    """
    import torch
    import torch.nn.functional as F

    cfg = dict(FLASH_PARAMS if cfg is None else cfg)
    dmin, dmax, n_entries = lut_range(cfg)
    if size is not None:
        n_entries = size
    if delta_min is not None:
        dmin = delta_min
    if delta_max is not None:
        dmax = delta_max
    n, i_s, u_t, v_d = float(cfg["n"]), float(cfg["I_S"]), float(cfg["U_T"]), float(cfg["V_D"])
    delta = torch.linspace(dmin, dmax, n_entries, dtype=torch.float32)           # :25
    inv_2nut = 1.0 / (2.0 * n * u_t)                                              # :26
    u1 = delta * inv_2nut                                                         # :27
    u2 = (delta - v_d) * inv_2nut                                                 # :28
    sp1 = F.softplus(u1)                                                          # :29
    sp2 = F.softplus(u2)                                                          # :30
    base = i_s * (sp1.square() - sp2.square())                                    # :31
    sig1 = torch.where(sp1 > 20.0, torch.ones_like(sp1), 1.0 - torch.exp(-sp1))  # :32
    sig2 = torch.where(sp2 > 20.0, torch.ones_like(sp2), 1.0 - torch.exp(-sp2))  # :33
    grad_delta = i_s * 2.0 * inv_2nut * (sp1 * sig1 - sp2 * sig2)                 # :34
    return (base.numpy().copy(), grad_delta.numpy().copy(),
            base.contiguous().to(torch.bfloat16), grad_delta.contiguous().to(torch.bfloat16))  # :35


def lut_lookup(table: np.ndarray, delta: float, delta_min: float, delta_max: float) -> float:
    t = _f32(table)
    return float(lib().oracle_lut_lookup(_p32(t), float(delta), delta_min, delta_max, t.size))


def forward(x, wp, wn, table_i, delta_min: float, delta_max: float, v_sat: float,
            out_min: float = -4.0, out_max: float = 4.0) -> np.ndarray:
    x, wp, wn, ti = _f32(x), _f32(wp), _f32(wn), _f32(table_i)
    M, K = x.shape
    O = wp.shape[0]
    out = np.empty((M, O), np.float64)
    lib().oracle_forward(_p32(x), _p32(wp), _p32(wn), _p32(ti), M, K, O, ti.size, delta_min, delta_max,
                         v_sat, out_min, out_max, _p64(out))
    return out


def grad_x(x, wp, wn, grad, table_i, table_d, delta_min: float, delta_max: float, v_sat: float) -> np.ndarray:
    x, wp, wn, g, ti, td = _f32(x), _f32(wp), _f32(wn), _f32(grad), _f32(table_i), _f32(table_d)
    M, K = x.shape
    O = wp.shape[0]
    out = np.empty((M, K), np.float64)
    lib().oracle_grad_x(_p32(x), _p32(wp), _p32(wn), _p32(g), _p32(ti), _p32(td), M, K, O, ti.size,
                        delta_min, delta_max, v_sat, _p64(out))
    return out


def grad_w(x, wp, wn, grad, table_d, delta_min: float, delta_max: float, v_sat: float):
    x, wp, wn, g, td = _f32(x), _f32(wp), _f32(wn), _f32(grad), _f32(table_d)
    M, K = x.shape
    O = wp.shape[0]
    gp = np.empty((O, K), np.float64)
    gn = np.empty((O, K), np.float64)
    lib().oracle_grad_w(_p32(x), _p32(wp), _p32(wn), _p32(g), _p32(td), M, K, O, td.size,
                        delta_min, delta_max, v_sat, _p64(gp), _p64(gn))
    return gp, gn


def backward(x, wp, wn, grad, table_i, table_d, delta_min: float, delta_max: float, v_sat: float):
    dx = grad_x(x, wp, wn, grad, table_i, table_d, delta_min, delta_max, v_sat)
    gp, gn = grad_w(x, wp, wn, grad, table_d, delta_min, delta_max, v_sat)
    return dx, gp, gn


def normwise_error(actual, expected) -> float:
    """max|actual - expected| / max|expected| (0 when both are all-zero)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    den = float(np.max(np.abs(e))) if e.size else 0.0
    num = float(np.max(np.abs(a - e))) if e.size else 0.0
    if den == 0.0:
        return num
    return num / den


def elementwise_error(actual, expected, floor_frac: float = 1e-3) -> float:
    """max |actual - expected| / max(|expected|, floor_frac * max|expected|)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    if not e.size:
        return 0.0
    floor = floor_frac * float(np.max(np.abs(e)))
    den = np.maximum(np.abs(e), floor if floor > 0 else 1e-300)
    return float(np.max(np.abs(a - e) / den))


def threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
