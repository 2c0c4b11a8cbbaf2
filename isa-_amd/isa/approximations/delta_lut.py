"""Flash-EKV delta-V lookup tables.

Mirrors `src/isa/approximations/delta_lut.py:41-63` (`get_ekv_lut_tables(cfg, device)`,
cached per device and parameters). Two table modes:

* the default, `LUT_DTYPE = "float32"`: the table is evaluated on the GPU in fp64 and
  rounded once to fp32 (`isa_ekv_lut_build`), which follows the closed form to ~2e-7
  relative everywhere (the fp32 torch steps of the reference lose the derivative table's
  subthreshold end to cancellation in `1 - exp(-sp)`);
* `LUT_DTYPE = "bfloat16"`: the reference's own tables, byte for byte. The fp32
  intermediate is built on the host with the reference's fp32 torch steps
  (`delta_lut.py:25-34`: fp32 `linspace`, `F.softplus`, `1 - exp(-sp)` under the
  `sp > 20` switch, the scalar factors applied in the same order), cast to bf16 with
  round-to-nearest-even (`:35`) and uploaded once (`:62`); the kernels then read the
  widened bf16 values, as the reference's CUDA backward does (`cuda_backend.py:68-69`).

`get_packed_tables` adds the padded kernel records (forward {I, dI}, backward
{I, dI, D, dD}) derived from the plain pair, cached under the same key.
"""

from __future__ import annotations

from typing import Any, Dict, Tuple

import torch
import torch.nn.functional as F

from isa.kernels.transformer_ffn import _hip, ops


def lut_range(cfg: Dict[str, Any]) -> Tuple[float, float, int]:
    """(delta_min, delta_max, size) as delta_lut.py:42-48."""
    v_min = float(cfg.get("LUT_V_MIN", cfg.get("V_signed_min", -4.0)))
    v_max = float(cfg.get("LUT_V_MAX", cfg.get("V_signed_max", 4.0)))
    vth_min = float(cfg.get("LUT_VTH_MIN", cfg.get("V_TH_MIN", 0.0)))
    vth_max = float(cfg.get("LUT_VTH_MAX", cfg.get("V_TH_MAX", 5.0)))
    delta_min = float(cfg.get("LUT_DELTA_MIN", v_min - vth_max))
    delta_max = float(cfg.get("LUT_DELTA_MAX", v_max - vth_min))
    delta_size = int(cfg.get("LUT_DELTA_SIZE", 16384))
    return delta_min, delta_max, delta_size


def lut_is_bf16(cfg: Dict[str, Any]) -> bool:
    dt = str(cfg.get("LUT_DTYPE", "float32")).lower()
    if dt in ("float32", "fp32", "f32"):
        return False
    if dt in ("bfloat16", "bf16"):
        return True
    raise ValueError(f"LUT_DTYPE must be 'float32' or 'bfloat16', got {cfg.get('LUT_DTYPE')!r}")


def _cpu_key(cfg: Dict[str, Any]) -> Tuple:
    delta_min, delta_max, delta_size = lut_range(cfg)
    return (
        float(cfg["n"]),
        float(cfg["V_sat"]),
        float(cfg["I_S"]),
        float(cfg["U_T"]),
        float(cfg["V_D"]),
        delta_min,
        delta_max,
        delta_size,
        lut_is_bf16(cfg),
    )


def reference_bf16_tables(n: float, i_s: float, u_t: float, v_d: float, delta_min: float, delta_max: float,
                          size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """The reference's bf16 (table_i, table_ddelta) on the host (`delta_lut.py:25-35`).

    Every step is the fp32 torch operation the reference runs, in its order, because the
    bytes depend on each rounding: the grid is fp32 `linspace`; the Python-float factors
    (1/(2 n U_T), V_D, I_S, 2 I_S/(2 n U_T)) enter each op as fp32 scalars; the softplus is
    torch's (threshold 20); the sigmoid is `1 - exp(-sp)`, switched to 1 where sp > 20.
    """
    grid = torch.linspace(delta_min, delta_max, size, dtype=torch.float32)
    scale = 1.0 / (2.0 * n * u_t)
    sp_hi = F.softplus(grid * scale)
    sp_lo = F.softplus((grid - v_d) * scale)
    one = torch.ones_like(sp_hi)
    sig_hi = torch.where(sp_hi > 20.0, one, 1.0 - torch.exp(-sp_hi))
    sig_lo = torch.where(sp_lo > 20.0, one, 1.0 - torch.exp(-sp_lo))
    table_i = i_s * (sp_hi.square() - sp_lo.square())
    table_d = i_s * 2.0 * scale * (sp_hi * sig_hi - sp_lo * sig_lo)
    return table_i.contiguous().to(torch.bfloat16), table_d.contiguous().to(torch.bfloat16)


_device_cache: dict[Tuple, Tuple[torch.Tensor, torch.Tensor]] = {}
_packed_cache: dict[Tuple, Tuple[torch.Tensor, torch.Tensor]] = {}


def _resolve(device) -> torch.device:
    device = torch.device(device)
    if device.type != "cuda":
        raise RuntimeError(f"EKV LUT tables are built on a ROCm device; got device {device}")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return device


def get_ekv_lut_tables(cfg: Dict[str, Any], device) -> Tuple[torch.Tensor, torch.Tensor]:
    """(table_i, table_ddelta) on `device`, each [LUT_DELTA_SIZE]."""
    device = _resolve(device)
    key = _cpu_key(cfg)
    cache_key = (str(device), key)
    if cache_key not in _device_cache:
        n, _v_sat, i_s, u_t, v_d, delta_min, delta_max, size, bf16 = key
        if size < 1:
            raise ValueError(f"LUT_DELTA_SIZE must be >= 1, got {size}")
        if bf16:
            host = reference_bf16_tables(n, i_s, u_t, v_d, delta_min, delta_max, size)
            tables = tuple(t.to(device=device) for t in host)
        else:
            tables = ops.build_plain_tables((n, u_t, i_s, v_d), delta_min, delta_max, size, device)
        # later users may run on other streams: finish the one-time build first
        torch.cuda.current_stream(device).synchronize()
        _device_cache[cache_key] = tables
    return _device_cache[cache_key]


def get_packed_tables(cfg: Dict[str, Any], device) -> Tuple[torch.Tensor, torch.Tensor]:
    """(forward records, backward records) for the HIP kernels, derived from the plain pair."""
    device = _resolve(device)
    cache_key = (str(device), _cpu_key(cfg))
    if cache_key not in _packed_cache:
        table_i, table_d = get_ekv_lut_tables(cfg, device)
        fwd = ops.pack_tables(table_i, None, _hip.LUT_FWD)
        bwd = ops.pack_tables(table_i, table_d, _hip.LUT_BWD)
        torch.cuda.current_stream(device).synchronize()
        _packed_cache[cache_key] = (fwd, bwd)
    return _packed_cache[cache_key]


def clear_cache() -> None:
    _device_cache.clear()
    _packed_cache.clear()
