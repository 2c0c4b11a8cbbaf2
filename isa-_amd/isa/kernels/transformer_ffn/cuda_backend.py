"""Loader and shared backward of the Flash-EKV HIP library.

Same entry points as the reference's `src/isa/kernels/transformer_ffn/cuda_backend.py`:

* `load_extension(verbose=False)` (lru-cached, :16-42) returns an extension object whose
  `forward`, `grad_x`, `grad_x_shared`, `grad_w`, `grad_w_shared` take and return tensors
  like the reference's pybind11 module (`cuda/binding.cpp:56-62`). They run the HIP
  library; the library itself is prebuilt in-tree (`isa-_amd/csrc/build.py`), there is no
  JIT step. `EKV_CUDA_BUILD_DIR` may point at another directory holding the library.
* `prebuild()` (:45-47) loads the library and, on a ROCm device, builds and caches the
  default tables, then prints `[ekv-cuda] ready: ...`.
* `shared_backward(...)` (:50-99) keeps the reference's signature and casts.
"""

from __future__ import annotations

import os
from functools import lru_cache
from pathlib import Path
from typing import Optional, Tuple

import torch

from isa.kernels.transformer_ffn import _hip, ops


def _check(t: torch.Tensor, name: str) -> None:
    # ekv_cuda.cu:343-347
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _forward_unclamped(x, wpos, wneg, table_i, delta_min, delta_max, v_sat):
    for t, n in ((x, "x"), (wpos, "wpos"), (wneg, "wneg"), (table_i, "table_i")):
        _check(t, n)
    fwd = ops.pack_tables(table_i, None, _hip.LUT_FWD)
    inf = float("inf")
    # binding.cpp:57 `forward` returns the unclamped sum (ekv_cuda.cu:97-137)
    return ops.lut_forward(x, wpos, wneg, fwd, table_i.numel(), delta_min, delta_max, v_sat, -inf, inf)


def _grad_x(x, wpos, wneg, grad_out, table_i, table_ddelta, delta_min, delta_max, v_sat, shared: bool):
    for t, n in ((x, "x"), (wpos, "wpos"), (wneg, "wneg"), (grad_out, "grad_out"), (table_i, "table_i"),
                 (table_ddelta, "table_ddelta")):
        _check(t, n)
    if shared and table_i.numel() > ops.MAX_ENTRIES_BACKWARD:
        raise RuntimeError("shared grad_x supports LUT_DELTA_SIZE <= 8192")
    bwd = ops.pack_tables(table_i, table_ddelta, _hip.LUT_BWD)
    gx, _, _ = ops.lut_backward(x, wpos, wneg, grad_out, bwd, table_i.numel(), delta_min, delta_max, v_sat,
                                True, False)
    return gx


def _grad_w(x, wpos, wneg, grad_out, table_ddelta, delta_min, delta_max, v_sat, shared: bool):
    for t, n in ((x, "x"), (wpos, "wpos"), (wneg, "wneg"), (grad_out, "grad_out"), (table_ddelta, "table_ddelta")):
        _check(t, n)
    if shared and table_ddelta.numel() > ops.MAX_ENTRIES_BACKWARD:
        raise RuntimeError("shared grad_w supports LUT_DELTA_SIZE <= 8192")
    bwd = ops.pack_tables(table_ddelta, table_ddelta, _hip.LUT_BWD)
    _, gp, gn = ops.lut_backward(x, wpos, wneg, grad_out, bwd, table_ddelta.numel(), delta_min, delta_max, v_sat,
                                 False, True)
    return [gp, gn]


class _Extension:
    """Tensor-level view of libisa_ekv_hip.so shaped like the reference's extension module."""

    def __init__(self, lib, path: Path):
        self.lib = lib
        self.path = path
        self.__name__ = "isa_ekv_hip"

    def forward(self, x, wpos, wneg, table_i, delta_min, delta_max, v_sat):
        return _forward_unclamped(x, wpos, wneg, table_i, delta_min, delta_max, v_sat)

    def grad_x(self, x, wpos, wneg, grad_out, table_i, table_ddelta, delta_min, delta_max, v_sat):
        return _grad_x(x, wpos, wneg, grad_out, table_i, table_ddelta, delta_min, delta_max, v_sat, shared=False)

    def grad_x_shared(self, x, wpos, wneg, grad_out, table_i, table_ddelta, delta_min, delta_max, v_sat):
        return _grad_x(x, wpos, wneg, grad_out, table_i, table_ddelta, delta_min, delta_max, v_sat, shared=True)

    def grad_w(self, x, wpos, wneg, grad_out, table_ddelta, delta_min, delta_max, v_sat):
        return _grad_w(x, wpos, wneg, grad_out, table_ddelta, delta_min, delta_max, v_sat, shared=False)

    def grad_w_shared(self, x, wpos, wneg, grad_out, table_ddelta, delta_min, delta_max, v_sat):
        return _grad_w(x, wpos, wneg, grad_out, table_ddelta, delta_min, delta_max, v_sat, shared=True)


@lru_cache(maxsize=1)
def load_extension(verbose: bool = False) -> _Extension:
    build_dir = os.environ.get("EKV_CUDA_BUILD_DIR")
    path = Path(build_dir) / _hip.LIB_NAME if build_dir else _hip.LIB_PATH
    lib = _hip.load(path)
    if verbose:
        print(f"[ekv-cuda] loaded {path}")
    return _Extension(lib, path)


def prebuild() -> None:
    extension = load_extension(verbose=os.environ.get("EKV_CUDA_VERBOSE_BUILD", "0") == "1")
    if torch.cuda.is_available():
        from isa.approximations.delta_lut import get_packed_tables
        from isa.device_models.config import FLASH_TRANSISTOR_EKV_CONFIG

        get_packed_tables(FLASH_TRANSISTOR_EKV_CONFIG, torch.device("cuda", torch.cuda.current_device()))
    print(f"[ekv-cuda] ready: {extension.__name__}")


def shared_backward(
    x: torch.Tensor,
    wpos: torch.Tensor,
    wneg: torch.Tensor,
    grad_out: torch.Tensor,
    table_i: torch.Tensor,
    table_ddelta: torch.Tensor,
    delta_min: float,
    delta_max: float,
    v_sat: float,
    need_grad_x: bool,
    need_grad_w: bool,
) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor], Optional[torch.Tensor]]:
    load_extension()
    if table_i.numel() > ops.MAX_ENTRIES_BACKWARD:
        raise RuntimeError("shared grad_x supports LUT_DELTA_SIZE <= 8192")
    bwd = ops.pack_tables(table_i, table_ddelta, _hip.LUT_BWD)
    gx, gp, gn = ops.lut_backward(x, wpos, wneg, grad_out, bwd, table_i.numel(), delta_min, delta_max, v_sat,
                                  bool(need_grad_x), bool(need_grad_w))
    if gx is not None:
        gx = gx.to(dtype=x.dtype)
    if gp is not None:
        gp = gp.to(dtype=wpos.dtype)
        gn = gn.to(dtype=wneg.dtype)
    return gx, gp, gn
