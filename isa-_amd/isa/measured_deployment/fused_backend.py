"""Opt-in fused backend (drop-in for `src/isa/measured_deployment/fused_backend.py`).

`install_fused_backend()` makes every `DeploymentAwareCIMLinear` configured afterwards from
the same codebook tensors on the same device share one device copy of the codebook and of
its coefficient tables, instead of each layer holding its own (the reference's
`codebook_cache`, `fused_backend.py:37-131`: with the 32,240-curve Monte Carlo codebook
that is ~24 MB per layer). Installing twice is a no-op.

The cache here differs from the reference's in two ways a caller can see:

* it holds the source tensors weakly: an entry lives while its sources do (a finalizer on
  each source drops the entries built from it), so dropping a codebook frees its cached
  copy, while the layers configured from it keep the device tables they were given (the
  reference's entries hold the sources, so every codebook ever configured stays alive);
* the key includes the sources' in-place version counters, so a source edited in place
  after configuration is a new codebook, not a stale hit.

What the reference's install also switches, and why it does not apply here: it routes
no-grad measured forwards below a token threshold (`FG50_*_FUSED_TOKEN_THRESHOLD`) to its
Triton gather kernel and the rest to the segmented GEMM path; here `measured_forward`
always runs the fused HIP kernel, with its gradient for x, at every token count. Its
restrictions to uniform voltage grids and `vin_lut_bins == 0` do not apply either (the HIP
kernel supports both); the `FG50_*` variables are not read.
"""

from __future__ import annotations

import weakref
from typing import Callable

import torch

# key -> the book of tensors DeploymentAwareCIMLinear.configure_codebook builds. The key names
# the source tensors by id and by version: (device type, device index, id(vg), id(currents),
# vg._version, currents._version, shapes, vin_lut_bins, V_min, V_max).
_SHARED_CODEBOOKS: dict[tuple, dict[str, object]] = {}
_WATCHED_SOURCES: set[int] = set()  # ids of the live source tensors that carry a finalizer


def _drop_codebooks(source_id: int) -> None:
    """Finalizer of a source tensor: drop every entry built from it."""
    _WATCHED_SOURCES.discard(source_id)
    for key in [k for k in _SHARED_CODEBOOKS if source_id in (k[2], k[3])]:
        _SHARED_CODEBOOKS.pop(key, None)


def _watch_source(t: torch.Tensor) -> None:
    if id(t) not in _WATCHED_SOURCES:
        _WATCHED_SOURCES.add(id(t))
        weakref.finalize(t, _drop_codebooks, id(t))


def shared_codebook(vg: torch.Tensor, currents_a: torch.Tensor, device: torch.device, bins: int, v_min: float,
                    v_max: float, build: Callable[..., dict]) -> dict:
    """The shared book for these sources on `device`, built with `build(vg, currents_a, device,
    bins, v_min, v_max)` on a miss (the cache of fused_backend.py:58-125)."""
    key = (device.type, device.index, id(vg), id(currents_a), vg._version, currents_a._version,
           tuple(vg.shape), tuple(currents_a.shape), int(bins), float(v_min), float(v_max))
    book = _SHARED_CODEBOOKS.get(key)
    if book is not None and book["sources"][0]() is vg and book["sources"][1]() is currents_a:
        return book
    book = dict(build(vg, currents_a, device, bins, v_min, v_max))
    book["sources"] = (weakref.ref(vg), weakref.ref(currents_a))
    for stale in [k for k in _SHARED_CODEBOOKS if k[2:4] == key[2:4]]:
        _SHARED_CODEBOOKS.pop(stale)  # built from an earlier version of these sources
    _watch_source(vg)
    _watch_source(currents_a)
    _SHARED_CODEBOOKS[key] = book
    return book


def install_fused_backend() -> None:
    from isa.measured_deployment.operator import DeploymentAwareCIMLinear

    DeploymentAwareCIMLinear._fg50_fused_backend_installed = True
