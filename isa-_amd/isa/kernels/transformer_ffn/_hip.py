"""ctypes binding of libisa_ekv_hip.so (declared in include/isa_ekv.h).

The library is the only compute path: loading fails loudly when it is missing or was
built for another ABI. ``torch`` is imported first so the library binds to the HIP
runtime torch already loaded (both carry the soname libamdhip64.so.7).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library must share)

ABI_VERSION = 10
LIB_NAME = "libisa_ekv_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

LUT_PLAIN_F32 = 0
LUT_FWD = 1
LUT_BWD = 2
LUT_PLAIN_BF16 = 3

PLAN_FORWARD = 0
PLAN_BACKWARD = 1
PLAN_LAYER_BACKWARD = 2
PLAN_INFO_LEN = 8
NOALLOC_MAX_BYTES = 128 << 20  # ISA_EKV_NOALLOC_MAX_BYTES
OPT_COPY_MIN_CELLS = 1
OPT_RANKED = 2
OPT_WINDOW_COPIES = 3
OPT_RANK_MAX_SPREAD = 4
OPT_RANK_GREEDY_MIN = 5
OPT_RANK_XCD_ORDER = 6

EXPORTS = (
    "isa_ekv_abi_version",
    "isa_ekv_last_error",
    "isa_ekv_lut_pad",
    "isa_ekv_lut_bytes",
    "isa_ekv_lut_build",
    "isa_ekv_lut_pack",
    "isa_ekv_forward_workspace",
    "isa_ekv_forward",
    "isa_ekv_forward_noalloc",
    "isa_ekv_backward_workspace",
    "isa_ekv_backward",
    "isa_ekv_exact_forward_workspace",
    "isa_ekv_exact_forward",
    "isa_ekv_exact_backward_workspace",
    "isa_ekv_exact_backward",
    "isa_ekv_layer_forward_workspace",
    "isa_ekv_layer_backward_workspace",
    "isa_ekv_layer_forward",
    "isa_ekv_layer_backward",
    "isa_ekv_measured_forward_workspace",
    "isa_ekv_measured_backward_workspace",
    "isa_ekv_measured_forward",
    "isa_ekv_measured_backward",
    "isa_ekv_profile_begin",
    "isa_ekv_profile_end",
    "isa_ekv_profile_clock",
    "isa_ekv_probe_lds_gather",
    "isa_ekv_probe_valu_issue",
    "isa_ekv_plan_info",
    "isa_ekv_set_option",
)

_lock = threading.Lock()
_lib = None


class HipExtensionError(RuntimeError):
    pass


class Glue(ctypes.Structure):
    """isa_ekv_glue: device pointers (0 = step skipped) and clamp bounds of the layer glue."""

    _fields_ = [
        ("in_affine", ctypes.c_void_p),
        ("in_lo", ctypes.c_float),
        ("in_hi", ctypes.c_float),
        ("r_tia", ctypes.c_void_p),
        ("y_lo", ctypes.c_float),
        ("y_hi", ctypes.c_float),
        ("adc_scale", ctypes.c_void_p),
        ("adc_shift", ctypes.c_void_p),
        ("stat_abs_max", ctypes.c_void_p),
        ("stat_total", ctypes.c_void_p),
        ("r_log_scale", ctypes.c_void_p),
        ("r_log_lo", ctypes.c_float),
        ("r_log_hi", ctypes.c_float),
    ]


SEG_UNIFORM = 0
SEG_SEARCH = 1
SEG_ROUND = 2


class Codebook(ctypes.Structure):
    """isa_ekv_codebook: measured-curve tables (device pointers) and the segment rule."""

    _fields_ = [
        ("slopes", ctypes.c_void_p),
        ("intercepts", ctypes.c_void_p),
        ("n_seg", ctypes.c_int),
        ("n_rows", ctypes.c_int),
        ("seg_mode", ctypes.c_int),
        ("vg", ctypes.c_void_p),
        ("voltage_min", ctypes.c_float),
        ("inverse_step", ctypes.c_float),
        ("lookup_min", ctypes.c_float),
        ("lookup_max", ctypes.c_float),
    ]


class GlueGrads(ctypes.Structure):
    """isa_ekv_glue_grads: device pointers for the glue parameters' gradients (0 = not needed)."""

    _fields_ = [
        ("in_affine", ctypes.c_void_p),
        ("r_tia", ctypes.c_void_p),
        ("adc_scale", ctypes.c_void_p),
        ("adc_shift", ctypes.c_void_p),
        ("r_log_scale", ctypes.c_void_p),
    ]


def _declare(lib) -> None:
    vp = ctypes.c_void_p
    i64 = ctypes.c_int64
    f32 = ctypes.c_float
    f64 = ctypes.c_double
    ci = ctypes.c_int
    sz = ctypes.c_size_t
    lib.isa_ekv_abi_version.argtypes = []
    lib.isa_ekv_abi_version.restype = ci
    lib.isa_ekv_last_error.argtypes = []
    lib.isa_ekv_last_error.restype = ctypes.c_char_p
    lib.isa_ekv_lut_pad.argtypes = []
    lib.isa_ekv_lut_pad.restype = ci
    lib.isa_ekv_lut_bytes.argtypes = [ci, ci]
    lib.isa_ekv_lut_bytes.restype = sz
    lib.isa_ekv_lut_build.argtypes = [ctypes.POINTER(f64), f64, f64, ci, ci, vp, vp]
    lib.isa_ekv_lut_build.restype = ci
    lib.isa_ekv_lut_pack.argtypes = [vp, vp, ci, ci, ci, vp, vp]
    lib.isa_ekv_lut_pack.restype = ci
    lib.isa_ekv_forward_workspace.argtypes = [i64, i64, i64]
    lib.isa_ekv_forward_workspace.restype = sz
    lib.isa_ekv_forward.argtypes = [vp, vp, vp, vp, i64, i64, i64, ci, f32, f32, f32, f32, f32, vp, vp, sz, vp]
    lib.isa_ekv_forward.restype = ci
    lib.isa_ekv_forward_noalloc.argtypes = [vp, vp, vp, vp, i64, i64, i64, ci, f32, f32, f32, f32, f32, vp, vp]
    lib.isa_ekv_forward_noalloc.restype = ci
    lib.isa_ekv_backward_workspace.argtypes = [i64, i64, i64, ci, ci, ci]
    lib.isa_ekv_backward_workspace.restype = sz
    lib.isa_ekv_backward.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, ci, f32, f32, f32, vp, vp, vp, vp, sz, vp]
    lib.isa_ekv_backward.restype = ci
    lib.isa_ekv_exact_forward_workspace.argtypes = [i64, i64, i64]
    lib.isa_ekv_exact_forward_workspace.restype = sz
    lib.isa_ekv_exact_forward.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.POINTER(f64), f32, vp, vp, sz, vp]
    lib.isa_ekv_exact_forward.restype = ci
    lib.isa_ekv_exact_backward_workspace.argtypes = [i64, i64, i64, ci, ci]
    lib.isa_ekv_exact_backward_workspace.restype = sz
    lib.isa_ekv_exact_backward.argtypes = [vp, vp, vp, vp, i64, i64, i64, ctypes.POINTER(f64), f32,
                                           vp, vp, vp, vp, sz, vp]
    lib.isa_ekv_exact_backward.restype = ci
    lib.isa_ekv_layer_forward_workspace.argtypes = [i64, i64, i64]
    lib.isa_ekv_layer_forward_workspace.restype = sz
    lib.isa_ekv_layer_backward_workspace.argtypes = [i64, i64, i64, ci, ci, ci]
    lib.isa_ekv_layer_backward_workspace.restype = sz
    lib.isa_ekv_layer_forward.argtypes = [vp, vp, vp, vp, i64, i64, i64, ci, f32, f32, f32, f32, f32,
                                          ctypes.POINTER(Glue), vp, vp, vp, sz, vp]
    lib.isa_ekv_layer_forward.restype = ci
    lib.isa_ekv_layer_backward.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, f32, f32, f32,
                                           ctypes.POINTER(Glue), vp, vp, vp, ctypes.POINTER(GlueGrads), vp, sz, vp]
    lib.isa_ekv_layer_backward.restype = ci
    lib.isa_ekv_measured_forward_workspace.argtypes = [i64, i64, i64, ci, ci]
    lib.isa_ekv_measured_forward_workspace.restype = sz
    lib.isa_ekv_measured_backward_workspace.argtypes = [i64, i64, i64, ci, ci]
    lib.isa_ekv_measured_backward_workspace.restype = sz
    lib.isa_ekv_measured_forward.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.POINTER(Codebook), f32, vp, f32, f32,
                                             vp, vp, vp, sz, vp]
    lib.isa_ekv_measured_forward.restype = ci
    lib.isa_ekv_measured_backward.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.POINTER(Codebook), f32, vp, vp, vp,
                                              f32, f32, vp, vp, sz, vp]
    lib.isa_ekv_measured_backward.restype = ci
    lib.isa_ekv_profile_begin.argtypes = []
    lib.isa_ekv_profile_begin.restype = ci
    lib.isa_ekv_profile_end.argtypes = [ctypes.POINTER(f64), ctypes.POINTER(ci)]
    lib.isa_ekv_profile_end.restype = ci
    lib.isa_ekv_probe_lds_gather.argtypes = [ci, ci, ci, vp, i64, ctypes.POINTER(ci), vp, ctypes.POINTER(ci), vp]
    lib.isa_ekv_probe_lds_gather.restype = ci
    lib.isa_ekv_profile_clock.argtypes = [ctypes.POINTER(f64)]
    lib.isa_ekv_profile_clock.restype = ci
    lib.isa_ekv_probe_valu_issue.argtypes = [ci, ci, vp, vp, i64, vp, ctypes.POINTER(f64), ctypes.POINTER(ci), vp]
    lib.isa_ekv_probe_valu_issue.restype = ci
    lib.isa_ekv_plan_info.argtypes = [ci, i64, i64, i64, ci, ci, ci, ctypes.POINTER(i64), ci]
    lib.isa_ekv_plan_info.restype = ci
    lib.isa_ekv_set_option.argtypes = [ci, i64, ctypes.POINTER(i64)]
    lib.isa_ekv_set_option.restype = ci


def load(path: Path | None = None):
    """Load and cache the library; raise HipExtensionError if it is absent or mismatched."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise HipExtensionError(
                f"{LIB_NAME} not found at {p}; build it with `python isa-_amd/csrc/build.py` "
                "(or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(p))
        missing = [name for name in EXPORTS if not hasattr(lib, name)]
        if missing:
            raise HipExtensionError(f"{p} lacks exports {missing}")
        _declare(lib)
        version = lib.isa_ekv_abi_version()
        if version != ABI_VERSION:
            raise HipExtensionError(f"{p} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Raise RuntimeError carrying the library's message for a nonzero status."""
    if rc != 0:
        msg = load().isa_ekv_last_error()
        text = msg.decode("utf-8", "replace") if msg else ""
        raise RuntimeError(f"{what} failed ({rc}): {text}")


class KernelTimer:
    """Context manager summing HIP-event durations the library records: main kernels
    (fwd_ms, bwd_ms) and whole calls including prep and reductions (fwd_call_ms, bwd_call_ms);
    and the mean shader clock the LUT main kernels' blocks ran at (clocks)."""

    def __enter__(self):
        check(load().isa_ekv_profile_begin(), "isa_ekv_profile_begin")
        return self

    def __exit__(self, *exc):
        ms = (ctypes.c_double * 4)()
        n = (ctypes.c_int * 4)()
        rc = load().isa_ekv_profile_end(ms, n)
        self.fwd_ms, self.bwd_ms, self.fwd_call_ms, self.bwd_call_ms = ms
        self.fwd_launches, self.bwd_launches, self.fwd_calls, self.bwd_calls = n
        check(rc, "isa_ekv_profile_end")
        clk = (ctypes.c_double * 12)()
        check(load().isa_ekv_profile_clock(clk), "isa_ekv_profile_clock")
        # per LUT main kernel, the mean shader clock (GHz) of its blocks, their count and their
        # summed seconds (None / 0 when none ran)
        self.clocks = {}
        for name, k in (("fwd_kernel", 0), ("bwd_kernel", 1), ("bwd_two_copies_kernel", 2),
                        ("bwd_ranked_kernel", 3)):
            cyc, sec, blocks = clk[3 * k], clk[3 * k + 1], clk[3 * k + 2]
            self.clocks[name] = {"ghz": cyc / sec / 1e9 if sec > 0 else None, "blocks": int(blocks),
                                 "block_seconds": sec}
        return False


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The hipStream_t of the device's current stream (the raw handle without building a
    torch.cuda.Stream object where torch offers it: a few microseconds per call)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


class on_device:
    """torch.cuda.device(device) that skips the device switch when it is already current."""

    __slots__ = ("index", "prev")

    def __init__(self, device):
        device = device if isinstance(device, torch.device) else torch.device(device)
        self.index = device.index if device.index is not None else torch.cuda.current_device()
        self.prev = -1

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.index:
            self.prev = cur
            torch.cuda.set_device(self.index)
        return self

    def __exit__(self, *exc):
        if self.prev >= 0:
            torch.cuda.set_device(self.prev)
        return False
