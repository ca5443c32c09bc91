"""ctypes binding of ``libe4b_amd.so`` (the C ABI declared in ``include/e4b_amd.h``).

The shared library is built in-tree by :func:`experts4bit_qlora_amd._build.build` (``hipcc
--offload-arch=gfx950``) and loaded from this package directory. Nothing here falls back to
another implementation: :func:`lib` raises :class:`NativeUnavailable` when the library is
missing, and every non-zero status from the library is raised as :class:`NativeError` with the
library's own message.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libe4b_amd.so"
LIB_PATH = os.path.join(_HERE, LIB_NAME)

# enums mirrored from include/e4b_amd.h
E4B_OK = 0
FMT_NF4, FMT_NF4_DQ, FMT_MXFP4 = 0, 1, 2
BF16, FP16, FP32 = 0, 1, 2
EPI_NONE, EPI_SWIGLU, EPI_ACT, EPI_CLAMP_SWIGLU, EPI_GPTOSS = 0, 1, 2, 3, 4
# e4b_probe_site: launch sites of the prefill path that e4b_set_probe can watch
PROBE_OFF, PROBE_GATE_UP_BIG, PROBE_GATE_UP_TAIL, PROBE_DOWN_BIG, PROBE_DOWN_TAIL = 0, 1, 2, 3, 4
PATH_AUTO, PATH_GEMV, PATH_MFMA = 0, 1, 2
NOALLOC_WORKSPACE_BYTES = 64 << 20  # E4B_NOALLOC_WORKSPACE_BYTES

# every symbol include/e4b_amd.h declares (tests check the library exports all of them)
EXPORTS = (
    "e4b_version",
    "e4b_last_error",
    "e4b_mfma_tile_m",
    "e4b_dequant",
    "e4b_weight_shift",
    "e4b_route_scratch_ints",
    "e4b_route",
    "e4b_route_groups",
    "e4b_gather_rows",
    "e4b_grouped_gemm",
    "e4b_combine",
    "e4b_lora_delta",
    "e4b_lora_delta_epilogue",
    "e4b_lora_t",
    "e4b_lora_t_add",
    "e4b_lora_wgrad",
    "e4b_grouped_dgrad",
    "e4b_decode_gate_up",
    "e4b_decode_down_combine",
    "e4b_moe_workspace_bytes",
    "e4b_moe_forward",
    "e4b_moe_forward_noalloc",
    "e4b_moe_lora_workspace_bytes",
    "e4b_moe_lora_forward",
    "e4b_set_probe",
)


class NativeUnavailable(RuntimeError):
    """The HIP library is not built (run ``__graft_entry__.build()``) or cannot be loaded."""


class NativeError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


class QWeight(ctypes.Structure):
    _fields_ = [
        ("format", ctypes.c_int32),
        ("num_experts", ctypes.c_int32),
        ("n", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("packed", ctypes.c_void_p),
        ("absmax", ctypes.c_void_p),
        ("absmax2", ctypes.c_void_p),
        ("offset", ctypes.c_void_p),
        ("code", ctypes.c_void_p),
        ("code2", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("shift", ctypes.c_void_p),
    ]


class Lora(ctypes.Structure):
    """``e4b_lora``: the four adapter matrices of an ExpertsLoRA, their dtype, rank and scaling."""
    _fields_ = [
        ("a1", ctypes.c_void_p),
        ("b1", ctypes.c_void_p),
        ("a2", ctypes.c_void_p),
        ("b2", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("scaling", ctypes.c_float),
    ]


class Routing(ctypes.Structure):
    _fields_ = [
        ("sorted_flat", ctypes.c_void_p),
        ("inv", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
        ("active", ctypes.c_void_p),
        ("tiles", ctypes.c_void_p),
        ("meta", ctypes.c_void_p),
        ("max_tiles", ctypes.c_int32),
        ("tile_m", ctypes.c_int32),
        ("scratch", ctypes.c_void_p),
    ]


_lib = None
_load_error: str | None = None


def _bind(L):
    P, I32, I64, F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    QW, RT = ctypes.POINTER(QWeight), ctypes.POINTER(Routing)
    L.e4b_version.restype = ctypes.c_char_p
    L.e4b_version.argtypes = []
    L.e4b_last_error.restype = ctypes.c_char_p
    L.e4b_last_error.argtypes = []
    L.e4b_mfma_tile_m.restype = I32
    L.e4b_mfma_tile_m.argtypes = []
    L.e4b_dequant.restype = ctypes.c_int
    L.e4b_dequant.argtypes = [QW, I32, I32, I32, P, P]
    L.e4b_weight_shift.restype = ctypes.c_int
    L.e4b_weight_shift.argtypes = [QW, P, P]
    L.e4b_route_scratch_ints.restype = I64
    L.e4b_route_scratch_ints.argtypes = [I64, I32]
    L.e4b_route.restype = ctypes.c_int
    L.e4b_route.argtypes = [P, I64, I32, I32, RT, P]
    L.e4b_route_groups.restype = ctypes.c_int
    L.e4b_route_groups.argtypes = [ctypes.POINTER(ctypes.c_int64), I32, P, I32, RT, P]
    L.e4b_gather_rows.restype = ctypes.c_int
    L.e4b_gather_rows.argtypes = [P, I64, I64, P, P, P, I32, I64, P, P]
    L.e4b_grouped_gemm.restype = ctypes.c_int
    L.e4b_grouped_gemm.argtypes = [P, I32, I32, QW, RT, I64, I64, I32, F32, F32, I32, P, I32, P]
    L.e4b_combine.restype = ctypes.c_int
    L.e4b_combine.argtypes = [P, I32, P, P, I32, I64, I32, I64, P, I32, P]
    L.e4b_lora_delta.restype = ctypes.c_int
    L.e4b_lora_delta.argtypes = [P, I32, I32, RT, I64, I32, P, P, I32, I32, I64, I64, F32, I32,
                                 P, P, P]
    L.e4b_lora_delta_epilogue.restype = ctypes.c_int
    L.e4b_lora_delta_epilogue.argtypes = [P, I32, I32, RT, I64, I32, P, P, I32, I32, I64, I64, F32, I32, P, P,
                                          I32, F32, P, I32, P]
    L.e4b_lora_t.restype = ctypes.c_int
    L.e4b_lora_t.argtypes = [P, I32, I32, RT, I64, I32, P, I32, I32, I64, P, P]
    L.e4b_lora_t_add.restype = ctypes.c_int
    L.e4b_lora_t_add.argtypes = [P, RT, I64, I32, P, I32, I32, I64, F32, I32, P, P]
    L.e4b_lora_wgrad.restype = ctypes.c_int
    L.e4b_lora_wgrad.argtypes = [P, I32, P, I32, I32, RT, I64, I32, I64, F32, P, P]
    L.e4b_grouped_dgrad.restype = ctypes.c_int
    L.e4b_grouped_dgrad.argtypes = [P, I32, QW, RT, I64, P, P]
    L.e4b_decode_gate_up.restype = ctypes.c_int
    L.e4b_decode_gate_up.argtypes = [P, I32, I64, P, I32, QW, I32, F32, F32, P, P]
    L.e4b_decode_down_combine.restype = ctypes.c_int
    L.e4b_decode_down_combine.argtypes = [P, I32, I64, P, P, I32, I32, QW, P, I32, P]
    L.e4b_moe_workspace_bytes.restype = ctypes.c_size_t
    L.e4b_moe_workspace_bytes.argtypes = [I64, I32, I32, I64, I64, I32, I32]
    L.e4b_moe_forward.restype = ctypes.c_int
    L.e4b_moe_forward.argtypes = [P, I32, I64, P, P, I32, I32, QW, QW, I32, F32, F32, I32, P, ctypes.c_size_t, P,
                                  I32, P]
    L.e4b_moe_forward_noalloc.restype = ctypes.c_int
    L.e4b_moe_forward_noalloc.argtypes = [P, I32, I64, P, P, I32, I32, QW, QW, I32, F32, F32, I32, P, I32, P]
    L.e4b_moe_lora_workspace_bytes.restype = ctypes.c_size_t
    L.e4b_moe_lora_workspace_bytes.argtypes = [I64, I32, I32, I64, I64, I32, I32, I32]
    L.e4b_moe_lora_forward.restype = ctypes.c_int
    L.e4b_moe_lora_forward.argtypes = [P, I32, I64, P, P, I32, I32, QW, QW, ctypes.POINTER(Lora), I32, F32, I32, P,
                                       ctypes.c_size_t, P, I32, P]
    L.e4b_set_probe.restype = ctypes.c_int
    L.e4b_set_probe.argtypes = [I32, P, P]
    return L


def load(path: str | None = None):
    """Load (once) and return the library, or None with the reason kept for :func:`lib`."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        _load_error = f"{p} is not built (run __graft_entry__.build())"
        return None
    try:
        _lib = _bind(ctypes.CDLL(p))
    except OSError as e:  # pragma: no cover - broken build
        _load_error = f"cannot load {p}: {e}"
        return None
    return _lib


def available() -> bool:
    return load() is not None


def lib():
    L = load()
    if L is None:
        raise NativeUnavailable(f"the MI355X kernel library is unavailable: {_load_error}")
    return L


def check(fn: str, status: int) -> None:
    if status != E4B_OK:
        msg = lib().e4b_last_error().decode(errors="replace")
        raise NativeError(fn, status, msg)
