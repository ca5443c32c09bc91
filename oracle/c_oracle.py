"""ctypes loader for ``oracle/liboracle_c.so`` (test infrastructure only).

The library is the C restatement in ``oracle/c/oracle.c``; ``oracle/Makefile`` builds it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_c.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        L.orc_dequant_4bit.argtypes = [P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P]
        L.orc_dequant_absmax_dq.argtypes = [P, P, ctypes.c_float, P, ctypes.c_int64, ctypes.c_int, P]
        L.orc_dequant_mxfp4.argtypes = [P, P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, P]
        L.orc_route.argtypes = [P, ctypes.c_int64, ctypes.c_int, P, P, P]
        L.orc_route.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def dequant_4bit(packed, absmax, code, blocksize=64, out="fp32") -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8).reshape(-1)
    absmax = np.ascontiguousarray(absmax, np.float32).reshape(-1)
    code = np.ascontiguousarray(code, np.float32)
    n = packed.size * 2
    res = np.empty(n, np.float32 if out == "fp32" else np.uint16)
    lib().orc_dequant_4bit(_p(packed), _p(absmax), _p(code), n, blocksize, 0 if out == "fp32" else 1, _p(res))
    return res


def dequant_absmax_dq(q, absmax2, offset, code2, blocksize2=256) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8).reshape(-1)
    absmax2 = np.ascontiguousarray(absmax2, np.float32).reshape(-1)
    code2 = np.ascontiguousarray(code2, np.float32)
    res = np.empty(q.size, np.float32)
    lib().orc_dequant_absmax_dq(_p(q), _p(absmax2), ctypes.c_float(float(offset)), _p(code2), q.size,
                                blocksize2, _p(res))
    return res


def dequant_mxfp4(blocks, scales, rows, K, out="fp32") -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    scales = np.ascontiguousarray(scales, np.uint8).reshape(-1)
    res = np.empty(rows * K, np.float32 if out == "fp32" else np.uint16)
    lib().orc_dequant_mxfp4(_p(blocks), _p(scales), rows, K, 0 if out == "fp32" else 1, _p(res))
    return res.reshape(rows, K)


def route(flat_idx, num_experts):
    flat = np.ascontiguousarray(flat_idx, np.int64).reshape(-1)
    M = flat.size
    order = np.empty(M, np.int64)
    inv = np.empty(M, np.int64)
    offsets = np.empty(num_experts + 1, np.int64)
    rc = lib().orc_route(_p(flat), M, num_experts, _p(order), _p(inv), _p(offsets))
    if rc != 0:
        raise ValueError(f"orc_route failed ({rc})")
    return order, inv, offsets
