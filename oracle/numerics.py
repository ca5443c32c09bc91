"""Bit-level float helpers for the oracle (test infrastructure only).

torch's ``Tensor.to(torch.bfloat16)`` and bitsandbytes' ``__float2bfloat16`` both round
fp32 to bf16 to-nearest-even; ``np.float16`` casts round to-nearest-even too. These helpers
restate the bf16 rounding on raw bits so the oracle never depends on a library's bf16 type.
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16), round-to-nearest-even; NaN stays a quiet NaN."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(f)
    out = rounded.astype(np.uint16)
    if nan.any():
        out = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), out)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    """bf16 bit pattern (uint16) -> exact fp32 value."""
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """fp32 value rounded to the nearest bf16, returned as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_fp16(x) -> np.ndarray:
    """fp32 value rounded to the nearest fp16, returned as fp32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    """Round fp32 values to ``dtype`` in {"bf16", "fp16", "fp32"} and return fp32."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp16":
        return round_fp16(x)
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


def silu_f32(x) -> np.ndarray:
    """SiLU evaluated in fp32, as torch evaluates ``F.silu`` on a reduced-precision tensor
    (upcast to fp32, ``x / (1 + exp(-x))``, then the caller rounds)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def sigmoid_f32(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x))).astype(np.float32)
