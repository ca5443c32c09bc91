"""4-bit and 8-bit code tables (oracle, test infrastructure only).

The reference builds its codebook with ``bitsandbytes.functional.get_4bit_type`` /
``create_dynamic_map`` (``experts4bit_qlora/_vendor/experts.py:61-77``, ``code`` buffer at
``:276``). bitsandbytes is not installed here, so the tables are restated from their
published definitions:

* ``NF4_CODE`` -- the 16 fp32 literals of the QLoRA NormalFloat4 table (QLoRA paper,
  App. E; bitsandbytes ``get_4bit_type("nf4")``). Pinned by ``normal_map_nf4()``, which
  rebuilds it from the published construction (bitsandbytes ``create_normal_map`` with
  ``offset=0.9677083``, ``use_extra_value=True``) and must agree bit for bit.
* ``FP4_CODE`` -- bitsandbytes' fp4 (e2m1 with bias 3 and a subnormal step) table, divided by
  its max. PARITY UNPINNED: only structural checks; not on the fast path.
* ``dynamic_map_signed()`` -- bitsandbytes ``create_dynamic_map(signed=True,
  max_exponent_bits=7, total_bits=8)``, the second-level code of double quantization.
  PARITY UNPINNED for its exact bits (structural checks only).
"""
from __future__ import annotations

import numpy as np

NF4_CODE = np.array(
    [
        -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
        -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
        0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
        0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
    ],
    dtype=np.float32,
)

_FP4_RAW = [0.0, 0.0625, 8.0, 12.0, 4.0, 6.0, 2.0, 3.0,
            -0.0, -0.0625, -8.0, -12.0, -4.0, -6.0, -2.0, -3.0]
FP4_CODE = (np.array(_FP4_RAW, dtype=np.float32) / np.float32(12.0)).astype(np.float32)


def normal_map_nf4(offset: float = 0.9677083) -> np.ndarray:
    """Rebuild the NF4 table from normal quantiles (the published construction).

    Positive half: ``Phi^-1`` at 8 points of ``linspace(offset, 0.5, 9)[:-1]``; negative half:
    ``-Phi^-1`` at 7 points of ``linspace(offset, 0.5, 8)[:-1]``; plus an exact zero; sorted and
    normalised by the max. The linspace is evaluated in torch fp32, as the published code does.
    """
    import torch
    from scipy.stats import norm

    pos = norm.ppf(torch.linspace(offset, 0.5, 9)[:-1].numpy()).tolist()
    neg = (-norm.ppf(torch.linspace(offset, 0.5, 8)[:-1].numpy())).tolist()
    v = np.array(sorted(pos + [0.0] + neg), dtype=np.float32)
    return (v / v.max()).astype(np.float32)


def dynamic_map_signed(max_exponent_bits: int = 7, total_bits: int = 8) -> np.ndarray:
    """The signed dynamic quantization map (bitsandbytes ``create_dynamic_map``), 256 fp32.

    For exponent level ``i`` in ``0..max_exponent_bits-1`` it takes ``2**i`` midpoints of a
    ``linspace(0.1, 1, 2**i + 1)`` grid, scales them by ``10**(i - max_exponent_bits + 1)`` and
    adds them with both signs; then ``0`` and ``1.0``; sorted ascending.
    """
    import torch

    non_sign_bits = total_bits - 1
    data: list[float] = []
    for i in range(max_exponent_bits):
        fraction_items = int(2 ** (i + non_sign_bits - max_exponent_bits) + 1)
        boundaries = torch.linspace(0.1, 1, fraction_items, dtype=torch.float32)
        means = (boundaries[:-1] + boundaries[1:]) / 2.0
        scale = 10 ** (-(max_exponent_bits - 1) + i)
        data += (scale * means).tolist()
        data += (-scale * means).tolist()
    data.append(0.0)
    data.append(1.0)
    data += [0.0] * (2 ** total_bits - len(data))
    data.sort()
    return np.array(data, dtype=np.float32)


def code_for(quant_type: str) -> np.ndarray:
    if quant_type == "nf4":
        return NF4_CODE.copy()
    if quant_type == "fp4":
        return FP4_CODE.copy()
    raise ValueError(f"no 4-bit code table for {quant_type!r}")
