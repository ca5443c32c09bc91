"""4-bit and 8-bit code tables (oracle, test infrastructure only).

The reference builds its codebook with ``bitsandbytes.functional.get_4bit_type`` /
``create_dynamic_map`` (``experts4bit_qlora/_vendor/experts.py:61-77``, ``code`` buffer at
``:276``). bitsandbytes is not installed here, so the tables are restated from their
published definitions, and each restatement is pinned by a second, independent derivation:

* ``NF4_CODE`` -- the 16 fp32 literals of the QLoRA NormalFloat4 table (QLoRA paper,
  App. E; bitsandbytes ``get_4bit_type("nf4")``). Pinned by ``normal_map_nf4()``, which
  rebuilds it from the published construction (bitsandbytes ``create_normal_map`` with
  ``offset=0.9677083``, ``use_extra_value=True``) and must agree bit for bit.
* ``FP4_CODE`` -- bitsandbytes' fp4 table (``get_4bit_type("fp4")``: sign + the raw values
  ``[0, 0.0625, 8, 12, 4, 6, 2, 3]``, divided by their max). Pinned by ``fp4_tree_value``,
  the published CUDA decode of the same format (bitsandbytes ``csrc/kernels.cu``,
  ``dDequantizeFP4Tree``: a bit-by-bit decision tree over the nibble with the normalised
  values written out), which must agree bit for bit.
* ``dynamic_map_signed()`` -- bitsandbytes ``create_dynamic_map(signed=True,
  max_exponent_bits=7, total_bits=8)``, the second-level code of double quantization.
  Pinned by ``dynamic_map_exact()``: the same table in exact rational arithmetic (entry
  ``(i, j)`` is ``10**(i-6) * (0.1 + (j + 1/2) * 0.9 / 2**i)``, the midpoint of the ``j``-th
  cell of an ``2**i``-cell grid over [0.1, 1] in decade ``i``). Every fp32 entry lies within
  2 ulp of its exact value (the fp32 linspace, midpoint and scale roundings), and selected
  entries of every decade carry hand-derived fp32 bit patterns (``DYNAMIC_MAP_PINS``).
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
    ``linspace(0.1, 1, 2**i + 1)`` grid (torch fp32), scales them by
    ``10**(i - max_exponent_bits + 1)`` and adds them with both signs; then ``0`` and ``1.0``;
    sorted ascending. Pinned against ``dynamic_map_exact`` and ``DYNAMIC_MAP_PINS``.
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


def dynamic_map_exact(max_exponent_bits: int = 7) -> list:
    """The signed dynamic map in exact rational arithmetic, sorted ascending (256 Fractions).

    Decade ``i`` (``0 <= i < max_exponent_bits``) splits [0.1, 1] into ``2**i`` equal cells
    and takes each cell's midpoint, scaled by ``10**(i - max_exponent_bits + 1)``, with both
    signs; then 0 and 1. This is the value the fp32 construction approximates.
    """
    from fractions import Fraction

    vals = [Fraction(0), Fraction(1)]
    lo, hi = Fraction(1, 10), Fraction(1)
    for i in range(max_exponent_bits):
        cells = 2 ** i
        scale = Fraction(10) ** (i - max_exponent_bits + 1)
        for j in range(cells):
            mid = lo + (hi - lo) * (2 * j + 1) / (2 * cells)
            vals += [scale * mid, -scale * mid]
    return sorted(vals)


# (index into the sorted table, fp32 bits): the first and last cell of every decade, derived
# step by step in fp32 from the construction (start 0.1f, step fl32(1 - 0.1f) / 2**i, boundary
# start + step or 1 - step, midpoint fl32(a + b) / 2, scale fl32(10**(i-6)) times the
# midpoint); tests/test_oracle.py repeats that derivation in numpy. Index 127 is the exact 0,
# 255 the appended 1.0; the positive half holds decade i's 2**i midpoints at sorted indices
# 128 + 2**i - 1 ... 128 + 2**(i+1) - 2. (Mid-grid entries of the larger decades depend on the
# evaluation order of the fp32 linspace -- torch's vectorised kernel -- by up to 1 ulp; the
# exact-value check bounds every entry at 2 ulp.)
DYNAMIC_MAP_PINS = {
    0: 0xBF7E3333,    # -(decade 6, cell 63) = -0.99296874
    127: 0x00000000,  # the appended 0
    128: 0x3513A3B7,  # decade 0, cell 0: 1e-6 * 0.55       -> 5.5000004e-07
    129: 0x365A1A94,  # decade 1, cell 0: 1e-5 * 0.325      -> 3.2500002e-06
    130: 0x370205FF,  # decade 1, cell 1: 1e-5 * 0.775      -> 7.75e-06
    131: 0x37B24206,  # decade 2, cell 0: 1e-4 * 0.2125     -> 2.1249998e-05
    134: 0x38BA1F4B,  # decade 2, cell 3: 1e-4 * 0.8875     -> 8.875e-05
    135: 0x3923D70B,  # decade 3, cell 0: 1e-3 * 0.15625    -> 1.5625001e-04
    142: 0x3A7765FF,  # decade 3, cell 7: 1e-3 * 0.94375    -> 9.4375008e-04
    143: 0x3AA7EF9D,  # decade 4, cell 0: 1e-2 * 0.128125   -> 1.2812499e-03
    158: 0x3C1F3B64,  # decade 4, cell 15: 1e-2 * 0.971875  -> 9.7187497e-03
    159: 0x3C3AE148,  # decade 5, cell 0: 1e-1 * 0.1140625  -> 1.1406250e-02
    190: 0x3DC9EB85,  # decade 5, cell 31: 1e-1 * 0.9859375 -> 9.8593749e-02
    191: 0x3DDB3334,  # decade 6, cell 0: 0.10703125        -> 1.0703126e-01
    254: 0x3F7E3333,  # decade 6, cell 63: 0.99296875       -> 9.9296874e-01
    255: 0x3F800000,  # the appended 1.0
}


def fp4_tree_value(nibble: int) -> float:
    """bitsandbytes' fp4 nibble decode as its published CUDA decision tree spells it out
    (``dDequantizeFP4Tree``): bit 3 is the sign; bits 2..0 select the normalised magnitude."""
    sign = -1.0 if nibble & 0b1000 else 1.0
    if nibble & 0b0100:
        if nibble & 0b0010:
            mag = 0.25000000 if nibble & 0b0001 else 0.16666667
        else:
            mag = 0.50000000 if nibble & 0b0001 else 0.33333333
    else:
        if nibble & 0b0010:
            mag = 1.00000000 if nibble & 0b0001 else 0.66666667
        else:
            mag = 5.208333333e-03 if nibble & 0b0001 else 0.0
    return float(np.float32(sign) * np.float32(mag))


def code_for(quant_type: str) -> np.ndarray:
    if quant_type == "nf4":
        return NF4_CODE.copy()
    if quant_type == "fp4":
        return FP4_CODE.copy()
    raise ValueError(f"no 4-bit code table for {quant_type!r}")
