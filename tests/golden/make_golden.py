"""Writes the committed golden fixtures under tests/golden/ (run once; output is data).

* ``mxfp4_transformers.npz`` -- MXFP4 decodes written by transformers'
  ``integrations.mxfp4.convert_moe_packed_tensors`` (the third-party function the reference's
  ``formats/mxfp4.py`` is verified bit-identical against, ``tests/test_mxfp4_dequant.py:54-70``),
  on seeded random blocks/scales at small gpt-oss-shaped slices, in bf16 and fp32.
* ``mxfp4_reference_vector.npz`` -- the reference's own hand-checkable golden vector
  (``tests/test_mxfp4_dequant.py:20-33``): its input bytes and expected values, as data.
* ``nf4_hand.npz`` -- hand-computed NF4 decode vectors (bytes, absmax, expected fp32 values),
  derived below from the code-table definition one nibble at a time.

bf16 arrays are stored as their uint16 bit patterns.
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def mxfp4_transformers():
    from transformers.integrations.mxfp4 import convert_moe_packed_tensors

    out = {}
    cases = [("a", (2, 64, 4, 16), 0), ("b", (1, 32, 90, 16), 1), ("c", (3, 16, 2, 16), 2)]
    for name, shape, seed in cases:
        g = torch.Generator().manual_seed(seed)
        blocks = torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)
        scales = torch.randint(107, 148, shape[:-1], generator=g, dtype=torch.uint8)
        out[f"{name}_blocks"] = blocks.numpy()
        out[f"{name}_scales"] = scales.numpy()
        for dt, tag in ((torch.bfloat16, "bf16"), (torch.float32, "fp32")):
            ref = convert_moe_packed_tensors(blocks.clone(), scales.clone(), dtype=dt)
            out[f"{name}_{tag}"] = bits(ref.contiguous())
    np.savez_compressed(os.path.join(HERE, "mxfp4_transformers.npz"), **out)


def mxfp4_reference_vector():
    # E=1, rows=2, G=1, B=2 bytes; scales 128 (+1) and 126 (-1); expected [1, 4, 2] after transpose
    np.savez_compressed(
        os.path.join(HERE, "mxfp4_reference_vector.npz"),
        blocks=np.array([[[[0x21, 0x30]], [[0x00, 0x54]]]], dtype=np.uint8),
        scales=np.array([[[128], [126]]], dtype=np.uint8),
        expected=np.array([[[1.0, 0.0], [2.0, 0.0], [0.0, 1.0], [3.0, 1.5]]], dtype=np.float32),
    )


def nf4_hand():
    code = np.array([
        -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
        -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
        0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
        0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)
    # one 64-value block with absmax 2.0 (power of two: every product exact), then a block
    # with absmax 0.5; bytes walk all 256 (hi, lo) pairs over four blocks
    data = np.arange(256, dtype=np.uint8)                  # 512 values = 8 blocks
    absmax = np.array([2.0, 0.5, 4.0, 1.0, 0.25, 8.0, 1.5, 3.0], dtype=np.float32)
    expected = np.empty(512, dtype=np.float32)
    for j, byte in enumerate(data):
        hi, lo = int(byte) >> 4, int(byte) & 0xF          # first value rides the high nibble
        expected[2 * j] = np.float32(code[hi]) * absmax[(2 * j) // 64]
        expected[2 * j + 1] = np.float32(code[lo]) * absmax[(2 * j + 1) // 64]
    np.savez_compressed(os.path.join(HERE, "nf4_hand.npz"), packed=data, absmax=absmax, expected=expected)


if __name__ == "__main__":
    mxfp4_transformers()
    mxfp4_reference_vector()
    nf4_hand()
    print("golden fixtures written to", HERE)
