"""MXFP4 (OCP microscaling e2m1) decode for gpt-oss-style fused expert stacks.

Same API and bit-exact output as ``experts4bit_qlora/formats/mxfp4.py:35-105`` (which is
itself bit-identical to transformers' ``convert_moe_packed_tensors``): ``blocks [..., rows, G, B]``
uint8 with two e2m1 nibbles per byte (LOW nibble = first value), ``scales [..., rows, G]`` e8m0
exponents (bias 127), result ``[..., G*2B, rows]`` -- the trailing pair transposed. Storage bytes
are reinterpreted, never value-converted (int8 blocks / float8_e8m0 scales are viewed as uint8).

On a HIP device with 16-byte blocks and 64-value-aligned rows the decode runs the library's
``e4b_dequant`` kernel; otherwise it runs in torch. Both compute ``FP4[nib] * 2**(s-127)`` in fp32
and round once to ``dtype``.
"""
from __future__ import annotations

import torch

from ..quant import FP4_VALUES, dequant_mxfp4_torch


def dequantize_mxfp4(blocks: torch.Tensor, scales: torch.Tensor, *, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    if blocks.shape[:-1] != scales.shape:
        raise ValueError(f"blocks.shape[:-1]={tuple(blocks.shape[:-1])} != scales.shape={tuple(scales.shape)}")
    if blocks.ndim < 3:
        raise ValueError(
            f"blocks must be [..., rows, G, B] with at least one leading row axis; got {tuple(blocks.shape)}. "
            "A single expert projection is [rows, G, B]; gpt-oss fused stacks are [E, rows, G, B].")
    if blocks.dtype != torch.uint8:
        blocks = blocks.view(torch.uint8)
    if scales.dtype != torch.uint8:
        scales = scales.view(torch.uint8)
    *prefix, G, B = blocks.shape
    rows = 1
    for d in prefix:
        rows *= d
    K = G * B * 2
    if blocks.is_cuda and B == 16 and K % 64 == 0:
        from .. import ops

        qw = ops.mxfp4_qweight(blocks.reshape(1, rows, K // 2), scales.reshape(1, rows, G), rows, K, num_experts=1)
        dense = ops.dequant(qw, 0, 1, dtype=dtype)[0]
    elif B == 16:
        dense = dequant_mxfp4_torch(blocks.reshape(rows, K // 2), scales.reshape(rows, G), rows, K, dtype)
    else:
        # general block width: decode value by value
        blk = blocks.reshape(rows * G, B)
        lut = torch.tensor(FP4_VALUES, dtype=torch.float32, device=blk.device)
        vals = torch.empty(rows * G, 2 * B, dtype=torch.float32, device=blk.device)
        vals[:, 0::2] = lut[(blk & 0x0F).long()]
        vals[:, 1::2] = lut[(blk >> 4).long()]
        exp = scales.reshape(rows * G, 1).to(torch.int32) - 127
        dense = torch.ldexp(vals, exp.float()).reshape(rows, K).to(dtype)
    return dense.reshape(*prefix, K).transpose(-2, -1).contiguous()
