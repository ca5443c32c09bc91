"""Blockwise 4-bit storage: NF4 (fp32 or double-quant absmax) and MXFP4 (oracle only).

Layouts restated from the reference:

* NF4 (``experts4bit_qlora/_vendor/experts.py:244-276`` storage, ``:398-426``
  ``_quantize_stack``): each expert's ``[out, in]`` weight is flattened row-major and
  quantized on its own; two values per byte with the FIRST (even) element in the HIGH
  nibble (``experts4bit_qlora/engines/cold_engine.py:104-115``); one fp32 absmax per 64
  consecutive elements (``compress_statistics=False``, ``_vendor/experts.py:415``). ``in``
  is a multiple of the blocksize (``:220-226``), so blocks never straddle rows or experts.
* Dequant (``_vendor/experts.py:428-457`` -> bitsandbytes ``dequantize_4bit``; the pure-torch
  equivalent at ``cold_engine.py:104-115``): ``W = dtype(code[nib] * absmax[block])`` -- an
  fp32 product, then one round-to-nearest-even into the output dtype.
* Double-quant absmax (not in the reference, which passes ``compress_statistics=False``;
  restated from bitsandbytes' nested ``QuantState``): ``offset = mean(absmax)``; the centred
  absmax is quantized blockwise (256 per block) with the signed dynamic map;
  ``absmax = fp32(fp32(code2[q] * absmax2[block // 256]) + offset)``.
* MXFP4 (``experts4bit_qlora/formats/mxfp4.py:29-105``): e2m1 nibbles, LOW nibble first,
  one e8m0 exponent (bias 127) per 32 values, ``ldexp`` scaling; the reference returns the
  trailing ``(rows, K)`` pair transposed.
"""
from __future__ import annotations

import numpy as np

from .codes import NF4_CODE, dynamic_map_signed
from .numerics import round_to

FP4_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)


# ----------------------------------------------------------------------------- NF4


def unpack_nibbles_hi_first(packed: np.ndarray) -> np.ndarray:
    """uint8 [..., nb] -> uint8 [..., 2*nb]; element 2j is the HIGH nibble of byte j."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p >> 4
    out[..., 1::2] = p & 0xF
    return out


def pack_nibbles_hi_first(idx: np.ndarray) -> np.ndarray:
    idx = np.asarray(idx, dtype=np.uint8)
    return ((idx[..., 0::2] << 4) | (idx[..., 1::2] & 0xF)).astype(np.uint8)


def dequant_nf4(packed, absmax, code=NF4_CODE, blocksize: int = 64, dtype: str = "fp32") -> np.ndarray:
    """Decode a flat NF4 stream: ``packed [..., n/2] u8``, ``absmax [..., n/blocksize] f32``.

    Restates ``cold_engine.py:104-115`` (high nibble first, ``code[idx] * absmax`` in fp32) and
    the output cast of bitsandbytes' ``dequantize_4bit`` (``_vendor/experts.py:447-457``).
    Returns fp32 values already rounded to ``dtype``.
    """
    idx = unpack_nibbles_hi_first(packed)
    vals = np.asarray(code, dtype=np.float32)[idx]
    n = vals.shape[-1]
    am = np.asarray(absmax, dtype=np.float32)
    if am.shape[-1] * blocksize != n:
        raise ValueError(f"absmax has {am.shape[-1]} blocks for {n} values at blocksize {blocksize}")
    prod = (vals.reshape(vals.shape[:-1] + (n // blocksize, blocksize)) * am[..., None]).astype(np.float32)
    return round_to(prod.reshape(vals.shape), dtype)


def _nearest_sorted(code: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Index of the nearest entry of a sorted fp32 table (ties to the lower index)."""
    code = np.asarray(code, dtype=np.float32)
    mids = ((code[:-1].astype(np.float64) + code[1:].astype(np.float64)) / 2.0).astype(np.float32)
    return np.searchsorted(mids, x, side="left").astype(np.uint8)


def quantize_nf4(w, code=NF4_CODE, blocksize: int = 64):
    """Blockwise 4-bit quantization of a flat fp32 stream (input generation only).

    absmax = max |x| per block; x is scaled by ``1/absmax`` in fp32 and mapped to the nearest
    code value (midpoint thresholds). An all-zero block maps to the code's zero. The exact byte
    choices of bitsandbytes' quantizer are not pinned here; the dequant-parity requirement is
    per given bytes.
    """
    w = np.asarray(w, dtype=np.float32)
    n = w.shape[-1]
    if n % blocksize:
        raise ValueError(f"{n} values are not a multiple of blocksize {blocksize}")
    blk = w.reshape(w.shape[:-1] + (n // blocksize, blocksize))
    absmax = np.abs(blk).max(axis=-1).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(absmax > 0, np.float32(1.0) / absmax, np.float32(0.0)).astype(np.float32)
    scaled = (blk * inv[..., None]).astype(np.float32)
    idx = _nearest_sorted(code, scaled)
    zero_idx = int(np.argmin(np.abs(np.asarray(code, dtype=np.float32))))
    idx = np.where((absmax > 0)[..., None], idx, np.uint8(zero_idx))
    packed = pack_nibbles_hi_first(idx.reshape(w.shape))
    return packed, absmax


# ------------------------------------------------------------------- double quant


def double_quant_absmax(absmax, blocksize2: int = 256, code2=None):
    """Compress per-expert fp32 absmax ``[..., nb]`` to (u8 codes, fp32 absmax2, fp32 offset).

    ``offset`` is the mean of the absmax (accumulated in fp64, stored fp32); the centred values
    are quantized blockwise (``blocksize2`` per block) to the nearest entry of the signed
    dynamic map after scaling by ``1/absmax2``. Input generation only: bitsandbytes' own double
    quantizer (not importable here) may pick other bytes for the same absmax, which does not
    matter for parity -- that is defined per given bytes, and the decode of (codes, absmax2,
    offset, code2) is pinned.
    """
    if code2 is None:
        code2 = dynamic_map_signed()
    a = np.asarray(absmax, dtype=np.float32)
    offset = a.astype(np.float64).mean(axis=-1).astype(np.float32)
    centred = (a - offset[..., None]).astype(np.float32)
    nb = a.shape[-1]
    nb2 = -(-nb // blocksize2)
    pad = nb2 * blocksize2 - nb
    c = np.concatenate([centred, np.zeros(a.shape[:-1] + (pad,), np.float32)], axis=-1)
    c = c.reshape(a.shape[:-1] + (nb2, blocksize2))
    absmax2 = np.abs(c).max(axis=-1).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(absmax2 > 0, np.float32(1.0) / absmax2, np.float32(0.0)).astype(np.float32)
    q = _nearest_sorted(code2, (c * inv[..., None]).astype(np.float32))
    q = q.reshape(a.shape[:-1] + (nb2 * blocksize2,))[..., :nb]
    return q.astype(np.uint8), absmax2, offset


def dequant_absmax_dq(q, absmax2, offset, code2=None, blocksize2: int = 256) -> np.ndarray:
    """``absmax[b] = fp32(fp32(code2[q[b]] * absmax2[b // blocksize2]) + offset)``."""
    if code2 is None:
        code2 = dynamic_map_signed()
    q = np.asarray(q, dtype=np.uint8)
    nb = q.shape[-1]
    a2 = np.repeat(np.asarray(absmax2, np.float32), blocksize2, axis=-1)[..., :nb]
    prod = (np.asarray(code2, np.float32)[q] * a2).astype(np.float32)
    return (prod + np.asarray(offset, np.float32)[..., None]).astype(np.float32)


# ----------------------------------------------------------------------------- MXFP4


def e8m0_scale(scales) -> np.ndarray:
    """2**(s - 127) as fp32 for an e8m0 byte (0 -> 2**-127, a subnormal; 255 -> inf)."""
    s = np.asarray(scales, dtype=np.int32)
    return np.ldexp(np.float32(1.0), s - 127).astype(np.float32)


def dequant_mxfp4_rows(blocks, scales, dtype: str = "fp32") -> np.ndarray:
    """``blocks [..., rows, G, B] u8``, ``scales [..., rows, G] u8`` -> ``[..., rows, G*2B]``.

    Restates ``formats/mxfp4.py:84-99``: low nibble -> even element, high -> odd, then
    ``ldexp`` by ``scale - 127`` per block. Row-major (not yet transposed).
    """
    blk = np.asarray(blocks, dtype=np.uint8)
    sc = np.asarray(scales, dtype=np.uint8)
    if blk.shape[:-1] != sc.shape:
        raise ValueError(f"blocks.shape[:-1]={blk.shape[:-1]} != scales.shape={sc.shape}")
    vals = np.empty(blk.shape[:-1] + (blk.shape[-1] * 2,), dtype=np.float32)
    vals[..., 0::2] = FP4_VALUES[blk & 0x0F]
    vals[..., 1::2] = FP4_VALUES[blk >> 4]
    with np.errstate(over="ignore", invalid="ignore"):
        out = np.ldexp(vals, (sc.astype(np.int32) - 127)[..., None]).astype(np.float32)
    out = round_to(out, dtype)
    return out.reshape(blk.shape[:-2] + (blk.shape[-2] * blk.shape[-1] * 2,))


def dequantize_mxfp4(blocks, scales, dtype: str = "fp32") -> np.ndarray:
    """The reference API (``formats/mxfp4.py:35-105``): decoded ``[..., K, rows]`` (transposed)."""
    blk = np.asarray(blocks)
    if blk.ndim < 3:
        raise ValueError("blocks must be [..., rows, G, B] with at least one leading row axis")
    rows = dequant_mxfp4_rows(blocks, scales, dtype)
    return np.ascontiguousarray(np.swapaxes(rows, -2, -1))


def quantize_mxfp4(w, group: int = 32):
    """OCP MX quantization of ``[..., K]`` fp32 rows (input generation only).

    Per 32 values: shared exponent ``X = floor(log2(amax)) - 2`` (e2m1's max exponent),
    stored as e8m0 ``X + 127`` clamped to [0, 254]; each ``x / 2**X`` rounds to the nearest
    e2m1 value, ties to the even code, saturating at +-6. Packs low nibble first.
    Returns ``(blocks [..., K/32, 16] u8, scales [..., K/32] u8)``.
    """
    w = np.asarray(w, dtype=np.float32)
    K = w.shape[-1]
    if K % group:
        raise ValueError(f"K={K} is not a multiple of {group}")
    g = w.reshape(w.shape[:-1] + (K // group, group))
    amax = np.abs(g).max(axis=-1)
    with np.errstate(divide="ignore"):
        X = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1.0))) - 2, -127)
    e = np.clip(X + 127, 0, 254).astype(np.int32)
    scaled = (g.astype(np.float64) / np.ldexp(1.0, e - 127)[..., None])
    mag = np.abs(scaled)
    grid = FP4_VALUES[:8].astype(np.float64)
    d = np.abs(mag[..., None] - grid)
    best = np.argmin(d, axis=-1)
    # ties to the even code: if the next code up is equally near and even, prefer it
    dmin = np.take_along_axis(d, best[..., None], axis=-1)[..., 0]
    nxt = np.minimum(best + 1, 7)
    tie = (np.take_along_axis(d, nxt[..., None], axis=-1)[..., 0] == dmin) & (nxt != best) & (best % 2 == 1)
    best = np.where(tie, nxt, best)
    best = np.where(mag > 6.0, 7, best)
    code = (best | np.where((scaled < 0) & (best > 0), 8, 0)).astype(np.uint8)
    code = code.reshape(w.shape)
    packed = ((code[..., 1::2] << 4) | code[..., 0::2]).astype(np.uint8)
    blocks = packed.reshape(w.shape[:-1] + (K // group, group // 2))
    return blocks, e.astype(np.uint8)
