"""Blockwise quantization primitives (torch), the storage side of the expert modules.

These build the bytes the kernels read. The reference delegates them to bitsandbytes
(``quantize_4bit`` / ``quantize_blockwise`` at ``experts4bit_qlora/_vendor/experts.py:408-426``,
codebooks at ``:61-77``); bitsandbytes is not part of this build, so the published definitions
are restated here:

* ``NF4_CODE`` -- the QLoRA NormalFloat4 table (normal quantiles, offset 0.9677083).
* ``FP4_CODE`` -- bitsandbytes' fp4 table (``[0, .0625, 8, 12, 4, 6, 2, 3]`` with sign, / 12).
* ``dynamic_map()`` -- the signed 8-bit dynamic map (``create_dynamic_map``), used by the
  ``int8`` scheme and as the second-level code of double quantization.
* ``fp8_map()`` -- the signed e4m3 codebook (``create_fp8_map(True, 4, 3, 8)``).

Quantizers pick the nearest code after scaling a block by ``1 / absmax`` (fp32). Dequantizers
are exact: one fp32 product ``code[idx] * absmax`` and one rounding into the output dtype.
On a HIP device the 4-bit dequantizers run the library's ``e4b_dequant`` kernel.
"""
from __future__ import annotations

import torch

NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)
_FP4_RAW = (0.0, 0.0625, 8.0, 12.0, 4.0, 6.0, 2.0, 3.0, -0.0, -0.0625, -8.0, -12.0, -4.0, -6.0, -2.0, -3.0)

# e2m1 grid, index = nibble (formats/mxfp4.py:29-32)
FP4_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)

_DQ_BLOCKSIZE2 = 256


def code_4bit(quant_type: str, device=None) -> torch.Tensor:
    if quant_type == "nf4":
        return torch.tensor(NF4_CODE, dtype=torch.float32, device=device)
    if quant_type == "fp4":
        t = torch.tensor(_FP4_RAW, dtype=torch.float32)
        return (t / t.abs().max()).to(device)
    raise ValueError(f"no 4-bit code for {quant_type!r}")


def dynamic_map(signed: bool = True, max_exponent_bits: int = 7, total_bits: int = 8) -> torch.Tensor:
    """Signed dynamic quantization map: per exponent level ``i`` the midpoints of a
    ``linspace(0.1, 1, 2**i + 1)`` grid scaled by ``10**(i - max_exponent_bits + 1)``, both
    signs, plus 0 and 1; sorted (256 fp32)."""
    non_sign_bits = total_bits - (1 if signed else 0)
    data: list[float] = []
    for i in range(max_exponent_bits):
        items = int(2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed
                    else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1)
        b = torch.linspace(0.1, 1, items, dtype=torch.float32)
        means = (b[:-1] + b[1:]) / 2.0
        scale = 10 ** (-(max_exponent_bits - 1) + i)
        data += (scale * means).tolist()
        if signed:
            data += (-scale * means).tolist()
    data.append(0.0)
    data.append(1.0)
    data += [0.0] * (2 ** total_bits - len(data))
    data.sort()
    return torch.tensor(data, dtype=torch.float32)


def fp8_map(signed: bool = True, exponent_bits: int = 4, precision_bits: int = 3, total_bits: int = 8) -> torch.Tensor:
    """A signed minifloat codebook (e4m3 by default): every value of the format with the IEEE
    bias ``2**(e-1) - 1`` and subnormals, normalised by its max (256 entries, sorted)."""
    bias = 2 ** (exponent_bits - 1) - 1
    vals = set()
    for e in range(2 ** exponent_bits):
        for m in range(2 ** precision_bits):
            if e == 0:
                v = (m / 2 ** precision_bits) * 2 ** (1 - bias)
            else:
                v = (1 + m / 2 ** precision_bits) * 2 ** (e - bias)
            vals.add(v)
            if signed:
                vals.add(-v)
    out = sorted(vals)
    t = torch.tensor(out, dtype=torch.float32)
    t = t / t.abs().max()
    if t.numel() < 2 ** total_bits:
        t = torch.cat([t, torch.zeros(2 ** total_bits - t.numel())]).sort().values
    return t


def _nearest(code: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """Index into ``code`` of its nearest entry (midpoint thresholds over the sorted values, ties
    to the lower value). The fp4 table is not sorted, so the search runs on a sorted copy and
    maps back through the sort permutation."""
    c = code.to(torch.float64).cpu()
    sc, perm = torch.sort(c, stable=True)
    mids = ((sc[:-1] + sc[1:]) / 2.0).to(torch.float32).to(x.device)
    pos = torch.bucketize(x, mids, right=False)
    return perm.to(x.device)[pos]


def quantize_blocks(w: torch.Tensor, code: torch.Tensor, blocksize: int):
    """Flat fp32 stream ``[..., n]`` -> (codes uint8 ``[..., n]``, absmax fp32 ``[..., n/bs]``)."""
    w = w.float()
    n = w.shape[-1]
    if n % blocksize:
        raise ValueError(f"{n} values are not a multiple of blocksize {blocksize}")
    blk = w.reshape(*w.shape[:-1], n // blocksize, blocksize)
    absmax = blk.abs().amax(dim=-1)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    idx = _nearest(code, blk * inv.unsqueeze(-1))
    zero = int(torch.argmin(code.abs()).item())
    idx = torch.where((absmax > 0).unsqueeze(-1), idx, torch.full_like(idx, zero))
    return idx.reshape(w.shape).to(torch.uint8), absmax


def quantize_4bit(w: torch.Tensor, quant_type: str = "nf4", blocksize: int = 64):
    """Row-major ``[..., n]`` weights -> (packed uint8 ``[..., n/2]``, absmax ``[..., n/bs]``).
    Two values per byte, the first (even) value in the HIGH nibble."""
    code = code_4bit(quant_type, device=w.device)
    out_p, out_a = [], []
    flat = w.reshape(-1, w.shape[-1]) if w.dim() > 1 else w.reshape(1, -1)
    # chunk rows to bound the temporary memory of the bucketize
    step = max(1, (1 << 24) // max(1, flat.shape[-1]))
    for s in range(0, flat.shape[0], step):
        idx, am = quantize_blocks(flat[s:s + step], code, blocksize)
        out_p.append(((idx[..., 0::2] << 4) | idx[..., 1::2]).to(torch.uint8))
        out_a.append(am)
    packed = torch.cat(out_p).reshape(*w.shape[:-1], w.shape[-1] // 2)
    absmax = torch.cat(out_a).reshape(*w.shape[:-1], w.shape[-1] // blocksize)
    return packed, absmax


def double_quant(absmax: torch.Tensor, blocksize2: int = _DQ_BLOCKSIZE2, code2: torch.Tensor | None = None):
    """Compress fp32 absmax ``[..., nb]`` -> (u8 codes, fp32 absmax2 ``[..., ceil(nb/256)]``,
    fp32 offset ``[...]``). ``offset`` is the mean (accumulated in fp64); the centred values are
    quantized blockwise with the signed dynamic map."""
    if code2 is None:
        code2 = dynamic_map().to(absmax.device)
    a = absmax.float()
    offset = a.double().mean(dim=-1).float()
    c = a - offset.unsqueeze(-1)
    nb = a.shape[-1]
    nb2 = -(-nb // blocksize2)
    pad = nb2 * blocksize2 - nb
    if pad:
        c = torch.cat([c, torch.zeros(*c.shape[:-1], pad, dtype=c.dtype, device=c.device)], dim=-1)
    q, absmax2 = quantize_blocks(c, code2.to(c.device), blocksize2)
    return q[..., :nb].contiguous(), absmax2, offset


def dequant_absmax(q: torch.Tensor, absmax2: torch.Tensor, offset: torch.Tensor, code2: torch.Tensor,
                   blocksize2: int = _DQ_BLOCKSIZE2) -> torch.Tensor:
    """``fp32(fp32(code2[q] * absmax2[b // 256]) + offset)`` (CPU / reference path)."""
    nb = q.shape[-1]
    a2 = absmax2.repeat_interleave(blocksize2, dim=-1)[..., :nb]
    return code2.to(q.device)[q.long()] * a2 + offset.unsqueeze(-1)


def dequant_4bit_torch(packed: torch.Tensor, absmax: torch.Tensor, code: torch.Tensor, shape, blocksize: int,
                       dtype: torch.dtype) -> torch.Tensor:
    """Pure-torch 4-bit decode (engines/cold_engine.py:104-115): first value in the high nibble,
    ``code[idx] * absmax`` in fp32, one cast to ``dtype``."""
    pk = packed.reshape(-1)
    idx = torch.empty(pk.numel() * 2, dtype=torch.long, device=pk.device)
    idx[0::2] = (pk >> 4).long()
    idx[1::2] = (pk & 0xF).long()
    vals = code.to(pk.device).index_select(0, idx)
    return (vals.reshape(-1, blocksize) * absmax.reshape(-1, 1).float()).reshape(shape).to(dtype)


def quantize_mxfp4(w: torch.Tensor, group: int = 32):
    """OCP MX e2m1 quantization of ``[..., K]`` rows: per 32 values an e8m0 exponent
    ``floor(log2(amax)) - 2 + 127`` (clamped to [0, 254]) and each value rounded to the nearest
    e2m1 magnitude (ties to the even code, saturating at 6). Low nibble = first value.
    Returns ``(blocks [..., K/2] uint8, scales [..., K/32] uint8)``."""
    w = w.float()
    K = w.shape[-1]
    if K % group:
        raise ValueError(f"K={K} is not a multiple of {group}")
    g = w.reshape(*w.shape[:-1], K // group, group)
    amax = g.abs().amax(dim=-1)
    safe = torch.where(amax > 0, amax, torch.ones_like(amax))
    X = torch.where(amax > 0, torch.floor(torch.log2(safe)) - 2, torch.full_like(amax, -127.0))
    e = torch.clamp(X + 127, 0, 254)
    scaled = g.double() / torch.pow(2.0, (e - 127).double()).unsqueeze(-1)
    mag = scaled.abs()
    grid = torch.tensor(FP4_VALUES[:8], dtype=torch.float64, device=w.device)
    mids = (grid[:-1] + grid[1:]) / 2.0
    # nearest magnitude (bucketize sends an exact midpoint to the lower code); a midpoint
    # goes to the even code instead, the e2m1 round-to-nearest-even rule
    best = torch.bucketize(mag, mids, right=False)
    tie = (best < 7) & (mag == mids[best.clamp(max=6)])
    best = torch.where(tie & (best % 2 == 1), best + 1, best)
    sign = ((scaled < 0) & (best > 0)).to(torch.int64) * 8
    code = (best + sign).to(torch.uint8).reshape(w.shape)
    blocks = ((code[..., 1::2] << 4) | code[..., 0::2]).to(torch.uint8)
    return blocks, e.to(torch.uint8)


def dequant_mxfp4_torch(blocks: torch.Tensor, scales: torch.Tensor, rows: int, K: int,
                        dtype: torch.dtype) -> torch.Tensor:
    """Row-major MXFP4 decode: ``[rows, K/2]`` bytes + ``[rows, K/32]`` e8m0 -> ``[rows, K]``
    (low nibble first, ``FP4 * 2**(s-127)``, exact in fp32 then one cast)."""
    blk = blocks.reshape(rows, K // 2)
    lut = torch.tensor(FP4_VALUES, dtype=torch.float32, device=blk.device)
    out = torch.empty(rows, K, dtype=torch.float32, device=blk.device)
    out[:, 0::2] = lut[(blk & 0x0F).long()]
    out[:, 1::2] = lut[(blk >> 4).long()]
    exp = scales.reshape(rows, K // 32).to(torch.int32) - 127
    out = torch.ldexp(out.reshape(rows, K // 32, 32), exp.unsqueeze(-1).float())
    return out.reshape(rows, K).to(dtype)
