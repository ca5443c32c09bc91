"""GPU parity of each kernel, called through the C ABI, against the CPU oracle.

Bars: bit-exact for dequant, routing and the combine; rel-Frobenius <= 1e-2 and max-abs <= 2e-2
(on outputs normalised by the oracle's RMS) for the GEMMs, whose fp32 accumulation order
differs from the oracle's.
"""
import numpy as np
import pytest
import torch

from experts4bit_qlora_amd import _native as N
from experts4bit_qlora_amd import ops, quant as Q
from oracle import c_oracle, codes, moe, numerics, quant as oq, routing as orouting

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy().view(np.uint32)


def _nf4_stack(E, n, k, seed, dq=False):
    g = torch.Generator(device="cpu").manual_seed(seed)
    w = torch.randn(E, n * k, generator=g) * 0.02
    packed, absmax = Q.quantize_4bit(w)
    code = Q.code_4bit("nf4")
    if dq:
        q, a2, off = Q.double_quant(absmax)
        code2 = Q.dynamic_map()
        qw = ops.nf4_dq_qweight(packed.to(DEV), q.to(DEV), a2.to(DEV), off.to(DEV), code.to(DEV), code2.to(DEV), n, k,
                                num_experts=E)
        absmax_f = oq.dequant_absmax_dq(q.numpy(), a2.numpy(), off.numpy(), code2.numpy())
        return qw, packed.numpy(), absmax_f
    qw = ops.nf4_qweight(packed.to(DEV), absmax.to(DEV), code.to(DEV), n, k, num_experts=E)
    return qw, packed.numpy(), absmax.numpy()


# ------------------------------------------------------------------------------- dequant


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dq", [False, True])
def test_dequant_nf4_bit_exact(dt, dq):
    _announce(f"dequant nf4 dq={dq} {dt}")
    E, n, k = 3, 96, 256
    qw, packed, absmax = _nf4_stack(E, n, k, seed=1, dq=dq)
    got = ops.dequant(qw, 0, E, dtype=dt)
    want = c_oracle.dequant_4bit(packed.reshape(-1), absmax.reshape(-1), codes.NF4_CODE).reshape(E, n, k)
    if dt == torch.float32:
        assert np.array_equal(_bits(got), want.view(np.uint32))
    elif dt == torch.bfloat16:
        assert np.array_equal(_bits(got), numerics.f32_to_bf16_bits(want))
    else:
        gb, wb = _bits(got), want.astype(np.float16).view(np.uint16)
        bad = np.argwhere(gb != wb)
        detail = [(tuple(i), float(want[tuple(i)]), hex(int(gb[tuple(i)])), hex(int(wb[tuple(i)]))) for i in bad[:8]]
        assert bad.size == 0, f"{len(bad)} mismatches: {detail}"


def test_dequant_nf4_expert_range_and_full_size_expert():
    _announce("dequant nf4 OLMoE gate_up expert slice")
    E, n, k = 4, 2048, 2048
    qw, packed, absmax = _nf4_stack(E, n, k, seed=2)
    got = ops.dequant(qw, 2, 1, dtype=torch.bfloat16)[0]
    want = c_oracle.dequant_4bit(packed[2], absmax[2], codes.NF4_CODE, out="bf16").reshape(n, k)
    assert np.array_equal(_bits(got), want)


def test_dequant_mxfp4_bit_exact():
    _announce("dequant mxfp4")
    E, n, k = 2, 64, 2880
    g = torch.Generator().manual_seed(3)
    blocks = torch.randint(0, 256, (E, n, k // 2), generator=g, dtype=torch.uint8)
    scales = torch.randint(100, 150, (E, n, k // 32), generator=g, dtype=torch.uint8)
    qw = ops.mxfp4_qweight(blocks.to(DEV), scales.to(DEV), n, k, num_experts=E)
    for dt, tag in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        got = ops.dequant(qw, 0, E, dtype=dt)
        want = oq.dequant_mxfp4_rows(blocks.numpy().reshape(E, n, k // 32, 16), scales.numpy(), dtype=tag)
        if tag == "fp32":
            assert np.array_equal(_bits(got), want.reshape(E, n, k).view(np.uint32))
        else:
            assert np.array_equal(_bits(got), numerics.f32_to_bf16_bits(want.reshape(E, n, k)))


# ------------------------------------------------------------------------------- routing


def _check_route(idx: np.ndarray, E: int):
    T, k = idx.shape
    rb = ops.route(torch.from_numpy(idx).to(DEV), E)
    torch.cuda.synchronize()
    M = T * k
    valid = (idx >= 0) & (idx < E)
    ref = orouting.route(np.where(valid, idx, 0), E) if valid.all() else None
    meta = rb.meta.cpu().numpy()
    if ref is not None:
        assert np.array_equal(rb.sorted_flat[:M].cpu().numpy(), ref["order"])
        assert np.array_equal(rb.inv[:M].cpu().numpy(), ref["inv"])
        assert np.array_equal(rb.offsets.cpu().numpy(), ref["offsets"])
        assert meta[1] == ref["active"].size and meta[2] == 0
        assert np.array_equal(rb.active[:meta[1]].cpu().numpy(), ref["active"])
        tiles = orouting.m_tiles(ref["counts"], rb.tile_m)
        assert meta[0] == len(tiles)
        assert rb.tiles[:2 * meta[0]].cpu().numpy().reshape(-1, 2).tolist() == [list(t) for t in tiles]
    return rb, meta


@pytest.mark.parametrize("T,k,E", [(1, 8, 64), (8, 8, 64), (64, 8, 64), (1, 8, 128), (32, 8, 128), (256, 8, 128),
                                   (1, 4, 32), (2048, 4, 32), (4096, 8, 128), (37, 3, 1024), (5, 2, 4)])
def test_route_bit_exact(T, k, E):
    _announce(f"route T={T} k={k} E={E}")
    rng = np.random.default_rng(T * 1000 + E)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    _check_route(idx, E)


def test_route_zipf_prefill_and_duplicates():
    _announce("route zipf 4096x8 over 128 + duplicate ids")
    rng = np.random.default_rng(0)
    p = 1.0 / np.arange(1, 129) ** 1.1
    idx = np.stack([rng.choice(128, 8, replace=False, p=p / p.sum()) for _ in range(4096)]).astype(np.int64)
    _check_route(idx, 128)
    dup = rng.integers(0, 3, (300, 4)).astype(np.int64)  # duplicates within tokens, empty experts
    _check_route(dup, 8)


def test_route_drops_out_of_range_ids():
    _announce("route invalid ids")
    idx = np.array([[0, 5], [9, 1], [-1, 2]], dtype=np.int64)  # E = 6
    rb, meta = _check_route(idx, 6)
    assert meta[2] == 2
    inv = rb.inv[:6].cpu().numpy()
    assert inv[2] == -1 and inv[4] == -1
    ref = orouting.route(np.array([[0, 5], [1, 2]]), 6)  # the valid ids keep their relative order
    assert rb.offsets.cpu().numpy()[-1] == 4
    order = rb.sorted_flat[:4].cpu().numpy()
    assert order.tolist() == [0, 3, 5, 1]
    assert ref["counts"].sum() == 4


@pytest.mark.parametrize("M,E", [(4096, 64), (4097, 64), (4353, 1024), (40000, 256), (140000, 128),
                                 (262144, 64)])
def test_chunked_route_boundaries_and_dropped_ids(M, E):
    """Around the one-workgroup limit (4096 rows) and on the chunked route: ragged last chunk,
    many experts, ~1% invalid ids spread through the chunks. Above 512 chunks (131,072 ids) the
    per-expert column scan carries its running sum from one pass of 512 chunks to the next
    (140,000 and 262,144 ids); the tile list and its count are checked against the offsets."""
    _announce(f"chunked route M={M} E={E}")
    rng = np.random.default_rng(M + E)
    flat = rng.integers(0, E, M).astype(np.int64)
    bad = rng.random(M) < 0.01
    flat[bad] = np.where(rng.random(bad.sum()) < 0.5, -1, E + 3)
    idx = flat.reshape(M, 1)
    rb = ops.route(torch.from_numpy(idx).to(DEV), E)
    meta = rb.meta.cpu().numpy()
    assert meta[2] == bad.sum()
    valid = np.flatnonzero(~bad)
    order = valid[np.argsort(flat[valid], kind="stable")]
    n = len(order)
    assert rb.sorted_flat[:n].cpu().numpy().tolist() == order.tolist()
    inv = rb.inv[:M].cpu().numpy()
    assert (inv[bad] == -1).all()
    assert (inv[order] == np.arange(n)).all()
    counts = np.bincount(flat[valid], minlength=E)
    assert rb.offsets.cpu().numpy().tolist() == np.concatenate([[0], np.cumsum(counts)]).tolist()
    assert meta[1] == (counts > 0).sum()
    tiles = orouting.m_tiles(counts, rb.tile_m)
    assert meta[0] == len(tiles)
    assert rb.tiles[:2 * meta[0]].cpu().numpy().reshape(-1, 2).tolist() == [list(t) for t in tiles]


# --------------------------------------------------------------------------------- GEMMs


def _dense_from_oracle(qw) -> np.ndarray:
    """``[E, n, k]`` fp32 weights of a descriptor, decoded from its bytes by the oracle's C
    restatement -- not by the dequant kernel, whose parity is tested on its own."""
    from oracle import c_oracle

    E, n, k = qw.num_experts, qw.n, qw.k
    packed = qw.packed.cpu().numpy().reshape(E, -1)
    absmax = qw.absmax.cpu().numpy().reshape(E, -1)
    out = np.empty((E, n, k), np.float32)
    for e in range(E):
        if qw.fmt == N.FMT_MXFP4:
            out[e] = c_oracle.dequant_mxfp4(packed[e], absmax[e], n, k)
            continue
        am = absmax[e]
        if qw.fmt == N.FMT_NF4_DQ:
            am = c_oracle.dequant_absmax_dq(am, qw.absmax2.cpu().numpy().reshape(E, -1)[e],
                                            float(qw.offset.cpu().numpy().reshape(E)[e]), qw.code2.cpu().numpy())
        out[e] = c_oracle.dequant_4bit(packed[e], am, qw.code.cpu().numpy()).reshape(n, k)
    return out


def _weights_for(path, W):
    """The weights each kernel family multiplies: fp32 decode (GEMV) or the reference's exact
    bf16 dequantized weight (MFMA operands)."""
    return numerics.round_bf16(W) if path == N.PATH_MFMA else W


def _gemm_oracle(a_rows, W, rows_expert, bias=None):
    """fp64 per-row GEMM against the dequantized fp32 weights."""
    out = np.empty((a_rows.shape[0], W.shape[1]), np.float64)
    for r in range(a_rows.shape[0]):
        out[r] = W[rows_expert[r]].astype(np.float64) @ a_rows[r].astype(np.float64)
        if bias is not None:
            out[r] += bias[rows_expert[r]]
    return out


def _errs(got, want):
    fro, maxabs, _ = moe.rel_errors(got, want)
    return fro, maxabs


def _errs_rounded_bf16(got, exact):
    """Errors of a bf16 result against the exact (unrounded) values, net of the result's own
    rounding: each element may sit half a bf16 ulp from the exact value before any error counts.
    (Against round_bf16(exact), an fp32 sum a hair across a rounding boundary would cost a whole
    ulp of the element -- 2.3e-2 of the RMS for an element 3x the RMS.)"""
    g = np.asarray(got, np.float64)
    w = np.asarray(exact, np.float64)
    half_ulp = np.ldexp(0.5, np.frexp(np.abs(w))[1] - 8)
    excess = np.maximum(np.abs(g - w) - half_ulp, 0.0)
    rms = max(np.sqrt(np.mean(w * w)), 1e-30)
    return float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30)), float(excess.max() / rms)


@pytest.mark.parametrize("path", [N.PATH_GEMV, N.PATH_MFMA])
@pytest.mark.parametrize("fmt", ["nf4", "nf4_dq", "mxfp4"])
@pytest.mark.parametrize("T", [1, 3, 40])
def test_grouped_gemm_plain(path, fmt, T):
    _announce(f"grouped gemm plain path={path} fmt={fmt} T={T}")
    E, n, k, top = 8, 192, 320, 2
    if fmt == "mxfp4":
        g = torch.Generator().manual_seed(5)
        w = torch.randn(E, n, k, generator=g) * 0.02
        b, s = Q.quantize_mxfp4(w)
        qw = ops.mxfp4_qweight(b.reshape(E, -1).to(DEV), s.reshape(E, -1).to(DEV), n, k, num_experts=E)
    else:
        qw, _, _ = _nf4_stack(E, n, k, seed=6, dq=(fmt == "nf4_dq"))
    W = _dense_from_oracle(qw)
    rng = np.random.default_rng(T)
    idx = np.stack([rng.permutation(E)[:top] for _ in range(T)]).astype(np.int64)
    x = torch.randn(T, k, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    rb = ops.route(torch.from_numpy(idx).to(DEV), E)
    out = ops.grouped_gemm(x.to(DEV), qw, rb, T, T * top, N.EPI_NONE, gather_k=top, path=path)
    ref = orouting.route(idx, E)
    want = _gemm_oracle(x.float().numpy()[ref["token_rows"]], _weights_for(path, W), idx.reshape(-1)[ref["order"]])
    fro, maxabs = _errs(out.float().cpu().numpy(), want)
    assert fro <= 1e-2 and maxabs <= 2e-2, (fro, maxabs)
    # the fp32 output of the same GEMM is the unrounded sum
    out32 = ops.grouped_gemm(x.to(DEV), qw, rb, T, T * top, N.EPI_NONE, gather_k=top, path=path,
                             out_dtype=torch.float32)
    fro32, _ = _errs(out32.cpu().numpy(), want)
    assert out32.dtype == torch.float32 and fro32 < 1e-5, fro32


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", ["nf4", "nf4_dq", "mxfp4"])
@pytest.mark.parametrize("k", [64, 192, 320, 512])
def test_grouped_gemm_wide_tiles(fmt, k, dt):
    """256-row tiles (gemm_wide_kernel, four waves of 128 x 128, 32 x 32 MFMAs, the staging of a
    step spread over the previous step's MFMAs): 1, 3, 5 and 8 steps of 64 (the odd counts take
    the loop's single-step tail), partial tiles (experts of 37 to 300 rows, two tiles for the
    largest), bf16 rows and fp32 rows, against the fp64 oracle over the oracle's weights."""
    _announce(f"grouped gemm wide tiles fmt={fmt} k={k} dt={dt}")
    E, n, top = 5, 320, 2
    sizes = [300, 37, 150, 0, 113]
    if fmt == "mxfp4":
        g = torch.Generator().manual_seed(70 + k)
        w = torch.randn(E, n, k, generator=g) * 0.02
        b, s = Q.quantize_mxfp4(w)
        qw = ops.mxfp4_qweight(b.reshape(E, -1).to(DEV), s.reshape(E, -1).to(DEV), n, k, num_experts=E)
    else:
        qw, _, _ = _nf4_stack(E, n, k, seed=71 + k, dq=(fmt == "nf4_dq"))
    W = _dense_from_oracle(qw)
    # token t's two slots: experts chosen so that expert e gets sizes[e] rows in all
    slots = np.concatenate([np.full(c, e) for e, c in enumerate(sizes)])
    rng = np.random.default_rng(k)
    rng.shuffle(slots)
    idx = slots.reshape(-1, top).astype(np.int64)
    T = idx.shape[0]
    x = torch.randn(T, k, generator=torch.Generator().manual_seed(72 + k)).to(dt)
    rb = ops.route(torch.from_numpy(idx).to(DEV), E, tile_m=256)
    ref = orouting.route(idx, E)
    Wm = numerics.round_bf16(W) if dt == torch.bfloat16 else numerics.round_fp16(W)
    want = _gemm_oracle(x.float().numpy()[ref["token_rows"]], Wm, idx.reshape(-1)[ref["order"]])
    # 16-bit rows: errors net of the row's own rounding (half an ulp of each element)
    errs = _errs_rounded_bf16 if dt == torch.bfloat16 else _errs
    out = ops.grouped_gemm(x.to(DEV), qw, rb, T, T * top, N.EPI_NONE, gather_k=top, path=N.PATH_MFMA)
    fro, maxabs = errs(out.float().cpu().numpy(), want)
    assert fro <= 1e-2 and maxabs <= 2e-2, (fro, maxabs)
    out32 = ops.grouped_gemm(x.to(DEV), qw, rb, T, T * top, N.EPI_NONE, gather_k=top, path=N.PATH_MFMA,
                             out_dtype=torch.float32)
    fro32, _ = _errs(out32.cpu().numpy(), want)
    assert fro32 < 1e-5, fro32
    # the 128-row tiles of the same rows give the same fp32 rows up to summation order
    out128 = ops.grouped_gemm(x.to(DEV), qw, ops.route(torch.from_numpy(idx).to(DEV), E, tile_m=128), T, T * top,
                              N.EPI_NONE, gather_k=top, path=N.PATH_MFMA, out_dtype=torch.float32)
    assert torch.allclose(out32, out128, rtol=1e-5, atol=1e-6)
    # gated epilogue: silu(g) * u on the fp32 sums, one rounding
    gated = ops.grouped_gemm(x.to(DEV), qw, rb, T, T * top, N.EPI_SWIGLU, gather_k=top, path=N.PATH_MFMA)
    half = n // 2
    h_want = moe._glu_exact(want, "swiglu", half)
    fro_g, maxabs_g = errs(gated.float().cpu().numpy(), h_want)
    assert fro_g <= 1e-2 and maxabs_g <= 2e-2, (fro_g, maxabs_g)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_mxfp4_mfma_weights_at_every_scale(dt):
    """One-hot activations turn the MFMA GEMM's output into the weights it multiplies: row i of
    the output is column i of W (one product by 1.0, the rest zeros, fp32 accumulation). The
    stack cycles through every e8m0 scale whose largest product stays finite in the activation
    type (bf16: 0..252, fp16: 0..140; an inf weight would turn the zero products into NaN), so
    the in-register scaled e2m1 conversion is pinned bit for bit to dt(ldexp(code, e - 127)) of
    the oracle, subnormal results included (zeros compared without their sign)."""
    _announce(f"mxfp4 mfma weights at every scale dt={dt}")
    n, k = 128, 512
    emax = 252 if dt == torch.bfloat16 else 140
    rng = np.random.default_rng(50)
    blocks = rng.integers(0, 256, size=(n, k // 32, 16), dtype=np.uint8)
    scales = (np.arange(n * (k // 32)) % (emax + 1)).astype(np.uint8).reshape(n, k // 32)
    qw = ops.mxfp4_qweight(torch.from_numpy(blocks).reshape(1, -1).to(DEV),
                           torch.from_numpy(scales).reshape(1, -1).to(DEV), n, k, num_experts=1)
    want = oq.dequant_mxfp4_rows(blocks, scales, "bf16" if dt == torch.bfloat16 else "fp16").T
    x = torch.eye(k, dtype=dt)
    rb = ops.route(torch.zeros(k, 1, dtype=torch.int64, device=DEV), 1)
    out = ops.grouped_gemm(x.to(DEV), qw, rb, k, k, N.EPI_NONE, gather_k=1, path=N.PATH_MFMA)
    got = _bits(out)
    exp = (numerics.f32_to_bf16_bits(want) if dt == torch.bfloat16
           else np.ascontiguousarray(want.astype(np.float16)).view(np.uint16)).copy()
    # a -0 weight (e2m1 code 8) comes out +0: the fp32 sum adds +0 products to it
    exp[exp == 0x8000] = 0
    assert np.array_equal(got, exp), int((got != exp).sum())


@pytest.mark.parametrize("path", [N.PATH_GEMV, N.PATH_MFMA])
@pytest.mark.parametrize("epi", ["swiglu", "act", "clamp", "gptoss"])
def test_grouped_gemm_fused_epilogues(path, epi):
    _announce(f"grouped gemm epilogue path={path} epi={epi}")
    E, H, I, top, T = 6, 256, 128, 2, 9
    gated = epi != "act"
    n = 2 * I if gated else I
    qw, _, _ = _nf4_stack(E, n, H, seed=7)
    g = torch.Generator().manual_seed(8)
    bias = None
    if epi == "gptoss":
        bias = (torch.randn(E, n, generator=g) * 0.5).to(torch.bfloat16)
        qw.bias = bias.to(DEV)
    W = _dense_from_oracle(qw)
    rng = np.random.default_rng(9)
    idx = np.stack([rng.permutation(E)[:top] for _ in range(T)]).astype(np.int64)
    x = (torch.randn(T, H, generator=g) * 3).to(torch.bfloat16)
    rb = ops.route(torch.from_numpy(idx).to(DEV), E)
    code = {"swiglu": N.EPI_SWIGLU, "act": N.EPI_ACT, "clamp": N.EPI_CLAMP_SWIGLU, "gptoss": N.EPI_GPTOSS}[epi]
    out = ops.grouped_gemm(x.to(DEV), qw, rb, T, T * top, code, gather_k=top, alpha=1.702, limit=1.5, path=path)
    ref = orouting.route(idx, E)
    e_rows = idx.reshape(-1)[ref["order"]]
    b = None if bias is None else bias.float().numpy().astype(np.float64)
    proj = _gemm_oracle(x.float().numpy()[ref["token_rows"]], _weights_for(path, W), e_rows, bias=b)
    # the fused epilogue runs in fp32 on the unrounded projection; h is rounded once
    spec = {"swiglu": "swiglu", "act": "act", "clamp": ("clamp_swiglu", 1.5), "gptoss": ("gptoss", 1.702, 1.5)}[epi]
    want = numerics.round_bf16(moe._glu_exact(proj, spec, I).astype(np.float32))
    fro, maxabs = _errs(out.float().cpu().numpy(), want)
    assert fro <= 1e-2 and maxabs <= 2e-2, (fro, maxabs)


def test_grouped_gemm_fp16_activations():
    _announce("grouped gemm fp16")
    E, n, k, top, T = 4, 128, 256, 2, 20
    qw, _, _ = _nf4_stack(E, n, k, seed=10)
    W = _dense_from_oracle(qw)
    rng = np.random.default_rng(11)
    idx = np.stack([rng.permutation(E)[:top] for _ in range(T)]).astype(np.int64)
    x = torch.randn(T, k, generator=torch.Generator().manual_seed(12)).to(torch.float16)
    rb = ops.route(torch.from_numpy(idx).to(DEV), E)
    ref = orouting.route(idx, E)
    want = _gemm_oracle(x.float().numpy()[ref["token_rows"]], W, idx.reshape(-1)[ref["order"]])
    for path in (N.PATH_GEMV, N.PATH_MFMA):
        out = ops.grouped_gemm(x.to(DEV), qw, rb, T, T * top, N.EPI_NONE, gather_k=top, path=path)
        assert out.dtype == torch.float16
        want_p = want if path == N.PATH_GEMV else _gemm_oracle(
            x.float().numpy()[ref["token_rows"]], numerics.round_fp16(W), idx.reshape(-1)[ref["order"]])
        fro, maxabs = _errs(out.float().cpu().numpy(), want_p)
        assert fro <= 1e-2 and maxabs <= 2e-2, (path, fro, maxabs)


def test_gemm_4bit_grouped_api_shape():
    _announce("gemm_4bit_grouped API")
    E, n, k = 5, 64, 128
    qw, packed, absmax = _nf4_stack(E, n, k, seed=13)
    W = _dense_from_oracle(qw)
    sizes, ids = [3, 1, 7], [0, 2, 4]
    a = torch.randn(sum(sizes), k, generator=torch.Generator().manual_seed(14)).to(torch.bfloat16)
    out = ops.gemm_4bit_grouped(a.to(DEV), qw.packed.view(E, n, k // 2), qw.absmax.view(E, n, k // 64), sizes, ids)
    rows_e = np.repeat(ids, sizes)
    want = _gemm_oracle(a.float().numpy(), W, rows_e)
    fro, maxabs = _errs(out.float().cpu().numpy(), want)
    assert out.shape == (11, n) and fro <= 1e-2 and maxabs <= 2e-2


# ------------------------------------------------------------------------------- combine


@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H", [256, 512, 2048, 2880, 100])
def test_combine_bit_exact(wdt, H):
    """k-slot combine, bit for bit against fp32 slot-order sums: multiples of 8 (256, 512, 2048,
    2880) take the eight-value vector path, 100 the scalar path."""
    _announce(f"combine H={H} w={wdt}")
    T, k, E = 33, 4, 16
    rng = np.random.default_rng(H)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    rb = ops.route(torch.from_numpy(idx).to(DEV), E)
    down = torch.randn(T * k, H, generator=torch.Generator().manual_seed(15)).to(torch.bfloat16)
    w = torch.rand(T, k, generator=torch.Generator().manual_seed(16)).to(wdt)
    out = ops.combine(down.to(DEV), rb, w.to(DEV), T, k, torch.float32)
    ref = orouting.route(idx, E)
    d = down.float().numpy()
    wf = w.float().numpy()
    acc = np.zeros((T, H), np.float32)
    for s in range(k):
        rows = ref["inv"].reshape(T, k)[:, s]
        acc = (acc + (d[rows] * wf[:, s:s + 1]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(_bits(out), acc.view(np.uint32))
    out16 = ops.combine(down.to(DEV), rb, w.to(DEV), T, k, torch.bfloat16)
    assert np.array_equal(_bits(out16), numerics.f32_to_bf16_bits(acc))


# ------------------------------------------------------------------------ LoRA delta


_LORA_CASES = [
    # (x dtype, adapter dtype, gather, E, tokens, rank, out features): the small cases run the
    # 1-row tiles; 800 rows run 8-row output tiles; 3072 rows (200 experts: about 15 rows each, so
    # most tiles hold several expert segments) run 8-row tiles in both kernels and a partial rank
    # group; 9000 rows run 32-row output tiles at the largest rank.
    (torch.bfloat16, torch.bfloat16, True, 12, 37, 16, 200),
    (torch.bfloat16, torch.float32, True, 12, 37, 16, 200),
    (torch.bfloat16, torch.bfloat16, False, 12, 37, 16, 200),
    (torch.bfloat16, torch.float32, False, 12, 37, 16, 200),
    (torch.float16, torch.bfloat16, True, 12, 37, 16, 200),
    (torch.float16, torch.float32, True, 12, 37, 16, 200),
    (torch.float16, torch.float16, False, 12, 37, 16, 200),
    (torch.float16, torch.float32, False, 12, 37, 16, 200),
    (torch.bfloat16, torch.float32, True, 12, 400, 5, 300),
    (torch.bfloat16, torch.bfloat16, True, 200, 1536, 40, 300),
    (torch.float16, torch.float32, False, 200, 1536, 40, 260),
    (torch.bfloat16, torch.float32, True, 64, 1200, 32, 300),
    (torch.bfloat16, torch.float32, True, 64, 4500, 64, 520),
    # ranks 17-31 inside the 32-rank register slice (the j < r masking), 1-row and 8-row tiles
    (torch.bfloat16, torch.float32, True, 12, 37, 20, 200),
    (torch.bfloat16, torch.bfloat16, True, 64, 1200, 24, 300),
    (torch.float16, torch.float16, False, 64, 1200, 20, 260),
]


@pytest.mark.parametrize("xdt,adt,gather,E,T,r,Nout", _LORA_CASES)
def test_lora_delta_matches_per_group_reference(xdt, adt, gather, E, T, r, Nout):
    """e4b_lora_delta adds scaling * (x_m @ A[e].T) @ B[e].T, rounded to the compute dtype, to
    every expert-sorted row of an fp32 projection in one pass -- the per-group `_lora` of
    lora.py:251-256 as fast.py:229-233 applies it, here checked per group against an fp64
    product. The bar is the delta's own rounding (2^-7 of it) plus the fp32 summation bound
    (2^-14 of the same product over absolute values: K + r = 320 terms at 2^-24 each, with room).
    Empty experts and an out-of-range id (a dropped row left untouched) are included."""
    _announce(f"lora delta xdt={xdt} adt={adt} gather={gather} E={E} T={T} r={r} Nout={Nout}")
    top, K, scaling = 2, 256, 0.75
    g = torch.Generator().manual_seed(60 + T + r)
    idx = torch.stack([torch.randperm(E - 3, generator=g)[:top] for _ in range(T)]).to(torch.int64)
    idx[5, 1] = E + 4  # dropped
    x = (torch.randn(T if gather else T * top, K, generator=g)).to(xdt)
    A = (torch.randn(E, r, K, generator=g) * 0.05).to(adt)
    B = (torch.randn(E, Nout, r, generator=g) * 0.05).to(adt)
    M = T * top
    rb = ops.route(idx.to(DEV), E)
    base = torch.randn(M, Nout, generator=g)
    out = base.clone().to(DEV)
    ops.lora_delta(x.to(DEV), rb, M, E, A.to(DEV), B.to(DEV), scaling, out, gather_k=top if gather else 0)
    flat = idx.numpy().reshape(-1)
    valid = np.flatnonzero((flat >= 0) & (flat < E))
    order = valid[np.argsort(flat[valid], kind="stable")]  # the routing's stable sort, dropped ids out
    offs = np.concatenate([[0], np.cumsum(np.bincount(flat[valid], minlength=E))])
    want = base.double().clone()
    bound = torch.zeros(M, Nout, dtype=torch.float64)
    for e in range(E):
        s, t = int(offs[e]), int(offs[e + 1])
        if s == t:
            continue
        rows = torch.from_numpy(order[s:t]) // top if gather else torch.arange(s, t)
        xm = x[rows].double()
        Ae, Be = A[e].double(), B[e].double()
        want[s:t] += scaling * (xm @ Ae.T) @ Be.T
        bound[s:t] = scaling * (xm.abs() @ Ae.abs().T) @ Be.abs().T
    got = out.cpu().double()
    n_valid = int(offs[E])
    assert torch.equal(got[n_valid:], base.double()[n_valid:])  # rows past the routed ones untouched
    err = (got[:n_valid] - want[:n_valid]).abs()
    tol = (want[:n_valid] - base.double()[:n_valid]).abs() * 2.0 ** -7 + bound[:n_valid] * 2.0 ** -14 + 1e-9
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("epi,adt,T,r", [("swiglu", torch.float32, 37, 16), ("swiglu", torch.bfloat16, 1536, 40),
                                         ("clamp_swiglu", torch.float32, 400, 8), ("act", torch.bfloat16, 37, 16),
                                         ("swiglu", torch.float32, 4500, 16), ("swiglu", torch.float32, 1200, 32),
                                         ("swiglu", torch.float32, 37, 20), ("swiglu", torch.bfloat16, 1200, 24)])
def test_lora_delta_epilogue_matches_delta_then_epilogue(epi, adt, T, r):
    """e4b_lora_delta_epilogue == e4b_lora_delta on the fp32 rows followed by the activation in
    fp32 (the base's `_epilogue`, lora.py:102-128, on proj.chunk(2, -1)) and one rounding to the
    compute dtype; they differ only by the sigmoid's few fp32 ulp, so within 2^-7 relative."""
    _announce(f"lora delta epilogue epi={epi} adt={adt} T={T} r={r}")
    E, top, K, n_out, scaling, limit = 40, 2, 256, 384, 0.5, 7.0
    code = {"swiglu": N.EPI_SWIGLU, "clamp_swiglu": N.EPI_CLAMP_SWIGLU, "act": N.EPI_ACT}[epi]
    g = torch.Generator().manual_seed(70 + T + r)
    idx = torch.stack([torch.randperm(E - 2, generator=g)[:top] for _ in range(T)]).to(torch.int64)
    idx[3, 0] = -1  # dropped
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).to(DEV)
    A = (torch.randn(E, r, K, generator=g) * 0.05).to(adt).to(DEV)
    B = (torch.randn(E, n_out, r, generator=g) * 0.05).to(adt).to(DEV)
    M = T * top
    rb = ops.route(idx.to(DEV), E)
    proj = (torch.randn(M, n_out, generator=g) * 4.0).to(DEV)
    proj0 = proj.clone()
    # the delta rounded to the compute dtype (the reference's `_lora` cast) or kept in fp32
    ddt = torch.float32 if r in (8, 20, 32) else None
    h = ops.lora_delta_epilogue(x, rb, M, E, A, B, scaling, proj, code, limit=limit, gather_k=top, delta_dtype=ddt)
    ref = proj.clone()
    ops.lora_delta(x, rb, M, E, A, B, scaling, ref, gather_k=top, delta_dtype=ddt)
    if code == N.EPI_ACT:
        want = torch.nn.functional.silu(ref)
    else:
        gte, up = ref.chunk(2, dim=-1)
        if code == N.EPI_CLAMP_SWIGLU:
            gte, up = gte.clamp(max=limit), up.clamp(-limit, limit)
        want = torch.nn.functional.silu(gte) * up
    n_valid = int(rb.offsets[E].item())
    got, want = h[:n_valid].float().cpu(), want[:n_valid].to(torch.bfloat16).float().cpu()
    assert got.shape == want.shape
    err = (got - want).abs()
    assert bool((err <= want.abs() * 2.0 ** -7 + 1e-6).all()), float(err.max())
    assert torch.equal(proj, proj0)  # the fp32 rows are only read


# ------------------------------------------------------------------- decode halves


def _stack(fmt, E, n, k, seed):
    """(qweight, the dense weights the decode kernels multiply, fp64 [E, n, k])."""
    if fmt == "mxfp4":
        g = torch.Generator().manual_seed(seed)
        w = torch.randn(E, n, k, generator=g) * 0.05
        b, s = Q.quantize_mxfp4(w)
        qw = ops.mxfp4_qweight(b.reshape(E, -1).to(DEV), s.reshape(E, -1).to(DEV), n, k, num_experts=E)
        return qw, _dense_from_oracle(qw).astype(np.float64)
    qw, _, _ = _nf4_stack(E, n, k, seed=seed, dq=(fmt == "nf4_dq"))
    return qw, _dense_from_oracle(qw).astype(np.float64)  # the exact fp32 code * absmax


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", ["nf4", "nf4_dq", "mxfp4"])
@pytest.mark.parametrize("T", [1, 5, 32])
def test_decode_halves_match_oracle(fmt, T, dt):
    """e4b_decode_gate_up (wave-local routing + gate_up + epilogue, h in flat order) and
    e4b_decode_down_combine (down + k-slot combine) against the fp64 oracle per flat row, in
    both activation types. T=32 with top-2 over 8 experts fills the 64-row limit with ~8 rows
    per expert; T=5 runs the per-wave item kernel, T=1 and T=32 the per-expert one."""
    _announce(f"decode halves fmt={fmt} T={T} dt={dt}")
    E, H, I, top = 8, 768, 320, 2
    w1, W1 = _stack(fmt, E, 2 * I, H, seed=20)
    w2, W2 = _stack(fmt, E, H, I, seed=21)
    epi, spec = N.EPI_SWIGLU, "swiglu"
    if fmt == "mxfp4":
        g = torch.Generator().manual_seed(22)
        w1.bias = (torch.randn(E, 2 * I, generator=g) * 0.1).to(dt).to(DEV)  # biases in the activation type
        w2.bias = (torch.randn(E, H, generator=g) * 0.1).to(dt).to(DEV)
        epi, spec = N.EPI_GPTOSS, ("gptoss", 1.702, 7.0)
    rng = np.random.default_rng(23 + T)
    idx = np.stack([rng.permutation(E)[:top] for _ in range(T)]).astype(np.int64)
    x = (torch.randn(T, H, generator=torch.Generator().manual_seed(24)) * 2).to(dt)
    wts = torch.rand(T, top, generator=torch.Generator().manual_seed(25)).to(torch.bfloat16)
    h = ops.decode_gate_up(x.to(DEV), torch.from_numpy(idx).to(DEV), w1, epi)
    flat_e = idx.reshape(-1)
    b1 = None if w1.bias is None else w1.bias.float().cpu().numpy().astype(np.float64)
    proj = _gemm_oracle(x.float().numpy()[np.arange(T * top) // top], W1, flat_e, bias=b1)
    exact_h = moe._glu_exact(proj, spec, I)
    fro, maxabs = _errs_rounded_bf16(h.float().cpu().numpy(), exact_h)
    assert fro <= 1e-2 and maxabs <= 2e-2, ("gate_up", fro, maxabs)
    out = ops.decode_down_combine(h, torch.from_numpy(idx).to(DEV), wts.to(DEV), w2, torch.float32)
    b2 = None if w2.bias is None else w2.bias.float().cpu().numpy().astype(np.float64)
    dn = _gemm_oracle(h.float().cpu().numpy(), W2, flat_e, bias=b2)
    want = (dn.reshape(T, top, H) * wts.float().numpy()[..., None]).sum(1)
    fro2, maxabs2 = _errs(out.cpu().numpy(), want)
    assert out.dtype == torch.float32 and fro2 <= 1e-4, ("down+combine", fro2, maxabs2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", ["nf4", "nf4_dq", "mxfp4"])
@pytest.mark.parametrize("T,H,I,epi", [(8, 2048, 192, "swiglu"), (2, 2048, 192, "none"), (8, 1600, 192, "swiglu"),
                                       (5, 2880, 192, "gptoss"), (6, 2880, 192, "none"), (3, 2048, 190, "swiglu")])
def test_decode_items_match_one_token_kernel(fmt, T, H, I, epi, dt):
    """2..8 tokens whose activations fit 16384 LDS elements run gate_up as per-wave work items
    over all tokens at once; one token runs one block per (column tile, routed expert). Both
    take the same chunk slots, table entries and reduction order per output element, so every
    h row of a batch equals the same token run alone, bit for bit. Covers the full stage
    (8 x 2048), rows whose chunk count is not a multiple of the lane group (H = 1600, 2880),
    the one-token-per-item edge (6 x 2880 > 16384 falls back to the per-expert kernel, also
    bit-identical), output widths that leave the last item's columns partly past the end
    (I = 190) and plain / SwiGLU / gpt-oss epilogues (biases for e2m1 and gpt-oss)."""
    _announce(f"decode items fmt={fmt} T={T} H={H} I={I} epi={epi} dt={dt}")
    E, top = 16, 8
    gated = epi != "none"
    w1, _ = _stack(fmt, E, 2 * I if gated else I, H, seed=40)
    code = {"none": N.EPI_NONE, "swiglu": N.EPI_SWIGLU, "gptoss": N.EPI_GPTOSS}[epi]
    if fmt == "mxfp4" or epi == "gptoss":  # the gpt-oss epilogue takes the gate_up bias
        g = torch.Generator().manual_seed(41)
        w1.bias = (torch.randn(E, w1.n, generator=g) * 0.1).to(dt).to(DEV)
    rng = np.random.default_rng(42 + T)
    idx = torch.from_numpy(np.stack([rng.permutation(E)[:top] for _ in range(T)]).astype(np.int64)).to(DEV)
    x = (torch.randn(T, H, generator=torch.Generator().manual_seed(43)) * 2).to(dt).to(DEV)
    h = ops.decode_gate_up(x, idx, w1, code)
    for t in range(T):
        one = ops.decode_gate_up(x[t:t + 1], idx[t:t + 1], w1, code)
        assert np.array_equal(_bits(h[t * top:(t + 1) * top]), _bits(one)), ("token", t)


@pytest.mark.parametrize("rows", [65, 600])
def test_decode_rejects_batches_beyond_its_limit(rows):
    qw, _, _ = _nf4_stack(4, 128, 128, seed=26)
    idx = torch.zeros(rows, 1, dtype=torch.int64, device=DEV)
    with pytest.raises(N.NativeError, match="decode path"):
        ops.decode_gate_up(torch.zeros(rows, 128, dtype=torch.bfloat16, device=DEV), idx, qw, N.EPI_NONE)


@pytest.mark.parametrize("fmt", ["nf4", "nf4_dq", "mxfp4"])
def test_prefill_split_tiles_match_one_tile_list(fmt):
    """Prefill-sized forwards run 128-row tiles plus, for an expert whose last tile would hold
    at most 32 rows, one 32-row tile: two launches per projection. Every output element goes
    through the same MFMA sequence along k at any tile height, so the layer equals the route ->
    gate_up -> down -> combine chain over one 128-row tile list bit for bit; a few rows are also
    checked against the oracle."""
    _announce(f"prefill split tiles fmt={fmt}")
    E, H, I, top, T = 8, 256, 192, 2, 1200
    w1, W1 = _stack(fmt, E, 2 * I, H, seed=40)
    w2, W2 = _stack(fmt, E, H, I, seed=41)
    epi, spec = N.EPI_SWIGLU, "swiglu"
    if fmt == "mxfp4":
        g = torch.Generator().manual_seed(43)
        w1.bias = (torch.randn(E, 2 * I, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
        w2.bias = (torch.randn(E, H, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
        epi, spec = N.EPI_GPTOSS, ("gptoss", 1.702, 7.0)
    rng = np.random.default_rng(42)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    idx = np.stack([rng.choice(E, size=top, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int64)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    rem = counts % 128
    assert ((rem > 0) & (rem <= 32)).any() and (rem > 32).any() and T * top >= 64 * E  # both tile lists in use
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(44)).to(torch.bfloat16).to(DEV)
    wts = torch.rand(T, top, generator=torch.Generator().manual_seed(45)).to(torch.bfloat16).to(DEV)
    ti = torch.from_numpy(idx).to(DEV)
    got = ops.moe_forward(x, ti, wts, w1, w2, epi, torch.bfloat16)
    rb = ops.route(ti, E, tile_m=128)
    h = ops.grouped_gemm(x, w1, rb, T, T * top, epilogue=epi, gather_k=top, path=N.PATH_MFMA)
    dn = ops.grouped_gemm(h, w2, rb, T, T * top, path=N.PATH_MFMA, out_dtype=torch.float32)
    want = ops.combine(dn, rb, wts, T, top, torch.bfloat16)
    assert torch.equal(got, want)
    rows = [0, 1, 599, 1199]
    b1 = None if w1.bias is None else w1.bias.float().cpu().numpy().astype(np.float64)
    b2 = None if w2.bias is None else w2.bias.float().cpu().numpy().astype(np.float64)
    flat = np.array([r * top + s for r in rows for s in range(top)])
    proj = _gemm_oracle(x.float().cpu().numpy()[flat // top], numerics.round_bf16(W1), idx.reshape(-1)[flat], bias=b1)
    hh = numerics.round_bf16(moe._glu_exact(proj, spec, I).astype(np.float32))
    d = _gemm_oracle(hh, numerics.round_bf16(W2), idx.reshape(-1)[flat], bias=b2)
    oracle = (d.reshape(len(rows), top, H) * wts.float().cpu().numpy()[rows][..., None]).sum(1)
    fro, maxabs = _errs(got[rows].float().cpu().numpy(), oracle)
    assert fro <= 1e-2 and maxabs <= 2e-2, (fro, maxabs)


@pytest.mark.parametrize("gated", [False, True])
def test_mfma_output_columns_not_a_multiple_of_eight(gated):
    """Output rows of 100 columns (a partial tile in n, rows not 16-byte multiples); 40 tokens
    over 4 experts leave partial tiles in m as well."""
    _announce(f"mfma odd output width gated={gated}")
    E, H, cols, top, T = 4, 256, 100, 2, 40
    n = 2 * cols if gated else cols
    qw, _, _ = _nf4_stack(E, n, H, seed=50)
    W = _dense_from_oracle(qw)
    rng = np.random.default_rng(51)
    idx = np.stack([rng.permutation(E)[:top] for _ in range(T)]).astype(np.int64)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(52)).to(torch.bfloat16)
    rb = ops.route(torch.from_numpy(idx).to(DEV), E)
    ref = orouting.route(idx, E)
    proj = _gemm_oracle(x.float().numpy()[ref["token_rows"]], numerics.round_bf16(W), idx.reshape(-1)[ref["order"]])
    epi = N.EPI_SWIGLU if gated else N.EPI_NONE
    exact = moe._glu_exact(proj, "swiglu", cols) if gated else proj
    for od in (torch.bfloat16, torch.float32):
        out = ops.grouped_gemm(x.to(DEV), qw, rb, T, T * top, epi, gather_k=top, path=N.PATH_MFMA, out_dtype=od)
        assert out.shape == (T * top, cols) and out.dtype == od
        if od == torch.float32:
            fro, _ = _errs(out.cpu().numpy(), exact)
            assert fro < 1e-5, fro
        else:
            fro, maxabs = _errs_rounded_bf16(out.float().cpu().numpy(), exact)
            assert fro <= 1e-2 and maxabs <= 2e-2, (fro, maxabs)
