"""Pins the CPU oracle (test infrastructure) before anything is checked against it.

Each check is chosen so a plausible mistake in the oracle fails it: a wrong code literal, a
swapped nibble order, a wrong block index, a dropped term, a transposed operand, an unstable
sort. Sources: the reference's golden vectors and special cases, transformers-written fixtures,
closed forms, and brute force on tiny inputs.
"""
import os

import numpy as np
import pytest
import torch

from oracle import c_oracle, codes, moe, numerics, quant, routing

GOLD = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------------------- numerics


def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(100000, generator=g) * 10 ** torch.randint(-20, 20, (100000,), generator=g).float(),
                   torch.tensor([0.0, -0.0, 1.0, 65504.0, 1e-40, 3.4e38, 1.00390625, 1.01171875])])
    ours = numerics.f32_to_bf16_bits(x.numpy())
    theirs = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


def test_bf16_rounding_ties_to_even():
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1.0078125 -> even (1.0)
    assert numerics.round_bf16(np.float32(1.0 + 2 ** -8)) == np.float32(1.0)
    # 1 + 3*2^-8 is halfway between 1.0078125 (odd) and 1.015625 (even) -> 1.015625
    assert numerics.round_bf16(np.float32(1.0 + 3 * 2 ** -8)) == np.float32(1.015625)


# ------------------------------------------------------------------------------ code tables


def test_nf4_table_rebuilds_from_normal_quantiles_bit_exactly():
    rebuilt = codes.normal_map_nf4()
    assert rebuilt.dtype == np.float32
    assert np.array_equal(rebuilt.view(np.uint32), codes.NF4_CODE.view(np.uint32))


def test_nf4_table_structure():
    c = codes.NF4_CODE
    assert c.shape == (16,) and np.all(np.diff(c) > 0)
    assert c[0] == -1.0 and c[-1] == 1.0 and c[7] == 0.0
    assert (c > 0).sum() == 8 and (c < 0).sum() == 7  # the asymmetric "extra" positive value


def test_nf4_table_perturbation_is_detected():
    # a one-ulp slip in a transcribed literal must fail the rebuild check above
    bad = codes.NF4_CODE.copy()
    bad[9] = np.nextafter(bad[9], np.float32(1))
    assert not np.array_equal(codes.normal_map_nf4(), bad)


def test_fp4_table_structure():
    c = codes.FP4_CODE
    assert c.shape == (16,) and c[3] == 1.0 and np.all(c[8:] == -c[:8])
    assert sorted(np.abs(c[:8]) * 12) == [0.0, 0.0625, 2.0, 3.0, 4.0, 6.0, 8.0, 12.0]


def test_fp4_table_matches_published_decode_tree_bit_for_bit():
    tree = np.array([codes.fp4_tree_value(n) for n in range(16)], np.float32)
    assert np.array_equal(tree.view(np.uint32), codes.FP4_CODE.view(np.uint32))
    # a plausible transcription slip (two magnitudes swapped) fails the check
    bad = codes.FP4_CODE.copy()
    bad[[4, 6]] = bad[[6, 4]]
    assert not np.array_equal(tree.view(np.uint32), bad.view(np.uint32))


def test_dynamic_map_structure():
    m = codes.dynamic_map_signed()
    assert m.shape == (256,) and np.all(np.diff(m) >= 0)
    assert m[-1] == 1.0 and (m == 0).sum() == 1
    pos, neg = m[m > 0], m[m < 0]
    assert pos.size == 128 and neg.size == 127
    # every negative entry mirrors a positive one; 1.0 is the unmatched extra
    assert np.allclose(np.sort(-neg), np.sort(pos[:-1]))


def _within_ulps_of_exact(table, exact, ulps=2.0):
    """Every fp32 entry within ``ulps`` of its exact rational value (same sorted position)."""
    from fractions import Fraction

    t = np.asarray(table, np.float32)
    if t.shape != (len(exact),):
        return False
    for v, ex in zip(t, exact):
        if ex == 0:
            if v != 0:
                return False
            continue
        if abs(Fraction(float(v)) - ex) > Fraction(ulps) * Fraction(float(np.spacing(np.abs(v)))):
            return False
    return True


def _dynamic_map_variant(points=lambda i: 2 ** i + 1, decade=lambda i: i - 6):
    """The fp32 construction with a swappable grid size / decade: the negative controls."""
    data = []
    for i in range(7):
        b = torch.linspace(0.1, 1, points(i), dtype=torch.float32)
        means = (b[:-1] + b[1:]) / 2.0
        data += ((10 ** decade(i)) * means).tolist() + ((-(10 ** decade(i))) * means).tolist()
    data += [0.0, 1.0]
    data += [0.0] * (256 - len(data))
    return np.array(sorted(data), np.float32)


def test_dynamic_map_within_two_ulps_of_its_exact_construction():
    exact = codes.dynamic_map_exact()
    assert len(exact) == 256 and exact[127] == 0 and exact[255] == 1
    assert _within_ulps_of_exact(codes.dynamic_map_signed(), exact)


def test_dynamic_map_negative_controls_fail_the_exact_check():
    exact = codes.dynamic_map_exact()
    assert _within_ulps_of_exact(_dynamic_map_variant(), exact)  # the construction itself passes
    # a grid one point short in every decade (2**i points instead of 2**i + 1)
    assert not _within_ulps_of_exact(_dynamic_map_variant(points=lambda i: max(2 ** i, 2)), exact)
    # every decade one power of ten too small
    assert not _within_ulps_of_exact(_dynamic_map_variant(decade=lambda i: i - 7), exact)


def _hand_derived_cell(i, j):
    """fp32 value of decade ``i``'s cell ``j`` in the construction's own fp32 steps, for the first
    (j = 0) and last (j = 2**i - 1) cell of a decade: boundaries ``start, start + step`` or
    ``1 - step, 1`` (``step = fl32(1 - 0.1f) / 2**i``, exact), midpoint ``fl32(a + b) / 2``,
    value ``fl32(fl32(10**(i-6)) * midpoint)``."""
    f = np.float32
    start, end = f(0.1), f(1.0)
    step = f(f(end - start) / f(2 ** i))
    if j == 0:
        a, b = start, f(start + step)
    else:
        assert j == 2 ** i - 1
        a, b = f(end - step), end
    mid = f(f(a + b) / f(2))
    return f(f(10.0 ** (i - 6)) * mid)


def test_dynamic_map_hand_derived_bits():
    m = codes.dynamic_map_signed().view(np.uint32)
    for idx, bits in codes.DYNAMIC_MAP_PINS.items():
        assert int(m[idx]) == bits, (idx, hex(int(m[idx])), hex(bits))
    # the pins are the fp32 steps of the construction, repeated here in numpy
    for i in range(7):
        for j in {0, 2 ** i - 1}:
            pos = 128 + (2 ** i - 1) + j
            want = _hand_derived_cell(i, j)
            assert int(np.array([want], np.float32).view(np.uint32)[0]) == codes.DYNAMIC_MAP_PINS[pos], (i, j)
            # the mirrored negative entry
            assert m[254 - pos] == np.array([-want], np.float32).view(np.uint32)[0]


# ------------------------------------------------------------------------------ NF4 decode


def test_nf4_hand_values():
    c = codes.NF4_CODE
    # 0x7F: high nibble 7 (0.0) first, low nibble 15 (1.0); absmax 2 -> [0, 2]
    # 0x0F: [-1, 1] * 2; 0xF0 with the second block's absmax 0.5 -> [0.5, -0.5]
    packed = np.zeros(64, np.uint8)
    packed[0], packed[1], packed[32] = 0x7F, 0x0F, 0xF0
    out = quant.dequant_nf4(packed, np.array([2.0, 0.5], np.float32))
    assert out[0] == 0.0 and out[1] == 2.0 and out[2] == -2.0 and out[3] == 2.0
    assert out[64] == 0.5 and out[65] == -0.5
    assert out[4] == np.float32(c[0]) * 2  # byte 0x00 -> code[0] = -1


def test_nf4_golden_fixture():
    d = np.load(os.path.join(GOLD, "nf4_hand.npz"))
    out = quant.dequant_nf4(d["packed"], d["absmax"])
    assert np.array_equal(out.view(np.uint32), d["expected"].view(np.uint32))


def test_nf4_decode_bruteforce_tiny():
    rng = np.random.default_rng(3)
    packed = rng.integers(0, 256, 96, dtype=np.uint8)        # 192 values = 3 blocks
    absmax = rng.random(3).astype(np.float32) + 0.1
    vec = quant.dequant_nf4(packed, absmax)
    for i in range(192):
        b = int(packed[i // 2])
        nib = (b >> 4) if i % 2 == 0 else (b & 15)
        assert vec[i] == np.float32(codes.NF4_CODE[nib]) * np.float32(absmax[i // 64])


def test_nf4_decode_rounding_to_bf16_is_one_rounding_of_the_fp32_product():
    rng = np.random.default_rng(4)
    packed = rng.integers(0, 256, 512, dtype=np.uint8)
    absmax = (rng.random(16) * 0.1).astype(np.float32)
    f32 = quant.dequant_nf4(packed, absmax, dtype="fp32")
    b16 = quant.dequant_nf4(packed, absmax, dtype="bf16")
    assert np.array_equal(b16, torch.from_numpy(f32).to(torch.bfloat16).float().numpy())


def test_whole_stack_equals_per_expert_decode():
    # blocks never straddle experts (_vendor/experts.py:220-226; test_fused_train_parity.py:241-281)
    rng = np.random.default_rng(5)
    E, n, k = 3, 8, 128
    w = rng.standard_normal((E, n * k)).astype(np.float32) * 0.02
    packed, absmax = quant.quantize_nf4(w)
    whole = quant.dequant_nf4(packed.reshape(-1), absmax.reshape(-1))
    for e in range(E):
        one = quant.dequant_nf4(packed[e], absmax[e])
        assert np.array_equal(one, whole[e * n * k:(e + 1) * n * k])


def test_quantizer_roundtrip_error_and_nearest_code():
    rng = np.random.default_rng(6)
    w = rng.standard_normal((4, 4096)).astype(np.float32) * 0.02
    packed, absmax = quant.quantize_nf4(w)
    deq = quant.dequant_nf4(packed, absmax)
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert 0.05 < rel < 0.15  # NF4 on Gaussian weights: ~0.09
    # every decoded value is the nearest code point of its scaled input
    scaled = (w.reshape(4, -1, 64) / absmax[..., None]).reshape(4, -1)
    idx = quant.unpack_nibbles_hi_first(packed)
    dist = np.abs(scaled[..., None] - codes.NF4_CODE)
    assert np.all(dist[np.arange(4)[:, None], np.arange(4096)[None], idx] <= dist.min(-1) + 1e-6)


def test_c_restatement_matches_numpy_nf4():
    rng = np.random.default_rng(7)
    packed = rng.integers(0, 256, 4096, dtype=np.uint8)
    absmax = rng.random(128).astype(np.float32)
    a = c_oracle.dequant_4bit(packed, absmax, codes.NF4_CODE)
    b = quant.dequant_nf4(packed, absmax)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    a16 = c_oracle.dequant_4bit(packed, absmax, codes.NF4_CODE, out="bf16")
    assert np.array_equal(a16, numerics.f32_to_bf16_bits(b))


# ------------------------------------------------------------------------ double quant


def test_double_quant_closed_form():
    code2 = codes.dynamic_map_signed()
    q = np.array([255, 0, 128, 127] * 130, dtype=np.uint8)  # 520 blocks -> 3 second-level blocks
    absmax2 = np.array([0.5, 2.0, 0.25], np.float32)
    offset = np.float32(0.125)
    out = quant.dequant_absmax_dq(q[None], absmax2[None], np.array([offset]), code2)[0]
    for b in (0, 1, 2, 3, 255, 256, 300, 511, 512, 519):
        want = np.float32(np.float32(code2[q[b]] * absmax2[b // 256]) + offset)
        assert out[b] == want
    assert out[0] == np.float32(1.0 * 0.5 + 0.125)  # code2[255] == 1.0


def test_double_quant_reconstruction():
    rng = np.random.default_rng(8)
    a = (rng.random((2, 1000)) * 0.05 + 0.01).astype(np.float32)
    q, a2, off = quant.double_quant_absmax(a)
    rec = quant.dequant_absmax_dq(q, a2, off)
    assert q.dtype == np.uint8 and a2.shape == (2, 4) and off.shape == (2,)
    assert np.max(np.abs(rec - a)) < 0.01 * np.max(np.abs(a))
    ca = c_oracle.dequant_absmax_dq(q[1], a2[1], off[1], codes.dynamic_map_signed())
    assert np.array_equal(ca, rec[1])


# ------------------------------------------------------------------------------- MXFP4


def test_mxfp4_reference_golden_vector():
    d = np.load(os.path.join(GOLD, "mxfp4_reference_vector.npz"))
    out = quant.dequantize_mxfp4(d["blocks"], d["scales"], dtype="fp32")
    assert out.shape == (1, 4, 2)
    assert np.array_equal(out, d["expected"])


@pytest.mark.parametrize("case", ["a", "b", "c"])
@pytest.mark.parametrize("dt", ["bf16", "fp32"])
def test_mxfp4_matches_transformers_fixtures(case, dt):
    d = np.load(os.path.join(GOLD, "mxfp4_transformers.npz"))
    out = quant.dequantize_mxfp4(d[f"{case}_blocks"], d[f"{case}_scales"], dtype=dt)
    want = d[f"{case}_{dt}"]
    if dt == "bf16":
        assert np.array_equal(numerics.f32_to_bf16_bits(out), want)
    else:
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


def test_mxfp4_c_restatement_matches_numpy():
    d = np.load(os.path.join(GOLD, "mxfp4_transformers.npz"))
    blocks, scales = d["b_blocks"], d["b_scales"]
    rows = int(np.prod(blocks.shape[:-2]))
    K = blocks.shape[-2] * blocks.shape[-1] * 2
    a = c_oracle.dequant_mxfp4(blocks, scales, rows, K)
    b = quant.dequant_mxfp4_rows(blocks, scales).reshape(rows, K)
    assert np.array_equal(a, b)


def test_mxfp4_quantizer_roundtrip():
    rng = np.random.default_rng(9)
    w = rng.standard_normal((8, 2880)).astype(np.float32) * 0.02
    blocks, scales = quant.quantize_mxfp4(w)
    rec = quant.dequant_mxfp4_rows(blocks, scales).reshape(8, 2880)
    rel = np.linalg.norm(rec - w) / np.linalg.norm(w)
    assert rel < 0.2
    # e2m1 grid points are reproduced exactly
    grid = np.tile(quant.FP4_VALUES[:8], 4)[None].astype(np.float32) * np.float32(0.25)
    b2, s2 = quant.quantize_mxfp4(grid)
    assert np.array_equal(quant.dequant_mxfp4_rows(b2, s2).reshape(grid.shape), grid)


# ----------------------------------------------------------------------------- routing


def test_route_matches_bruteforce_tiny():
    rng = np.random.default_rng(10)
    for T, k, E in ((1, 8, 64), (5, 2, 4), (16, 3, 7), (33, 8, 128)):
        idx = np.stack([rng.permutation(E)[:k] for _ in range(T)])
        r = routing.route(idx, E)
        assert np.array_equal(r["order"], routing.route_bruteforce(idx, E))
        assert np.array_equal(r["inv"][r["order"]], np.arange(T * k))
        assert np.array_equal(np.diff(r["offsets"]), np.bincount(idx.reshape(-1), minlength=E))


def test_route_is_stable_on_duplicates():
    idx = np.array([[1, 1], [0, 1], [1, 0]])
    r = routing.route(idx, 2)
    # expert 0 rows in flat order (2, 5), then expert 1 rows (0, 1, 3, 4)
    assert r["order"].tolist() == [2, 5, 0, 1, 3, 4]
    assert r["token_rows"].tolist() == [1, 2, 0, 0, 1, 2]
    assert r["top_pos"].tolist() == [0, 1, 0, 1, 1, 0]


def test_route_special_cases():
    # all tokens to experts {0, 1} (test_fast.py:110-120): experts 2, 3 empty
    idx = np.stack([np.zeros(8, int), np.ones(8, int)], 1)
    r = routing.route(idx, 4)
    assert r["counts"].tolist() == [8, 8, 0, 0] and r["active"].tolist() == [0, 1]
    # E=64 sparse hits (test_reference_parity.py:185-204)
    rng = np.random.default_rng(11)
    idx = rng.integers(0, 64, (8, 2))
    r = routing.route(idx, 64)
    assert set(r["active"].tolist()) == set(idx.reshape(-1).tolist())
    c_order, c_inv, c_off = c_oracle.route(idx, 64)
    assert np.array_equal(c_order, r["order"]) and np.array_equal(c_off, r["offsets"])


def test_m_tiles_cover_every_row_once():
    counts = np.array([0, 130, 1, 64, 65])
    tiles = routing.m_tiles(counts, 64)
    assert tiles == [(1, 0), (1, 64), (1, 128), (2, 130), (3, 131), (4, 195), (4, 259)]


# ---------------------------------------------------------------------------- forwards


def _tiny_problem(seed=0, E=6, H=128, I=64, T=12, k=2):
    rng = np.random.default_rng(seed)
    w1 = rng.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.05
    w2 = rng.standard_normal((E, H, I)).astype(np.float32) * 0.05
    x = rng.standard_normal((T, H)).astype(np.float32)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    wts = rng.random((T, k)).astype(np.float32)
    return x, idx, wts, w1, w2


def _torch_float_moe(x, idx, wts, w1, w2, swap=False, drop=False, roll=0):
    """Independent float reference in torch (structure of test_reference_parity.py:71-92)."""
    x, w1, w2 = (torch.from_numpy(a).double() for a in (x, w1, w2))
    idx_t, wts_t = torch.from_numpy(idx), torch.from_numpy(wts).double()
    out = torch.zeros(x.shape[0], w2.shape[1], dtype=torch.float64)
    E = w1.shape[0]
    for e in range(E):
        tok, pos = (idx_t == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        ew = (e + roll) % E
        p = torch.nn.functional.linear(x[tok], w1[ew])
        g, u = p.chunk(2, -1)
        if swap:
            g, u = u, g
        y = torch.nn.functional.linear(torch.nn.functional.silu(g) * u, w2[ew])
        if not drop:
            y = y * wts_t[tok, pos, None]
        out.index_add_(0, tok, y)
    return out.numpy()


def test_oracle_forward_matches_independent_torch_reference_and_rejects_bugs():
    x, idx, wts, w1, w2 = _tiny_problem()
    got = moe.forward_fp32(x, idx, wts, w1, w2)
    ok = np.linalg.norm(got - _torch_float_moe(x, idx, wts, w1, w2)) / np.linalg.norm(got)
    assert ok < 1e-6
    for bug in (dict(swap=True), dict(drop=True), dict(roll=1)):
        bad = _torch_float_moe(x, idx, wts, w1, w2, **bug)
        assert np.linalg.norm(got - bad) / np.linalg.norm(got) > 0.3, bug


def test_fused_numerics_close_to_fp32_oracle():
    x, idx, wts, w1, w2 = _tiny_problem(seed=1)
    want = moe.forward_fp32(x, idx, wts, w1, w2)
    got = moe.forward_fused_numerics(x, idx, wts, w1, w2)
    fro, maxabs, _ = moe.rel_errors(got, want)
    assert fro < 1e-2 and maxabs < 4e-2


def test_epilogue_variants_closed_form():
    p = np.array([[0.5, -2.0, 9.0, 1.0, -8.0, 3.0]], np.float32)  # gate | up halves of 3
    sw = moe.epilogue_rounded(p, "swiglu", 3, "fp32")
    assert np.allclose(sw, numerics.silu_f32(p[:, :3]) * p[:, 3:])
    cl = moe.epilogue_rounded(p, ("clamp_swiglu", 2.0), 3, "fp32")
    g = np.minimum(p[:, :3], 2.0)
    u = np.clip(p[:, 3:], -2.0, 2.0)
    assert np.allclose(cl, numerics.silu_f32(g) * u)
    assert not np.allclose(cl, sw)
    go = moe.epilogue_rounded(p, ("gptoss", 1.702, 7.0), 3, "fp32", b1=np.zeros(6, np.float32))
    g = np.minimum(p[:, :3], 7.0)
    u = np.clip(p[:, 3:], -7.0, 7.0)
    assert np.allclose(go, (u + 1) * (g * (1 / (1 + np.exp(-1.702 * g)))), rtol=1e-6)


def test_reference_loop_port_matches_oracle():
    x, idx, wts, w1, w2 = _tiny_problem(seed=2)
    w1t, w2t = torch.from_numpy(w1), torch.from_numpy(w2)
    got = moe.reference_loop(torch.from_numpy(x), torch.from_numpy(idx), torch.from_numpy(wts),
                             lambda e, dt: w1t[e].to(dt), lambda e, dt: w2t[e].to(dt), num_experts=6)
    want = moe.forward_fp32(x, idx, wts, w1, w2)
    assert np.linalg.norm(got.numpy() - want) / np.linalg.norm(want) < 1e-5



# ------------------------------------------------------------------------------- LoRA oracle


def _tiny_lora(seed=3, E=6, H=128, I=64, r=4):
    rng = np.random.default_rng(seed)
    A1 = rng.standard_normal((E, r, H)).astype(np.float32) * 0.2
    B1 = rng.standard_normal((E, 2 * I, r)).astype(np.float32) * 0.2
    A2 = rng.standard_normal((E, r, I)).astype(np.float32) * 0.2
    B2 = rng.standard_normal((E, H, r)).astype(np.float32) * 0.2
    return (A1, B1), (A2, B2)


def test_lora_oracle_zero_adapter_is_the_base_oracle():
    x, idx, wts, w1, w2 = _tiny_problem(seed=4)
    (A1, B1), (A2, B2) = _tiny_lora()
    got = moe.forward_lora_fp32(x, idx, wts, w1, w2, (A1, 0 * B1), (A2, 0 * B2), 2.0)
    want = moe.forward_fp32(x, idx, wts, w1, w2)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7)


def test_lora_oracle_closed_form_and_negative_control():
    """One token, one expert, rank 1: the delta is scaling * (x.a) * b, added BEFORE the
    activation; the same delta added after the activation (a plausible bug) must differ."""
    x, idx, wts, w1, w2 = _tiny_problem(seed=5, T=1, k=1)
    E, N1, H = w1.shape
    rng = np.random.default_rng(6)
    a1, b1 = rng.standard_normal(H), rng.standard_normal(N1)
    a2, b2 = rng.standard_normal(w2.shape[2]), rng.standard_normal(w2.shape[1])
    A1 = np.zeros((E, 1, H)); B1 = np.zeros((E, N1, 1))
    A2 = np.zeros((E, 1, w2.shape[2])); B2 = np.zeros((E, w2.shape[1], 1))
    e = int(idx[0, 0])
    A1[e, 0], B1[e, :, 0], A2[e, 0], B2[e, :, 0] = a1, b1, a2, b2
    s = 0.5
    got = moe.forward_lora_fp32(x, idx, wts, w1, w2, (A1, B1), (A2, B2), s)
    xd = x[0].astype(np.float64)
    proj = w1[e].astype(np.float64) @ xd + s * (xd @ a1) * b1
    g, u = proj[: N1 // 2], proj[N1 // 2:]
    h = g / (1 + np.exp(-g)) * u
    y = w2[e].astype(np.float64) @ h + s * (h @ a2) * b2
    want = y * wts[0, 0]
    assert np.allclose(got[0], want, rtol=1e-5, atol=1e-6)
    # negative control: the gate_up delta after the SwiGLU
    p0 = w1[e].astype(np.float64) @ xd
    h_bad = p0[: N1 // 2] / (1 + np.exp(-p0[: N1 // 2])) * p0[N1 // 2:] + (s * (xd @ a1) * b1)[: N1 // 2]
    bad = (w2[e].astype(np.float64) @ h_bad + s * (h_bad @ a2) * b2) * wts[0, 0]
    assert np.linalg.norm(got[0] - bad) / np.linalg.norm(want) > 0.05


@pytest.mark.parametrize("T", [1, 12])
def test_reference_lora_loop_matches_the_lora_oracle(T):
    """The reference's own loop (both its decode and its mask path) against the exact form,
    in fp32 (tight) and bf16 compute (the reference's rounding, loose)."""
    x, idx, wts, w1, w2 = _tiny_problem(seed=7, T=T)
    (A1, B1), (A2, B2) = _tiny_lora(seed=8)
    want = moe.forward_lora_fp32(x, idx, wts, w1, w2, (A1, B1), (A2, B2), 2.0)
    t = torch.from_numpy
    w1t, w2t = t(w1), t(w2)
    lo1, lo2 = (t(A1), t(B1)), (t(A2), t(B2))
    for cd, tol in ((torch.float32, 1e-5), (torch.bfloat16, 3e-2)):
        got = moe.reference_lora_loop(t(x), t(idx), t(wts), lambda e, dt: w1t[e].to(dt), lambda e, dt: w2t[e].to(dt),
                                      lo1, lo2, 2.0, num_experts=6, compute_dtype=cd)
        fro = np.linalg.norm(got.float().numpy() - want) / np.linalg.norm(want)
        assert fro < tol, (cd, fro)


# ----------------------------------------------------------------------------------- routers


def _router_bruteforce(logits_row, k, kind, renorm):
    """Pure-Python routing epilogue: rank experts by (-logit, index), softmax in fp64."""
    import math

    z = [float(v) for v in logits_row]
    ranked = sorted(range(len(z)), key=lambda e: (-z[e], e))[:k]
    if kind == routing.SOFTMAX_THEN_TOPK:
        mx = max(z)
        den = sum(math.exp(v - mx) for v in z)
        w = [math.exp(z[e] - mx) / den for e in ranked]
        if renorm:
            tot = sum(w)
            w = [v / tot for v in w]
    else:
        mx = max(z[e] for e in ranked)
        den = sum(math.exp(z[e] - mx) for e in ranked)
        w = [math.exp(z[e] - mx) / den for e in ranked]
    return w, ranked


@pytest.mark.parametrize("kind,renorm", [(routing.SOFTMAX_THEN_TOPK, False), (routing.SOFTMAX_THEN_TOPK, True),
                                         (routing.TOPK_THEN_SOFTMAX, False)])
def test_router_matches_bruteforce(kind, renorm):
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((20, 16)).astype(np.float32)
    logits[3, [2, 7, 11]] = 5.0  # ties resolve to the lower expert index
    w, i = routing.router_topk(logits, 4, kind, renorm)
    for t in range(20):
        bw, bi = _router_bruteforce(logits[t], 4, kind, renorm)
        assert list(i[t]) == bi
        assert np.allclose(w[t], bw, rtol=1e-6)
    assert list(i[3][:3]) == [2, 7, 11]
