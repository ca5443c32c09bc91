"""Host-side behaviour of the drop-in module API, on the CPU.

Mirrors the reference's CPU-runnable tests: construction and validation
(``_vendor/experts.py:194-276``), the state_dict / ``_extra_state`` contract (``:278-327``,
``tests/test_nbit_schemes.py``), the per-expert reference forward against the oracle
(``tests/test_reference_parity.py`` level 1, with its negative controls), eligibility and the
static positional-signature contract (``tests/test_fast_staging_composition.py``).
"""
import ast
import inspect
import io
import os

import numpy as np
import pytest
import torch

import experts4bit_qlora_amd as e4b
from experts4bit_qlora_amd import fast as F
from experts4bit_qlora_amd import quant as Q
from oracle import codes, moe
from oracle import quant as oq


def _weights(E=4, H=128, inter=192, seed=0, has_gate=True):
    torch.manual_seed(seed)
    gu = torch.randn(E, 2 * inter if has_gate else inter, H) * 0.1
    dn = torch.randn(E, H, inter) * 0.1
    return gu, dn


def test_code_tables_match_oracle():
    assert np.array_equal(Q.code_4bit("nf4").numpy(), codes.NF4_CODE)
    assert np.array_equal(Q.code_4bit("fp4").numpy(), codes.FP4_CODE)
    assert np.array_equal(Q.dynamic_map().numpy(), codes.dynamic_map_signed())


def test_quantizer_matches_oracle_bytes():
    w = torch.randn(3, 8192) * 0.02
    p, a = Q.quantize_4bit(w)
    op, oa = oq.quantize_nf4(w.numpy())
    assert np.array_equal(a.numpy(), oa)
    assert (p.numpy() != op).mean() < 1e-4  # midpoint ties are measure-zero


def test_mxfp4_quantizer_matches_oracle_bytes():
    w = torch.randn(4, 2880) * 0.02
    b, s = Q.quantize_mxfp4(w)
    ob, os_ = oq.quantize_mxfp4(w.numpy())
    assert np.array_equal(s.numpy(), os_)
    assert np.array_equal(b.numpy(), ob.reshape(4, -1))


def test_storage_layout_and_shapes():
    gu, dn = _weights()
    m = e4b.Experts4bit.from_float(gu, dn, compute_dtype=torch.bfloat16)
    assert m.gate_up_proj.shape == (4, 384 * 128 // 2) and m.gate_up_proj.dtype == torch.uint8
    assert m.gate_up_absmax.shape == (4, 384 * 128 // 64) and m.gate_up_absmax.dtype == torch.float32
    assert m.down_proj.shape == (4, 128 * 192 // 2)
    assert not m.gate_up_proj.requires_grad
    assert "code" not in m.state_dict()
    # each expert's bytes equal an independent per-expert quantization
    for e in range(4):
        p, a = Q.quantize_4bit(gu[e].reshape(1, -1))
        assert torch.equal(p[0], m.gate_up_proj[e]) and torch.equal(a[0], m.gate_up_absmax[e])


def test_constructor_validation():
    with pytest.raises(ValueError, match="divisible by blocksize"):
        e4b.ExpertsNbit(2, 100, 64)
    with pytest.raises(ValueError, match="quant_type must be one of"):
        e4b.Experts4bit(2, 64, 64, quant_type="int8")
    with pytest.raises(ValueError, match="transposed"):
        e4b.Experts4bit.from_float(torch.randn(2, 128, 64), torch.randn(2, 64, 128).transpose(1, 2))
    assert e4b.normalize_quant_type(" BFloat16 ") == "bf16"


@pytest.mark.parametrize("dq", [False, True])
def test_state_dict_round_trip(dq):
    gu, dn = _weights()
    m = e4b.Experts4bit.from_float(gu, dn, compute_dtype=torch.bfloat16, compress_statistics=dq)
    buf = io.BytesIO()
    torch.save(m.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    m2 = e4b.Experts4bit(4, 128, 192, compute_dtype=torch.bfloat16, compress_statistics=dq)
    m2.load_state_dict(sd)
    for k, v in m.state_dict().items():
        if torch.is_tensor(v):
            assert torch.equal(v, m2.state_dict()[k]), k
    x = torch.randn(5, 128).to(torch.bfloat16)
    idx = torch.randint(0, 4, (5, 2))
    w = torch.rand(5, 2).to(torch.bfloat16)
    assert torch.equal(m(x, idx, w), m2(x, idx, w))


CHECKPOINT = os.path.join(os.path.dirname(__file__), "golden", "expertsnbit_nf4_checkpoint.pt")


@pytest.mark.parametrize("tensors_only", [False, True])
def test_reference_format_checkpoint_loads_and_decodes(tensors_only):
    """A state_dict in the reference's on-disk format (tests/golden/make_checkpoint.py, written
    from the format definition of _vendor/experts.py:236-327, not by this package) loads under
    strict=True, with its _extra_state or without it (a tensors-only / safetensors save), and the
    module's reference forward matches the fixture's fp64 expectation to bf16 accuracy."""
    d = torch.load(CHECKPOINT, weights_only=True)
    sd = dict(d["state_dict"])
    if tensors_only:
        sd = {k: v for k, v in sd.items() if not k.endswith("_extra_state")}
    m = e4b.Experts4bit(4, 128, 64, quant_type="nf4", compute_dtype=torch.bfloat16)
    m.load_state_dict(sd, strict=True)
    assert torch.equal(m.gate_up_proj, d["state_dict"]["gate_up_proj"])
    assert torch.equal(m.down_absmax, d["state_dict"]["down_absmax"])
    with torch.no_grad():
        out = m(d["x"], d["top_k_index"], d["top_k_weights"]).double()
    exp = d["expected"]
    assert ((out - exp).norm() / exp.norm()).item() < 1e-2
    # a module of another construction refuses the metadata
    with pytest.raises(ValueError, match="intermediate_dim|hidden_dim"):
        e4b.Experts4bit(4, 128, 128, quant_type="nf4").set_extra_state(d["state_dict"]["_extra_state"])


def test_extra_state_rejects_a_different_scheme_and_accepts_legacy():
    gu, dn = _weights()
    sd = e4b.Experts4bit.from_float(gu, dn, quant_type="fp4").state_dict()
    m = e4b.Experts4bit(4, 128, 192, quant_type="nf4")
    with pytest.raises(ValueError, match="quant_type"):
        m.load_state_dict(sd)
    legacy = {k: v for k, v in sd.items() if not k.endswith("_extra_state")}
    e4b.Experts4bit(4, 128, 192, quant_type="fp4").load_state_dict(legacy, strict=True)
    with pytest.raises(ValueError, match="schema"):
        m.set_extra_state({"schema": 99})


@pytest.mark.parametrize("quant_type", ["nf4", "fp4", "int8", "fp8", "bf16", "fp16"])
def test_cpu_reference_forward_tracks_float_and_rejects_bugs(quant_type):
    E, HID, INTER, TOP_K, N_TOK = 6, 128, 256, 2, 40
    gu, dn = _weights(E, HID, INTER)
    cls = e4b.Experts4bit if quant_type in ("nf4", "fp4") else e4b.ExpertsNbit
    m = cls.from_float(gu, dn, quant_type=quant_type, compute_dtype=torch.float32)
    hs = torch.randn(N_TOK, HID)
    idx = torch.randint(0, E, (N_TOK, TOP_K))
    wts = torch.rand(N_TOK, TOP_K)
    got = m(hs, idx, wts).numpy()
    want = moe.forward_fp32(hs.numpy(), idx.numpy(), wts.numpy(), gu.numpy(), dn.numpy())
    tol = {"nf4": 0.25, "fp4": 0.30, "int8": 0.03, "fp8": 0.08, "bf16": 8e-3, "fp16": 1e-3}[quant_type]
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert err < tol
    drop = moe.forward_fp32(hs.numpy(), idx.numpy(), np.ones_like(wts.numpy()), gu.numpy(), dn.numpy())
    assert err < 0.5 * np.linalg.norm(got - drop) / np.linalg.norm(drop)


def test_cpu_dequant_is_the_oracle_bit_for_bit():
    gu, dn = _weights()
    for dq in (False, True):
        m = e4b.Experts4bit.from_float(gu, dn, compress_statistics=dq)
        for e in (0, 3):
            got = m._dequantize_expert(m.gate_up_proj, m.gate_up_absmax, m._gate_up_shape, e, torch.float32)
            if dq:
                am = oq.dequant_absmax_dq(m.gate_up_absmax[e:e + 1].numpy(), m.gate_up_absmax2[e:e + 1].numpy(),
                                          m.gate_up_absmax_offset[e:e + 1].numpy(), m.code2.numpy())[0]
            else:
                am = m.gate_up_absmax[e].numpy()
            want = oq.dequant_nf4(m.gate_up_proj[e].numpy(), am).reshape(m._gate_up_shape)
            assert np.array_equal(got.numpy().view(np.uint32), want.view(np.uint32))


def test_lora_zero_adapter_is_bit_identical_to_base():
    gu, dn = _weights()
    base = e4b.Experts4bit.from_float(gu, dn, compute_dtype=torch.float32)
    lora = e4b.ExpertsLoRA(base, r=8, alpha=16)
    hs, idx, wts = torch.randn(10, 128), torch.randint(0, 4, (10, 2)), torch.rand(10, 2)
    assert torch.equal(lora(hs, idx, wts), base(hs, idx, wts))
    with pytest.raises(ValueError, match="rank r >= 1"):
        e4b.ExpertsLoRA(base, r=0)


def test_enable_fast_skips_cpu_storage_and_reports_reasons(capsys):
    gu, dn = _weights()
    m = e4b.Experts4bit.from_float(gu, dn)
    assert F._eligible(m) == "storage not on CUDA"
    assert e4b.enable_fast(m, verbose=True) == 0
    assert "storage not on CUDA" in capsys.readouterr().out
    m.blocksize = 128
    assert F._eligible(m).startswith("blocksize")
    m8 = e4b.ExpertsNbit.from_float(gu, dn, quant_type="int8")
    assert F._eligible(m8) == "storage is not nf4-4bit"
    m._e4b_mxfp4_arena = True
    assert "MXFP4" in F._eligible(m)


def test_fast_available_is_false_without_a_device():
    if torch.cuda.is_available():
        pytest.skip("a device is visible")
    assert e4b.fast_available() is False


def _func(fn):
    src = inspect.getsource(fn)
    return ast.parse(src).body[0]


@pytest.mark.parametrize("fn", [F.fused_experts_forward, F.fused_experts_lora_forward, F.fused_mxfp4_forward])
def test_top_k_index_is_the_second_positional_arg(fn):
    node = _func(fn)
    names = [a.arg for a in node.args.args]
    assert names[:4] == ["mod", "hidden_states", "top_k_index", "top_k_weights"]
    assert "top_k_index" not in [a.arg for a in node.args.kwonlyargs]


def test_enable_fast_does_not_guard_staging_attributes():
    src = ast.unparse(_func(F.enable_fast))
    for attr in ("_spec_dev", "_spec_ids", "_routed_only"):
        assert attr not in src


def test_product_never_imports_the_oracle():
    import pathlib

    pkg = pathlib.Path(e4b.__file__).parent
    for p in pkg.rglob("*.py"):
        tree = ast.parse(p.read_text())
        for node in ast.walk(tree):
            if isinstance(node, ast.Import):
                assert all(not a.name.startswith("oracle") for a in node.names), p
            if isinstance(node, ast.ImportFrom) and node.module:
                assert not node.module.startswith("oracle"), p


def test_mxfp4_format_api_on_cpu():
    import os

    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "mxfp4_reference_vector.npz"))
    out = e4b.dequantize_mxfp4(torch.from_numpy(d["blocks"]), torch.from_numpy(d["scales"]), dtype=torch.float32)
    assert torch.equal(out, torch.from_numpy(d["expected"]))
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "mxfp4_transformers.npz"))
    out = e4b.dequantize_mxfp4(torch.from_numpy(g["b_blocks"]), torch.from_numpy(g["b_scales"]), dtype=torch.bfloat16)
    assert np.array_equal(out.view(torch.int16).numpy().view(np.uint16), g["b_bf16"])
    with pytest.raises(ValueError, match="at least one leading row axis"):
        e4b.dequantize_mxfp4(torch.zeros(4, 16, dtype=torch.uint8), torch.zeros(4, dtype=torch.uint8))


def test_gptoss_mxfp4_cpu_reference_forward():
    g = torch.Generator().manual_seed(0)
    E, H, I = 4, 64, 64
    gu, dn = torch.randn(E, 2 * I, H, generator=g) * 0.05, torch.randn(E, H, I, generator=g) * 0.05
    b1, b2 = torch.randn(E, 2 * I, generator=g) * 0.05, torch.randn(E, H, generator=g) * 0.05
    m = e4b.GptOssExpertsMxfp4.from_float(gu, b1, dn, b2, compute_dtype=torch.float32)
    x = torch.randn(6, H, generator=g)
    val, idx = torch.topk(torch.randn(6, E, generator=g), 2, dim=-1)
    w = torch.softmax(val, -1)
    got = m(x, idx, w).numpy()
    w1 = np.stack([m._dequantize_expert("gate_up", e, torch.float32).numpy() for e in range(E)])
    w2 = np.stack([m._dequantize_expert("down", e, torch.float32).numpy() for e in range(E)])
    want = moe.forward_fp32(x.numpy(), idx.numpy(), w.numpy(), w1, w2, ("gptoss", 1.702, 7.0), b1=b1.numpy(),
                            b2=b2.numpy())
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-5


# ------------------------------------------------------------- kernel descriptor cache


def _nf4_module(E=4, H=128, inter=64, dq=False):
    gu, dn = _weights(E=E, H=H, inter=inter)
    return e4b.Experts4bit.from_float(gu, dn, compute_dtype=torch.bfloat16, compress_statistics=dq)


def test_descriptor_cache_works_for_inference_tensors():
    """Weights built under inference_mode carry no version counter: their descriptors are keyed on
    storage, shape and dtype (cached, no raise), and a replaced tensor rebuilds them."""
    with torch.inference_mode():
        mod = _nf4_module()
    w1, w2 = F._qweights(mod)
    assert w1.struct().n == mod._gate_up_shape[0] and w2.struct().k == mod._down_shape[1]
    assert F._qweights(mod)[0] is w1  # cached: the per-call weight-exponent launches happen once
    with torch.inference_mode():
        mod.gate_up_absmax = mod.gate_up_absmax.clone()
    assert F._qweights(mod)[0] is not w1


def test_descriptor_cache_keeps_the_module_copyable_and_picklable():
    import copy

    mod = _nf4_module()
    w1, w2 = F._qweights(mod)
    w1.struct(), w2.struct()  # what a fused forward builds
    assert F._qweights(mod)[0] is w1  # cached
    clone = copy.deepcopy(mod)
    assert torch.equal(clone.gate_up_proj, mod.gate_up_proj)
    buf = io.BytesIO()
    torch.save(mod, buf)
    assert len(buf.getvalue()) > 0
    # an in-place update (what load_state_dict does) rebuilds the descriptors
    with torch.no_grad():
        mod.gate_up_absmax.mul_(2)
    assert F._qweights(mod)[0] is not w1


def test_evicted_storage_frees_the_cached_weights():
    """Swapping in a 0-element placeholder (offload eviction) and taking the fused forward's
    fallback must not keep the old weight stack alive through the descriptor cache; nor must
    disable_fast."""
    import gc
    import weakref

    mod = _nf4_module()
    F._qweights(mod)[0].struct()
    old = weakref.ref(mod.gate_up_proj)
    mod._e4b_fast_ref = lambda *a: "reference"
    mod.gate_up_proj = torch.nn.Parameter(torch.empty(0, dtype=torch.uint8), requires_grad=False)
    x = torch.randn(2, 128, dtype=torch.bfloat16)
    idx = torch.zeros(2, 2, dtype=torch.long)
    w = torch.ones(2, 2, dtype=torch.bfloat16)
    with torch.no_grad():
        assert F.fused_experts_forward(mod, x, idx, w) == "reference"
    gc.collect()
    assert old() is None
    # disable_fast forgets the descriptors of the modules it walks
    mod2 = _nf4_module()
    F._qweights(mod2)
    old2 = weakref.ref(mod2.down_proj)
    mod2._e4b_fast_ref = mod2.forward
    F.disable_fast(mod2)
    mod2.down_proj = torch.nn.Parameter(torch.empty(0, dtype=torch.uint8), requires_grad=False)
    gc.collect()
    assert old2() is None
