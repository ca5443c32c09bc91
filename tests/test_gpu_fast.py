"""GPU parity of the drop-in ``enable_fast`` path, mirroring the reference's own tests
(``tests/test_fast.py``, ``test_fast_lora.py``, ``test_fast_v4.py``,
``test_fast_expertslora_delegation.py``, ``test_deterministic_scatter.py``) plus the benchmark
configurations (OLMoE, Qwen3 double quant, gpt-oss) at their real shapes.

Accuracy bars: against the fp32 oracle over the same dequantized weights, rel-Frobenius <= 1e-2
and max-abs <= 2e-2 on oracle-RMS-normalised outputs, and no worse than
``max(2 * reference-loop error, 5e-3)`` (the reference's own ordering rule, test_fast.py:82-87).
"""
import numpy as np
import pytest
import torch

import experts4bit_qlora_amd as e4b
from experts4bit_qlora_amd import _native as N
from experts4bit_qlora_amd import fast as F
from experts4bit_qlora_amd import ops
from experts4bit_qlora_amd import quant as Q
from oracle import moe
from oracle import quant as oq
from oracle_weights import oracle_weights

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _announce(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(autouse=True)
def _auto_path():
    F.set_kernel_path("auto")
    yield
    F.set_kernel_path("auto")


def _b_rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-6)).item()


def _make(E=4, H=128, inter=64, k=2, tokens=16, seed=0, has_gate=True, scale=1.0, dq=False):
    torch.manual_seed(seed)
    gate_up = torch.randn(E, 2 * inter if has_gate else inter, H) * scale
    down = torch.randn(E, H, inter) * scale
    mod = e4b.Experts4bit.from_float(gate_up.to(DEV), down.to(DEV), compute_dtype=torch.bfloat16, has_gate=has_gate,
                                     compress_statistics=dq).eval()
    hs = torch.randn(tokens, H, dtype=torch.bfloat16, device=DEV)
    logits = torch.randn(tokens, E, device=DEV)
    top_w, top_i = torch.topk(torch.softmax(logits, -1), k=k, dim=-1)
    return mod, hs, top_i, top_w.to(torch.bfloat16)


def _oracle(mod, hs, top_i, top_w):
    """fp32 forward over the same NF4 values (test_fast.py:49-68), CPU oracle; the weights are
    the module's bytes decoded by the oracle, not by the kernel under test."""
    w1, w2 = oracle_weights(mod)
    epi = "swiglu" if mod.has_gate else "act"
    return moe.forward_fp32(hs.float().cpu().numpy(), top_i.cpu().numpy(), top_w.float().cpu().numpy(), w1, w2, epi)


def _assert_fidelity(fast, ref, oracle, label=""):
    fro, maxabs, brel = moe.rel_errors(fast.float().cpu().numpy(), oracle)
    fro_ref, maxabs_ref, brel_ref = moe.rel_errors(ref.float().cpu().numpy(), oracle)
    g_fast = moe.maxabs_global_rms(fast.float().cpu().numpy(), oracle)
    g_ref = moe.maxabs_global_rms(ref.float().cpu().numpy(), oracle)
    print(f"[fidelity] {label}: fused rel-fro {fro:.2e} max-abs/row-rms {maxabs:.2e} (global rms {g_fast:.2e}) "
          f"max-abs/max {brel:.2e} | reference loop rel-fro {fro_ref:.2e} max-abs/row-rms {maxabs_ref:.2e} "
          f"(global rms {g_ref:.2e}) max-abs/max {brel_ref:.2e}", flush=True)
    assert fro <= 1e-2 and maxabs <= 2e-2, (label, fro, maxabs)
    assert fro <= max(2 * fro_ref, 5e-3), (label, fro, fro_ref)


# ------------------------------------------------------------- test_fast.py equivalents


@pytest.mark.parametrize("path", ["auto", "gemv", "mfma"])
def test_fused_matches_reference(path):
    _announce(f"fused vs reference path={path}")
    F.set_kernel_path(path)
    mod, hs, top_i, top_w = _make()
    with torch.no_grad():
        ref = mod(hs, top_i, top_w)
    assert e4b.enable_fast(mod) == 1
    with torch.no_grad():
        fast = mod(hs, top_i, top_w)
    oracle = _oracle(mod, hs, top_i, top_w)
    assert fast.shape == ref.shape and fast.dtype == ref.dtype
    assert _b_rel(fast, ref) < 1.5e-2
    err_ref = _b_rel(ref, torch.from_numpy(oracle))
    err_fast = _b_rel(fast, torch.from_numpy(oracle))
    assert err_fast <= max(2 * err_ref, 5e-3), (err_fast, err_ref)
    assert e4b.disable_fast(mod) == 1
    with torch.no_grad():
        back = mod(hs, top_i, top_w)
    assert torch.equal(back, ref)


def test_training_path_falls_back_and_backprops():
    _announce("training fallback")
    mod, hs, top_i, top_w = _make()
    e4b.enable_fast(mod)
    x = hs.clone().requires_grad_(True)
    out = mod(x, top_i, top_w)
    out.float().sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    e4b.disable_fast(mod)


def test_skips_ineligible_blocksize():
    mod, *_ = _make()
    mod.blocksize = 128
    assert e4b.enable_fast(mod) == 0


def test_uneven_routing_and_empty_experts():
    _announce("uneven routing")
    mod, hs, top_i, top_w = _make(E=4, k=2, tokens=8, seed=3)
    top_i = torch.stack([torch.zeros(8, dtype=torch.long), torch.ones(8, dtype=torch.long)], 1).to(DEV)
    with torch.no_grad():
        ref = mod(hs, top_i, top_w)
    e4b.enable_fast(mod)
    with torch.no_grad():
        fast = mod(hs, top_i, top_w)
    assert _b_rel(fast, ref) < 1.5e-2
    e4b.disable_fast(mod)


def test_plain_up_projection_has_gate_false():
    _announce("has_gate=False")
    mod, hs, top_i, top_w = _make(has_gate=False, seed=4)
    with torch.no_grad():
        ref = mod(hs, top_i, top_w)
        e4b.enable_fast(mod)
        fast = mod(hs, top_i, top_w)
    _assert_fidelity(fast, ref, _oracle(mod, hs, top_i, top_w))


def test_custom_activation_runs_unfused_epilogue():
    _announce("custom activation")
    mod, hs, top_i, top_w = _make(seed=5)
    mod.act_fn = torch.nn.functional.gelu
    with torch.no_grad():
        ref = mod(hs, top_i, top_w)
        assert e4b.enable_fast(mod) == 1
        fast = mod(hs, top_i, top_w)
    assert _b_rel(fast, ref) < 1.5e-2


def test_fp32_input_dtype_round_trips():
    _announce("fp32 input")
    mod, hs, top_i, top_w = _make(seed=6)
    x = hs.float()
    with torch.no_grad():
        ref = mod(x, top_i, top_w.float())
        e4b.enable_fast(mod)
        fast = mod(x, top_i, top_w.float())
    assert fast.dtype == torch.float32 and _b_rel(fast, ref) < 1.5e-2


def test_fp16_compute_dtype():
    _announce("fp16 compute")
    torch.manual_seed(7)
    gate_up, down = torch.randn(4, 128, 128) * 0.1, torch.randn(4, 128, 64) * 0.1
    mod = e4b.Experts4bit.from_float(gate_up.to(DEV), down.to(DEV), compute_dtype=torch.float16)
    hs = torch.randn(10, 128, dtype=torch.float16, device=DEV)
    top_w, top_i = torch.topk(torch.softmax(torch.randn(10, 4, device=DEV), -1), 2)
    with torch.no_grad():
        ref = mod(hs, top_i, top_w.half())
        e4b.enable_fast(mod)
        fast = mod(hs, top_i, top_w.half())
    assert fast.dtype == torch.float16 and _b_rel(fast, ref) < 1.5e-2


def test_empty_batch():
    mod, hs, top_i, top_w = _make()
    e4b.enable_fast(mod)
    with torch.no_grad():
        out = mod(hs[:0], top_i[:0], top_w[:0])
    assert out.shape == (0, 128)


# --------------------------------------------------------------- determinism & sync-free


def test_forward_is_bit_stable_across_runs():
    _announce("bit-stable x25")
    mod, hs, top_i, top_w = _make(E=8, tokens=64, k=2, seed=8)
    e4b.enable_fast(mod)
    with torch.no_grad():
        first = mod(hs, top_i, top_w)
        for _ in range(25):
            assert torch.equal(first, mod(hs, top_i, top_w))


def test_bare_fused_forward_never_syncs():
    _announce("sync-free decode")
    mod, hs, top_i, top_w = _make(E=8, tokens=1, k=2, seed=9)
    e4b.enable_fast(mod)
    with torch.no_grad():
        mod(hs, top_i, top_w)  # warm the caching allocator
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            mod(hs, top_i, top_w)
        finally:
            torch.cuda.set_sync_debug_mode("default")


def test_weight_descriptor_cache_follows_in_place_updates():
    """The kernel descriptors are cached per module; an in-place update of a weight buffer (what
    load_state_dict does) must reach the next fused forward."""
    _announce("descriptor cache + in-place update")
    mod, hs, top_i, top_w = _make(seed=11)
    e4b.enable_fast(mod)
    with torch.no_grad():
        first = mod(hs, top_i, top_w)
        mod.gate_up_absmax.mul_(2.0)
        mod.down_absmax.mul_(0.5)
        second = mod(hs, top_i, top_w)
        e4b.disable_fast(mod)
        ref = mod(hs, top_i, top_w)
    assert not torch.equal(first, second)
    assert _b_rel(second, ref) < 1.5e-2


# ----------------------------------------------------------------------- ExpertsLoRA


def _lora(seed=0, E=8, H=128, inter=192):
    torch.manual_seed(seed)
    base = e4b.Experts4bit.from_float((torch.randn(E, 2 * inter, H) * 0.1).to(DEV),
                                      (torch.randn(E, H, inter) * 0.1).to(DEV), compute_dtype=torch.bfloat16)
    mod = e4b.ExpertsLoRA(base, r=8, alpha=16, dtype=torch.float32).to(DEV)
    with torch.no_grad():
        for p in (mod.gate_up_lora_B, mod.down_lora_B):
            p.normal_(0, 0.02)
    return mod.eval()


def _lora_inputs(n_tok, E=8, H=128, seed=1):
    torch.manual_seed(seed)
    hs = torch.randn(n_tok, H, dtype=torch.bfloat16, device=DEV)
    idx = torch.randint(0, E, (n_tok, 2), device=DEV)
    wts = torch.rand(n_tok, 2, dtype=torch.bfloat16, device=DEV)
    return hs, idx, wts


@pytest.mark.parametrize("n_tok", [1, 12])
def test_lora_zero_adapter_is_the_bare_fused_forward(n_tok):
    """An untrained adapter (both B zero) contributes exactly nothing: the patched wrapper then
    runs the base's own fused forward (one e4b_moe_forward call), equal to it bit for bit, as
    the reference delegates to an accelerated base (lora.py:181-214). Once the adapter is
    trained (and the cached verdict reset, as train() / a state load do) the LoRA path runs."""
    from experts4bit_qlora_amd import fast as F

    _announce(f"lora zero adapter n_tok={n_tok}")
    mod = _lora()
    with torch.no_grad():
        mod.gate_up_lora_B.zero_()
        mod.down_lora_B.zero_()
    mod._delegate_ok = None
    hs, idx, wts = _lora_inputs(n_tok)
    assert e4b.enable_fast(mod) == 1
    with torch.no_grad():
        got = mod(hs, idx, wts)
        bare = F.fused_experts_forward(mod.base, hs, idx, wts)
        assert torch.equal(got, bare)
        mod.down_lora_B.normal_(0, 0.02)
        mod._delegate_ok = None
        trained = mod(hs, idx, wts)
    assert not torch.equal(trained, bare)


def test_lora_patches_wrapper_and_skips_wrapped_base():
    mod = _lora()
    assert e4b.enable_fast(mod) == 1
    assert hasattr(mod, "_e4b_fast_ref") and not hasattr(mod.base, "_e4b_fast_ref")
    assert e4b.disable_fast(mod) == 1


@pytest.mark.parametrize("n_tok", [1, 12])
def test_lora_fused_matches_reference(n_tok):
    _announce(f"lora n_tok={n_tok}")
    mod = _lora()
    hs, idx, wts = _lora_inputs(n_tok)
    with torch.no_grad():
        ref = mod(hs, idx, wts)
    assert e4b.enable_fast(mod) == 1
    with torch.no_grad():
        got = mod(hs, idx, wts)
    rel = ((got.float() - ref.float()).norm() / ref.float().norm().clamp_min(1e-12)).item()
    assert got.dtype == ref.dtype and rel < 2e-2, rel


def _olmoe_lora(r, adapter_dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    E, H, I = 64, 2048, 1024
    base = e4b.Experts4bit.from_float(torch.randn(E, 2 * I, H, generator=g, device=DEV) * 0.02,
                                      torch.randn(E, H, I, generator=g, device=DEV) * 0.02,
                                      compute_dtype=torch.bfloat16).eval()
    mod = e4b.ExpertsLoRA(base, r=r, alpha=2 * r, dtype=adapter_dtype).to(DEV).eval()
    with torch.no_grad():
        # B ~ N(0, 0.02): the delta is of the order of the base projection, not a rounding error
        for p in (mod.gate_up_lora_B, mod.down_lora_B):
            p.copy_(torch.randn(p.shape, generator=g, device=DEV) * 0.02)
    return mod


@pytest.mark.parametrize("T,r,adt", [(1, 8, torch.bfloat16), (1, 16, torch.float32), (8, 16, torch.bfloat16),
                                     (8, 20, torch.float32), (8, 32, torch.bfloat16), (8, 64, torch.float32),
                                     (64, 8, torch.float32), (64, 16, torch.bfloat16)])
def test_lora_fused_matches_the_lora_oracle_at_olmoe_geometry(T, r, adt):
    """The fused LoRA forward against the fp64 restatement of ExpertsLoRA.forward
    (lora.py:251-256, 329-407) over the oracle-decoded NF4 weights, at the layer bars, and no
    worse than max(2 x the reference loop's own error, 5e-3)."""
    _announce(f"lora vs oracle OLMoE T={T} r={r} adapters={adt}")
    mod = _olmoe_lora(r, adt, seed=7000 + 10 * T + r)
    x, idx, w = _cfg_inputs(T, 64, 2048, 8, seed=7100 + T, renorm=False)
    assert e4b.enable_fast(mod) == 1
    with torch.no_grad():
        got = mod(x, idx, w)
    w1, w2 = oracle_weights(mod.base)
    lo1 = tuple(t.detach().float().cpu().numpy() for t in (mod.gate_up_lora_A, mod.gate_up_lora_B))
    lo2 = tuple(t.detach().float().cpu().numpy() for t in (mod.down_lora_A, mod.down_lora_B))
    xs, ids, ws = x.float().cpu().numpy(), idx.cpu().numpy(), w.float().cpu().numpy()
    want = moe.forward_lora_fp32(xs, ids, ws, w1, w2, lo1, lo2, mod.scaling)
    base_only = moe.forward_fp32(xs, ids, ws, w1, w2)
    delta = np.linalg.norm(want - base_only) / np.linalg.norm(want)
    assert delta > 0.05, delta  # the adapter moves the output well past the bars below
    lt1 = tuple(t.detach().cpu() for t in (mod.gate_up_lora_A, mod.gate_up_lora_B))
    lt2 = tuple(t.detach().cpu() for t in (mod.down_lora_A, mod.down_lora_B))
    ref = moe.reference_lora_loop(x.cpu(), idx.cpu(), w.cpu(), lambda e, dt: torch.from_numpy(w1[e]).to(dt),
                                  lambda e, dt: torch.from_numpy(w2[e]).to(dt), lt1, lt2, mod.scaling,
                                  num_experts=64, compute_dtype=torch.bfloat16)
    _assert_fidelity(got, ref, want, f"lora T={T} r={r} {adt}")


@pytest.mark.parametrize("T,r,adt", [(512, 16, torch.bfloat16), (512, 64, torch.float32), (4096, 16, torch.float32),
                                     (4096, 64, torch.bfloat16), (96, 12, torch.float16), (96, 33, torch.float32),
                                     (600, 24, torch.float16), (600, 40, torch.bfloat16)])
def test_lora_fused_matches_the_lora_oracle_at_prefill_sizes(T, r, adt):
    """The grouped form of the fused LoRA forward -- t = x . A^T on the matrix cores, the GEMM
    tiles' accumulators starting as their deltas; 256-row tiles (half tiles for <= 128 rows) with
    32-row tails from 512 tokens, only 32-row tiles at 96 tokens; ranks that are and are not
    multiples of 8, one and four 16-rank blocks, every adapter dtype -- against the fp64
    restatement of ExpertsLoRA.forward on the first and the last token routed to every expert
    (every expert's first tile and its last), at the layer bars and no worse than the reference
    loop's own error rule (the reference runs this grouped path for every batch,
    fast.py:209-257)."""
    _announce(f"lora vs oracle OLMoE prefill T={T} r={r} adapters={adt}")
    mod = _olmoe_lora(r, adt, seed=7500 + T + r)
    x, idx, w = _cfg_inputs(T, 64, 2048, 8, seed=7600 + T, renorm=False)
    assert e4b.enable_fast(mod) == 1
    with torch.no_grad():
        got = mod(x, idx, w)
    assert torch.isfinite(got).all()
    flat = idx.reshape(-1).cpu().numpy()
    rows = set()
    for e in np.unique(flat):
        hits = np.nonzero(flat == e)[0] // 8
        rows.update([int(hits[0]), int(hits[-1])])
    rows = sorted(rows)
    w1, w2 = oracle_weights(mod.base)
    lo1 = tuple(t.detach().float().cpu().numpy() for t in (mod.gate_up_lora_A, mod.gate_up_lora_B))
    lo2 = tuple(t.detach().float().cpu().numpy() for t in (mod.down_lora_A, mod.down_lora_B))
    xs, ids, ws = x[rows].float().cpu().numpy(), idx[rows].cpu().numpy(), w[rows].float().cpu().numpy()
    want = moe.forward_lora_fp32(xs, ids, ws, w1, w2, lo1, lo2, mod.scaling)
    delta = np.linalg.norm(want - moe.forward_fp32(xs, ids, ws, w1, w2)) / np.linalg.norm(want)
    assert delta > 0.05, delta
    lt1 = tuple(t.detach().cpu() for t in (mod.gate_up_lora_A, mod.gate_up_lora_B))
    lt2 = tuple(t.detach().cpu() for t in (mod.down_lora_A, mod.down_lora_B))
    ref = moe.reference_lora_loop(x[rows].cpu(), idx[rows].cpu(), w[rows].cpu(),
                                  lambda e, dt: torch.from_numpy(w1[e]).to(dt),
                                  lambda e, dt: torch.from_numpy(w2[e]).to(dt), lt1, lt2, mod.scaling,
                                  num_experts=64, compute_dtype=torch.bfloat16)
    _assert_fidelity(got[rows], ref, want, f"lora prefill T={T} r={r} {adt} on {len(rows)} tokens")


def test_lora_fused_forward_never_syncs():
    """The LoRA deltas of every expert group are added on the device (e4b_lora_delta), so the
    fused LoRA forward needs no group sizes on the host: no device synchronisation at all
    (the reference slices its groups after a .tolist(), fast.py:209-216)."""
    _announce("lora sync-free")
    mod = _lora()
    hs, idx, wts = _lora_inputs(12)
    assert e4b.enable_fast(mod) == 1
    with torch.no_grad():
        mod(hs, idx, wts)  # warm the caching allocator
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            mod(hs, idx, wts)
        finally:
            torch.cuda.set_sync_debug_mode("default")


def test_lora_training_and_grad_fall_back_exactly():
    _announce("lora fallback")
    mod = _lora()
    hs, idx, wts = _lora_inputs(12)
    mod.train()
    with torch.no_grad():
        ref_train = mod(hs, idx, wts)
    mod.eval()
    e4b.enable_fast(mod)
    mod.train()
    with torch.no_grad():
        got = mod(hs, idx, wts)
    assert torch.equal(got, ref_train)
    mod.eval()
    hs_g = hs.clone().requires_grad_(True)
    out = mod(hs_g, idx, wts)
    assert out.requires_grad
    out.float().sum().backward()
    assert hs_g.grad is not None


def test_lora_evicted_placeholder_falls_back_and_raises():
    mod = _lora()
    e4b.enable_fast(mod)
    hs, idx, wts = _lora_inputs(4)
    real = mod.base.gate_up_proj
    try:
        mod.base.gate_up_proj = torch.nn.Parameter(torch.empty(0, dtype=real.dtype, device=real.device),
                                                   requires_grad=False)
        with pytest.raises(Exception):
            with torch.no_grad():
                mod(hs, idx, wts)
    finally:
        mod.base.gate_up_proj = real


def test_zero_adapter_delegates_to_patched_base():
    _announce("lora delegation")
    torch.manual_seed(0)
    base = e4b.Experts4bit.from_float(torch.randn(4, 128, 128).to(DEV), torch.randn(4, 128, 64).to(DEV),
                                      compute_dtype=torch.bfloat16)
    mod = e4b.ExpertsLoRA(base, r=4, alpha=8).to(DEV).eval()
    x, idx, w = _lora_inputs(8, E=4)
    with torch.no_grad():
        ref = mod(x, idx, w).float().cpu()
    calls = {"n": 0}
    orig = F.fused_experts_forward

    def counting(*a, **kw):
        calls["n"] += 1
        return orig(*a, **kw)

    F.fused_experts_forward = counting
    try:
        assert e4b.enable_fast(mod.base) == 1
        with torch.no_grad():
            got = mod(x, idx, w).float().cpu()
        assert calls["n"] > 0
        assert not torch.equal(ref, got)
        assert ((ref - got).abs().max() / got.abs().max().clamp_min(1e-3)) < 5e-2
    finally:
        F.fused_experts_forward = orig
        e4b.disable_fast(mod.base)


# ---------------------------------------------------------------- DeepSeek-V4 clamps


def _v4(limit, seed, lora=False):
    from experts4bit_qlora_amd.arch.deepseek_v4 import _DeepseekV4ForwardMixin

    g = torch.Generator().manual_seed(seed)
    E, H, INTER, K, T = 8, 128, 64, 3, 24
    base = _DeepseekV4ForwardMixin.from_deepseek_v4(torch.randn(E, 2 * INTER, H, generator=g) * 0.35,
                                                    torch.randn(E, H, INTER, generator=g) * 0.35, limit=limit,
                                                    compute_dtype=torch.bfloat16).to(DEV).eval()
    mod = e4b.ExpertsLoRA(base, r=8, alpha=16, dtype=torch.bfloat16).to(DEV).eval() if lora else base
    x = (torch.randn(T, H, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    val, idx = torch.topk(torch.randn(T, E, generator=g), K, dim=-1)
    return mod, x, idx.to(DEV), torch.softmax(val, dim=-1).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("lora", [False, True])
def test_v4_fused_keeps_the_clamps(lora):
    _announce(f"v4 clamps lora={lora}")
    TOL = 1.5e-2
    mod, x, idx, w = _v4(2.0, seed=6, lora=lora)
    unclamped, *_ = _v4(0.0, seed=6, lora=lora)
    with torch.no_grad():
        ref = mod(x, idx, w)
        ref_noclamp = unclamped(x, idx, w)
        assert _b_rel(ref, ref_noclamp) > 10 * TOL
        assert e4b.enable_fast(mod) == 1
        got = mod(x, idx, w)
    assert _b_rel(got, ref) < TOL, _b_rel(got, ref)
    assert _b_rel(got, ref_noclamp) > 10 * TOL
    e4b.disable_fast(mod)


@pytest.mark.parametrize("T", [24, 96])
def test_v4_clamped_layer_matches_the_oracle(T):
    """DeepSeek-V4's clamped SwiGLU through the fused path against the fp32 oracle with the same
    clamp (``forward_fp32(..., ("clamp_swiglu", L))``, ref tests/test_fast_v4.py:73-104), on
    weights and activations large enough that the clamp changes most gate and up values; T=24
    runs the decode / GEMV kernels, T=96 the matrix-core ones. A negative control: the unclamped
    oracle is far from the result."""
    _announce(f"v4 clamped layer vs oracle T={T}")
    from experts4bit_qlora_amd.arch.deepseek_v4 import _DeepseekV4ForwardMixin

    E, H, INTER, K, L = 16, 256, 128, 4, 2.0
    g = torch.Generator().manual_seed(60 + T)
    mod = _DeepseekV4ForwardMixin.from_deepseek_v4(torch.randn(E, 2 * INTER, H, generator=g) * 0.35,
                                                   torch.randn(E, H, INTER, generator=g) * 0.35, limit=L,
                                                   compute_dtype=torch.bfloat16).to(DEV).eval()
    x = (torch.randn(T, H, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    val, idx = torch.topk(torch.randn(T, E, generator=g), K, dim=-1)
    idx, w = idx.to(DEV), torch.softmax(val, dim=-1).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        ref = mod(x, idx, w)
        assert e4b.enable_fast(mod) == 1
        got = mod(x, idx, w)
    ow1, ow2 = oracle_weights(mod)
    args = (x.float().cpu().numpy(), idx.cpu().numpy(), w.float().cpu().numpy(), ow1, ow2)
    oracle = moe.forward_fp32(*args, ("clamp_swiglu", L))
    _assert_fidelity(got, ref, oracle, f"v4 clamp T={T}")
    fro_nc, _, _ = moe.rel_errors(got.float().cpu().numpy(), moe.forward_fp32(*args, ("clamp_swiglu", 0.0)))
    assert fro_nc > 0.1, fro_nc  # the clamp is active and the result follows it
    e4b.disable_fast(mod)


def test_gptoss_nf4_stays_skipped():
    from experts4bit_qlora_amd.arch.gptoss import GptOssExperts4bit

    g = torch.Generator().manual_seed(3)
    E, H, INTER = 8, 128, 64
    base = GptOssExperts4bit.from_gptoss(torch.randn(E, H, 2 * INTER, generator=g) * 0.1,
                                         torch.randn(E, 2 * INTER, generator=g) * 0.05,
                                         torch.randn(E, INTER, H, generator=g) * 0.1,
                                         torch.randn(E, H, generator=g) * 0.05).to(DEV)
    assert e4b.enable_fast(base) == 0
    mod = e4b.ExpertsLoRA(base, r=8, alpha=16, dtype=torch.bfloat16).to(DEV).eval()
    assert e4b.enable_fast(mod) == 0


# ---------------------------------------------------------------------- gpt-oss MXFP4


@pytest.mark.parametrize("T", [1, 7, 80])
def test_gptoss_mxfp4_fused_matches_reference_and_oracle(T):
    _announce(f"gpt-oss mxfp4 T={T}")
    g = torch.Generator().manual_seed(T)
    E, H, I, k = 8, 256, 128, 4
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.05
    dn = torch.randn(E, H, I, generator=g) * 0.05
    b1 = torch.randn(E, 2 * I, generator=g) * 0.05
    b2 = torch.randn(E, H, generator=g) * 0.05
    mod = e4b.GptOssExpertsMxfp4.from_float(gu.to(DEV), b1.to(DEV), dn.to(DEV), b2.to(DEV)).eval()
    x = (torch.randn(T, H, generator=g) * 2).to(torch.bfloat16).to(DEV)
    val, idx = torch.topk(torch.randn(T, E, generator=g), k, dim=-1)
    w = torch.softmax(val, -1).to(torch.bfloat16).to(DEV)
    idx = idx.to(DEV)
    with torch.no_grad():
        ref = mod(x, idx, w)
        assert e4b.enable_fast(mod) == 1
        got = mod(x, idx, w)
    w1, w2 = oracle_weights(mod)
    oracle = moe.forward_fp32(x.float().cpu().numpy(), idx.cpu().numpy(), w.float().cpu().numpy(), w1, w2,
                              ("gptoss", 1.702, 7.0), b1=mod.gate_up_bias.float().cpu().numpy(),
                              b2=mod.down_bias.float().cpu().numpy())
    _assert_fidelity(got, ref, oracle, f"gptoss T={T}")


@pytest.mark.parametrize("sizes", [[1, 1, 1], [6, 0, 9, 1]])
def test_gemm_mxfp4_grouped_drop_in(sizes):
    """ops.gemm_mxfp4_grouped keeps mxfp4_grouped.gemm_mxfp4_grouped's call shape
    (nvme_experts.py:852-865): a[M, K] rows grouped by expert, blocks [E, N, K/2], scales
    [E, N, K/32]; checked against the oracle-decoded weights per group, for the all-size-1 (GEMV)
    and mixed (GEMM) cases the reference distinguishes (test_mxfp4_arena_train.py:669-673)."""
    _announce(f"gemm_mxfp4_grouped sizes={sizes}")
    g = torch.Generator().manual_seed(len(sizes))
    E, N, K = 4, 96, 256
    blocks = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.uint8)
    scales = torch.randint(118, 130, (E, N, K // 32), generator=g, dtype=torch.uint8)
    ids = [e for e, n_e in enumerate(sizes) if n_e > 0]  # one group per expert, ascending
    sz = [n_e for n_e in sizes if n_e > 0]
    M = sum(sz)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    got = ops.gemm_mxfp4_grouped(a.to(DEV), blocks.to(DEV), scales.to(DEV), sz, ids).float().cpu().numpy()
    from oracle import c_oracle

    want = np.zeros((M, N), np.float64)
    r0 = 0
    for e, n_e in zip(ids, sz):
        wdense = c_oracle.dequant_mxfp4(blocks[e].numpy(), scales[e].numpy(), N, K).astype(np.float64)
        want[r0:r0 + n_e] = a[r0:r0 + n_e].double().numpy() @ wdense.T
        r0 += n_e
    rel = np.abs(got - want).max() / np.abs(want).max()
    assert rel < 2e-2, rel  # the reference's kernel bar (test_mxfp4_arena_train.py:704-722)


def test_mxfp4_checkpoint_layout_is_deinterleaved_losslessly():
    g = torch.Generator().manual_seed(0)
    E, H, I = 2, 64, 64
    gb = torch.randint(0, 256, (E, 2 * I, H // 32, 16), generator=g, dtype=torch.uint8)
    gs = torch.randint(110, 140, (E, 2 * I, H // 32), generator=g, dtype=torch.uint8)
    db = torch.randint(0, 256, (E, H, I // 32, 16), generator=g, dtype=torch.uint8)
    ds = torch.randint(110, 140, (E, H, I // 32), generator=g, dtype=torch.uint8)
    b1, b2 = torch.randn(E, 2 * I, generator=g), torch.randn(E, H, generator=g)
    mod = e4b.GptOssExpertsMxfp4.from_gptoss_mxfp4(gb.to(DEV), gs.to(DEV), b1.to(DEV), db.to(DEV), ds.to(DEV),
                                                   b2.to(DEV))
    dense = e4b.dequantize_mxfp4(gb.to(DEV), gs.to(DEV), dtype=torch.float32)  # [E, H, 2I] interleaved
    for e in range(E):
        w = mod._dequantize_expert("gate_up", e, torch.float32)
        assert torch.equal(w[:I], dense[e].T[0::2]) and torch.equal(w[I:], dense[e].T[1::2])


def test_reference_format_checkpoint_through_the_fused_path():
    """The reference-format state_dict fixture (tests/golden/make_checkpoint.py: the on-disk
    format of _vendor/experts.py:236-327 built from its definition) loaded on the device and run
    through enable_fast: the fused forward against the fixture's fp64 expectation at the layer
    bars (rel-Frobenius <= 1e-2, max-abs <= 2e-2 per row RMS)."""
    import os

    _announce("reference-format checkpoint, fused")
    d = torch.load(os.path.join(os.path.dirname(__file__), "golden", "expertsnbit_nf4_checkpoint.pt"),
                   weights_only=True)
    m = e4b.Experts4bit(4, 128, 64, quant_type="nf4", compute_dtype=torch.bfloat16, device=DEV).eval()
    m.load_state_dict({k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in d["state_dict"].items()},
                      strict=True)
    assert e4b.enable_fast(m) == 1
    with torch.no_grad():
        got = m(d["x"].to(DEV), d["top_k_index"].to(DEV), d["top_k_weights"].to(DEV))
    fro, maxabs, _ = moe.rel_errors(got.float().cpu().numpy(), d["expected"].numpy())
    assert fro <= 1e-2 and maxabs <= 2e-2, (fro, maxabs)


@pytest.mark.parametrize("T", [1, 37])
def test_gptoss_release_layout_matches_transformers(T):
    """gpt-oss experts from tensors in the released checkpoint layout (gate/up rows interleaved,
    blocks [E, 2I, H/32, 16], e8m0 scales, interleaved biases), loaded by from_gptoss_mxfp4 and run
    through enable_fast, against transformers' own GptOssExperts (modeling_gpt_oss.py) built
    from the same tensors by transformers' convert_moe_packed_tensors, in fp32 on the CPU. Pins
    the de-interleave, transposes, bias order and clamped GLU against third-party code."""
    from transformers import GptOssConfig
    from transformers.integrations.mxfp4 import convert_moe_packed_tensors
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts

    _announce(f"gpt-oss release layout vs transformers T={T}")
    E, H, I, k = 8, 256, 128, 4
    g = torch.Generator().manual_seed(31 + T)
    gb = torch.randint(0, 256, (E, 2 * I, H // 32, 16), generator=g, dtype=torch.uint8)
    gs = torch.randint(118, 124, (E, 2 * I, H // 32), generator=g, dtype=torch.uint8)
    db = torch.randint(0, 256, (E, H, I // 32, 16), generator=g, dtype=torch.uint8)
    ds = torch.randint(118, 124, (E, H, I // 32), generator=g, dtype=torch.uint8)
    b1 = torch.randn(E, 2 * I, generator=g) * 0.1
    b2 = torch.randn(E, H, generator=g) * 0.1
    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=k)
    ref = GptOssExperts(cfg)
    with torch.no_grad():
        ref.gate_up_proj.copy_(convert_moe_packed_tensors(gb.clone(), gs.clone(), dtype=torch.float32))
        ref.down_proj.copy_(convert_moe_packed_tensors(db.clone(), ds.clone(), dtype=torch.float32))
        ref.gate_up_proj_bias.copy_(b1)
        ref.down_proj_bias.copy_(b2)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    top, idx = torch.topk(logits, k, dim=-1)
    w = torch.softmax(top, -1).to(torch.bfloat16)  # gpt-oss: top-4 of the logits, then softmax
    with torch.no_grad():
        want = ref(x.float(), router_indices=idx, routing_weights=w.float()).double().numpy()
    mod = e4b.GptOssExpertsMxfp4.from_gptoss_mxfp4(gb.to(DEV), gs.to(DEV), b1.to(DEV), db.to(DEV), ds.to(DEV),
                                                   b2.to(DEV)).eval()
    with torch.no_grad():
        loop = mod(x.to(DEV), idx.to(DEV), w.to(DEV))  # the module's own per-expert loop (compute dtype)
    assert e4b.enable_fast(mod) == 1
    with torch.no_grad():
        got = mod(x.to(DEV), idx.to(DEV), w.to(DEV))
    fro, maxabs, _ = moe.rel_errors(got.float().cpu().numpy(), want)
    fro_l, maxabs_l, _ = moe.rel_errors(loop.float().cpu().numpy(), want)
    print(f"[fidelity] gpt-oss release layout T={T}: fused rel-fro {fro:.2e} max-abs/row-rms {maxabs:.2e} | "
          f"loop {fro_l:.2e} / {maxabs_l:.2e}", flush=True)
    # the bf16 loop itself lands near 3.5e-2 max-abs on these outputs (up to ~7 in magnitude)
    assert fro <= 1e-2 and maxabs <= max(2e-2, 2 * maxabs_l), (fro, maxabs, maxabs_l)


# ---------------------------------------------------------- benchmark-shaped parity


def _cfg_module(E, H, I, seed, dq):
    g = torch.Generator(device=DEV).manual_seed(seed)
    gu = torch.randn(E, 2 * I, H, generator=g, device=DEV) * 0.02
    dn = torch.randn(E, H, I, generator=g, device=DEV) * 0.02
    return e4b.Experts4bit.from_float(gu, dn, compute_dtype=torch.bfloat16, compress_statistics=dq).eval()


def _cfg_inputs(T, E, H, k, seed, renorm):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, H, generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g, device=DEV)
    w, idx = torch.topk(torch.softmax(logits, -1), k, dim=-1)
    if renorm:
        w = w / w.sum(-1, keepdim=True)
    return x, idx, w.to(torch.bfloat16)


def _oracle_rows(mod, x, idx, w, rows):
    """CPU fp64 oracle on a subset of tokens; only the experts those tokens hit are decoded, by the
    oracle's C restatement from the module's stored bytes (never by the kernel under test)."""
    sub_idx = idx[rows].cpu().numpy()
    w1, w2 = oracle_weights(mod)
    return moe.forward_fp32(x[rows].float().cpu().numpy(), sub_idx, w[rows].float().cpu().numpy(), w1, w2)


@pytest.mark.parametrize("cfg,T", [("olmoe", 1), ("olmoe", 8), ("olmoe", 64), ("qwen3_dq", 1), ("qwen3_dq", 32),
                                   ("qwen3_dq", 256)])
def test_baseline_configs_decode(cfg, T):
    _announce(f"baseline config {cfg} T={T}")
    if cfg == "olmoe":
        E, H, I, k, dq, renorm = 64, 2048, 1024, 8, False, False
    else:
        E, H, I, k, dq, renorm = 128, 2048, 768, 8, True, True
    mod = _cfg_module(E, H, I, seed=1000 + T, dq=dq)
    x, idx, w = _cfg_inputs(T, E, H, k, seed=2000 + T, renorm=renorm)
    with torch.no_grad():
        ref = mod(x, idx, w)
        assert e4b.enable_fast(mod) == 1
        got = mod(x, idx, w)
    # every token up to 64; beyond that 64 tokens spread over the batch
    rows = list(range(T)) if T <= 64 else sorted(set(np.linspace(0, T - 1, 64).astype(int).tolist()))
    oracle = _oracle_rows(mod, x, idx, w, rows)
    _assert_fidelity(got[rows], ref[rows], oracle, f"{cfg} T={T}")


def test_qwen3_zipf_prefill_4096():
    _announce("qwen3 zipf prefill 4096")
    E, H, I, k, T = 128, 2048, 768, 8, 4096
    mod = _cfg_module(E, H, I, seed=3000, dq=True)
    g = torch.Generator(device=DEV).manual_seed(3001)
    x = torch.randn(T, H, generator=g, device=DEV).to(torch.bfloat16)
    rank = torch.randperm(E, generator=torch.Generator().manual_seed(3002)).to(DEV) + 1
    logits = torch.randn(T, E, generator=g, device=DEV) - 1.1 * torch.log(rank.float())
    w, idx = torch.topk(torch.softmax(logits, -1), k, dim=-1)
    w = (w / w.sum(-1, keepdim=True)).to(torch.bfloat16)
    e4b.enable_fast(mod)
    with torch.no_grad():
        got = mod(x, idx, w)
    assert torch.isfinite(got).all()
    # the first and the last token routed to every active expert: every expert's first tile and
    # its last (the 32-row tail tiles of the split tiling included) is checked
    flat = idx.reshape(-1).cpu().numpy()
    rows = set()
    for e in np.unique(flat):
        hits = np.nonzero(flat == e)[0] // k
        rows.update([int(hits[0]), int(hits[-1])])
    rows = sorted(rows)
    _announce(f"qwen3 prefill oracle on {len(rows)} tokens covering {len(np.unique(flat))} experts")
    oracle = _oracle_rows(mod, x, idx, w, rows)
    fro, maxabs, brel = moe.rel_errors(got[rows].float().cpu().numpy(), oracle)
    g_rms = moe.maxabs_global_rms(got[rows].float().cpu().numpy(), oracle)
    print(f"[fidelity] qwen3 prefill: rel-fro {fro:.2e} max-abs/row-rms {maxabs:.2e} (global rms {g_rms:.2e}) "
          f"max-abs/max {brel:.2e}", flush=True)
    assert fro <= 1e-2 and maxabs <= 2e-2, (fro, maxabs)
    # the GEMV and MFMA families agree on the same prefill (size-independent cross-check)
    F.set_kernel_path("gemv")
    with torch.no_grad():
        got_gemv = mod(x[:512], idx[:512], w[:512])
    F.set_kernel_path("mfma")
    with torch.no_grad():
        got_mfma = mod(x[:512], idx[:512], w[:512])
    fro2, _, _ = moe.rel_errors(got_gemv.float().cpu().numpy(), got_mfma.float().cpu().numpy())
    assert fro2 <= 1e-2


@pytest.mark.parametrize("T", [1, 2048])
def test_gptoss_config_shapes(T):
    _announce(f"gpt-oss config T={T}")
    E, H, I, k = 32, 2880, 2880, 4
    g = torch.Generator(device=DEV).manual_seed(4000 + T)
    gu = torch.randn(E, 2 * I, H, generator=g, device=DEV) * 0.02
    dn = torch.randn(E, H, I, generator=g, device=DEV) * 0.02
    b1 = torch.randn(E, 2 * I, generator=g, device=DEV) * 0.02
    b2 = torch.randn(E, H, generator=g, device=DEV) * 0.02
    mod = e4b.GptOssExpertsMxfp4.from_float(gu, b1, dn, b2).eval()
    del gu, dn
    x = torch.randn(T, H, generator=g, device=DEV).to(torch.bfloat16)
    val, idx = torch.topk(torch.randn(T, E, generator=g, device=DEV), k, dim=-1)
    w = torch.softmax(val, -1).to(torch.bfloat16)
    e4b.enable_fast(mod)
    # tokens 0-3, plus at T=2048 the first and the last token routed to every expert: every
    # expert's first 128-row tile and its last tile (partial 128-row tiles and the 32-row tail
    # tiles included) is compared with the oracle (ref tests/test_mxfp4_arena_train.py:663-722)
    rows = set(range(min(T, 4)))
    if T > 4:
        flat = idx.reshape(-1).cpu().numpy()
        for e in np.unique(flat):
            hits = np.nonzero(flat == e)[0] // k
            rows.update([int(hits[0]), int(hits[-1])])
    rows = sorted(rows)
    _announce(f"gpt-oss T={T}: oracle on {len(rows)} tokens")
    with torch.no_grad():
        got = mod(x, idx, w)
        ref = mod._e4b_fast_ref(x[rows], idx[rows], w[rows])
    sub = idx[rows].cpu().numpy()
    w1, w2 = oracle_weights(mod)
    oracle = moe.forward_fp32(x[rows].float().cpu().numpy(), sub, w[rows].float().cpu().numpy(), w1, w2,
                              ("gptoss", 1.702, 7.0), b1=mod.gate_up_bias.float().cpu().numpy(),
                              b2=mod.down_bias.float().cpu().numpy())
    _assert_fidelity(got[rows], ref, oracle, f"gptoss T={T}")


@pytest.mark.parametrize("T", [2, 8, 64])
def test_decode_path_forced_up_to_its_row_limit(T):
    """The GEMV kernels forced: the two-launch decode path (wave-local routing, combine fused into
    down) up to its 64-row limit (T=8, k=8), and beyond it (T=64) the grouped GEMV kernels after
    one routing launch -- batches the automatic rule sends to MFMA."""
    _announce(f"decode path forced T={T}")
    E, H, I, k = 64, 2048, 1024, 8
    mod = _cfg_module(E, H, I, seed=5000 + T, dq=False)
    x, idx, w = _cfg_inputs(T, E, H, k, seed=5100 + T, renorm=False)
    with torch.no_grad():
        ref = mod(x, idx, w)
        e4b.enable_fast(mod)
        F.set_kernel_path("gemv")
        got = mod(x, idx, w)
        F.set_kernel_path("mfma")
        got_mfma = mod(x, idx, w)
    rows = list(range(min(T, 6)))
    _assert_fidelity(got[rows], ref[rows], _oracle_rows(mod, x, idx, w, rows), f"decode forced T={T}")
    fro, _, _ = moe.rel_errors(got.float().cpu().numpy(), got_mfma.float().cpu().numpy())
    assert fro <= 1e-2


@pytest.mark.parametrize("xscale,wscale,dq", [(2.0 ** 20, 1.0, False), (2.0 ** -20, 1.0, False),
                                              (1.0, 2.0 ** -24, False), (1.0, 2.0 ** 12, True), (2.0 ** -8, 2.0 ** 8, True)])
def test_fp16_matrix_core_mode_keeps_the_bf16_range(xscale, wscale, dq):
    """The MFMA path (T=32) runs fp16 operands under power-of-two row and expert scales: with
    activations and weights far outside fp16's own range the layer still meets the bars against
    the oracle (an unscaled fp16 operand would overflow to inf or flush to zero here)."""
    _announce(f"fp16 mode range xscale={xscale} wscale={wscale} dq={dq}")
    E, H, I, k, T = 16, 256, 128, 4, 32
    g = torch.Generator().manual_seed(int(abs(np.log2(xscale * wscale))) + 17)
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.05 * wscale
    dn = torch.randn(E, H, I, generator=g) * 0.05 * wscale
    mod = e4b.Experts4bit.from_float(gu.to(DEV), dn.to(DEV), compute_dtype=torch.bfloat16,
                                     compress_statistics=dq).eval()
    x = (torch.randn(T, H, generator=g) * xscale).to(torch.bfloat16).to(DEV)
    val, idx = torch.topk(torch.randn(T, E, generator=g), k, dim=-1)
    w = torch.softmax(val, -1).to(torch.bfloat16).to(DEV)
    idx = idx.to(DEV)
    with torch.no_grad():
        ref = mod(x, idx, w)
        assert e4b.enable_fast(mod) == 1
        got = mod(x, idx, w)
        w1, w2 = F._qweights(mod)
        assert w1.shift is not None and w2.shift is not None  # the fp16 mode ran
    assert torch.isfinite(got).all()
    _assert_fidelity(got, ref, _oracle(mod, x, idx, w), f"fp16 mode x*{xscale} w*{wscale} dq={dq}")


@pytest.mark.parametrize("xscale,wscale,dq,outlier", [(2.0 ** 20, 1.0, False, False), (2.0 ** -20, 1.0, True, False),
                                                      (1.0, 2.0 ** -24, False, False), (1.0, 2.0 ** 12, True, False),
                                                      (1.0, 1.0, False, True)])
def test_prefill_fp16_down_rows_keep_the_range(xscale, wscale, dq, outlier):
    """At prefill sizes (256-row and 32-row tiles) with the down K a multiple of 256, the fp16 mode
    stores the down rows as fp16 with the operand scales left on, times 2^-(16 + ceil(log2 K)), and
    the combine folds the scales into the router weights. With activations and weights far outside
    fp16's own range, or a token column 2^12 above the others (h rows dominated by one value), the
    layer still meets the bars against the oracle on the first and last token of every expert."""
    _announce(f"prefill fp16 down rows x*{xscale} w*{wscale} dq={dq} outlier={outlier}")
    E, H, I, k, T = 16, 512, 256, 4, 512
    g = torch.Generator().manual_seed(int(abs(np.log2(xscale * wscale))) + 23 + outlier)
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.05 * wscale
    dn = torch.randn(E, H, I, generator=g) * 0.05 * wscale
    mod = e4b.Experts4bit.from_float(gu.to(DEV), dn.to(DEV), compute_dtype=torch.bfloat16,
                                     compress_statistics=dq).eval()
    del gu, dn
    x = torch.randn(T, H, generator=g) * xscale
    if outlier:
        x[:, 7] *= 2.0 ** 12
    x = x.to(torch.bfloat16).to(DEV)
    # Zipf-skewed routing: head experts fill 256-row tiles, tail experts end in 32-row tiles
    rank = torch.randperm(E, generator=g).float() + 1.0
    val, idx = torch.topk(torch.randn(T, E, generator=g) - 1.1 * torch.log(rank), k, dim=-1)
    w = torch.softmax(val, -1).to(torch.bfloat16).to(DEV)
    idx = idx.to(DEV)
    with torch.no_grad():
        assert e4b.enable_fast(mod) == 1
        got = mod(x, idx, w)
        w1, w2 = F._qweights(mod)
        assert w1.shift is not None and w2.shift is not None  # the fp16 mode ran
    assert torch.isfinite(got).all()
    flat = idx.reshape(-1).cpu().numpy()
    assert np.bincount(flat, minlength=E).max() > 256  # a full 256-row tile
    rows = set()
    for e in np.unique(flat):
        hits = np.nonzero(flat == e)[0] // k
        rows.update([int(hits[0]), int(hits[-1])])
    rows = sorted(rows)
    oracle = _oracle_rows(mod, x, idx, w, rows)
    fro, maxabs, brel = moe.rel_errors(got[rows].float().cpu().numpy(), oracle)
    print(f"[fidelity] prefill fp16 down rows x*{xscale} w*{wscale} dq={dq} outlier={outlier}: rel-fro {fro:.2e} "
          f"max-abs/row-rms {maxabs:.2e} max-abs/max {brel:.2e}", flush=True)
    assert fro <= 1e-2 and maxabs <= 2e-2, (fro, maxabs)


@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float16, torch.float32])
def test_prefill_combine_output_and_weight_dtypes(wdt):
    """The combine of the prefill's fp16 down rows sums in fp32 and rounds once: the bf16 and fp16
    outputs equal the fp32 output rounded, bit for bit, for router weights in bf16, fp16 and fp32
    (the power of two each slot's weight takes on is exact in all three)."""
    _announce(f"prefill combine dtypes wdt={wdt}")
    g = torch.Generator().manual_seed(61)
    E, H, I, k, T = 8, 512, 256, 2, 512
    qw = []
    for n, kk in ((2 * I, H), (H, I)):
        packed, absmax = Q.quantize_4bit(torch.randn(E, n * kk, generator=g) * 0.05)
        qw.append(ops.with_weight_shift(ops.nf4_qweight(packed.to(DEV), absmax.to(DEV),
                                                        Q.code_4bit("nf4").to(DEV), n, kk, num_experts=E)))
    w1, w2 = qw
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    rank = torch.randperm(E, generator=g).float() + 1.0
    val, idx = torch.topk(torch.randn(T, E, generator=g) - 1.1 * torch.log(rank), k, dim=-1)
    w = torch.softmax(val, -1).to(wdt).to(DEV)
    idx = idx.to(DEV)
    ref = ops.moe_forward(x, idx, w, w1, w2, N.EPI_SWIGLU, torch.float32)
    for odt in (torch.bfloat16, torch.float16):
        got = ops.moe_forward(x, idx, w, w1, w2, N.EPI_SWIGLU, odt)
        assert torch.equal(got, ref.to(odt)), (wdt, odt)
    assert torch.isfinite(ref).all()


@pytest.mark.parametrize("H,I,dq", [(1024, 192, False), (384, 256, True), (1280, 512, False), (1792, 640, True)])
def test_narrow_tiles_in_fp16_mode(H, I, dq):
    """32-row tiles in the fp16 mode with K a multiple of 256 (the narrow kernel: pairs of 128-deep
    steps, the weight bytes decoded in the MFMA operand layout): 2 to 14 steps (the loop's six-step
    passes and its two- and four-step tails), partial column tiles (n_out 192 and 384 against 128
    gated / 256 plain columns per tile), experts with more than one 32-row tile, NF4 and double
    quantization; the GEMMs whose K is not a multiple of 256 (192, 384, 640) take the 32-row MFMA
    kernel in the same forward."""
    _announce(f"narrow tiles H={H} I={I} dq={dq}")
    E, k, T = 16, 4, 48
    g = torch.Generator().manual_seed(H + I + dq)
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.05
    dn = torch.randn(E, H, I, generator=g) * 0.05
    mod = e4b.Experts4bit.from_float(gu.to(DEV), dn.to(DEV), compute_dtype=torch.bfloat16,
                                     compress_statistics=dq).eval()
    del gu, dn
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    # a skewed routing: expert 0 in every token (48 rows: two tiles), the rest spread
    scores = torch.randn(T, E, generator=g)
    scores[:, 0] += 100.0
    val, idx = torch.topk(scores, k, dim=-1)
    w = torch.softmax(val - val[:, :1], -1).to(torch.bfloat16).to(DEV)
    idx = idx.to(DEV)
    with torch.no_grad():
        ref = mod(x, idx, w)
        assert e4b.enable_fast(mod) == 1
        got = mod(x, idx, w)
        w1, w2 = F._qweights(mod)
        assert w1.shift is not None and w2.shift is not None  # the fp16 mode ran
    assert torch.isfinite(got).all()
    _assert_fidelity(got, ref, _oracle(mod, x, idx, w), f"narrow tiles H={H} I={I} dq={dq}")


@pytest.mark.parametrize("H,inter", [(128, 64), (1024, 320)])
def test_weight_shift_matches_the_oracle_exponents(H, inter):
    """e4b_weight_shift: 141 - max(E, 20), E the largest biased exponent of each expert's block
    scales (decoded ones for double quantization), from the oracle's decode of the same bytes.
    At H=1024 the gate_up projection has 10,240 block scales per expert, three blocks of the
    kernel's grid, and each expert's largest scale is planted in a different one (its first,
    middle or last row). Decode-sized calls never compute the exponents."""
    _announce(f"weight shift H={H} inter={inter}")
    E = 6
    for dq in (False, True):
        torch.manual_seed(20 + dq)
        gu = torch.randn(E, 2 * inter, H) * 0.05
        for e in range(E):
            gu[e, (0, inter, 2 * inter - 1)[e % 3]] *= 2.0 ** (1 + e)
        dn = torch.randn(E, H, inter) * 0.05
        mod = e4b.Experts4bit.from_float(gu.to(DEV), dn.to(DEV), compute_dtype=torch.bfloat16,
                                         compress_statistics=dq).eval()
        assert F._for_tokens(F._qweights(mod), F._SHIFT_FREE_TOKENS)[0].shift is None
        for i, qw in enumerate(F._for_tokens(F._qweights(mod), F._SHIFT_FREE_TOKENS + 1)):
            got = qw.shift.cpu().numpy()
            ow = oracle_weights(mod)[i]
            for e in range(E):
                am = ow.absmax[e]
                if dq:
                    from oracle import c_oracle

                    am = c_oracle.dequant_absmax_dq(am, ow.absmax2[e], ow.offset[e], ow.code2)
                E_ = int(((np.abs(am).astype(np.float32).view(np.uint32) >> 23) & 0xFF).max())
                assert got[e] == 141 - max(E_, 20), (dq, i, e, got[e], E_)


@pytest.mark.parametrize("tokens", [6, 512])
def test_out_of_range_ids_contribute_nothing(tokens):
    """Ids outside [0, E) drop their slots: at decode size, and at prefill size (256- and 32-row
    tiles in the fp16 mode, fp16 down rows whose scales the combine looks up per slot)."""
    _announce(f"dropped ids tokens={tokens}")
    if tokens <= 8:
        mod, hs, top_i, top_w = _make(E=8, tokens=tokens, k=2, seed=11)
    else:
        mod, hs, top_i, top_w = _make(E=8, H=512, inter=256, tokens=tokens, k=2, seed=12, scale=0.05)
    e4b.enable_fast(mod)
    bad = top_i.clone()
    bad[0, 1] = 99
    bad[3, 0] = -1
    if tokens > 8:
        bad[tokens - 1, 1] = -7
        bad[tokens // 2, 0] = 8
    with torch.no_grad():
        got = mod(hs, bad, top_w)
    w_keep = top_w.clone()
    w_keep[bad < 0] = 0
    w_keep[bad > 7] = 0
    safe = bad.clamp(0, 7)
    with torch.no_grad():
        want = mod(hs, safe, w_keep)
    assert _b_rel(got, want) < 1e-2


def test_prefill_side_stream_is_deterministic_and_graph_safe():
    """Prefill-size forwards (256-row wide tiles + 32-row narrow tiles, fp16 mode) run the 32-row
    tiles on a second stream forked from and joined to the caller's: repeated eager calls are
    bit-identical, and a captured forward replays bit-identically to eager, with eager forwards
    and synchronizations between the replays; the result meets the oracle bars."""
    _announce("prefill side stream, graph replays")
    mod, x, idx, w = _skewed_prefill_layer()
    with torch.no_grad():
        ref_loop = mod(x, idx, w)
        assert e4b.enable_fast(mod) == 1
        first = _eager_and_graph_agree(mod, x, idx, w)
    _assert_fidelity(first, ref_loop, _oracle(mod, x, idx, w), "prefill side stream")


def _skewed_prefill_layer(seed=77):
    """A double-quant layer at 1,024 tokens whose routing leaves the last experts a handful of
    rows each, so a forward runs 256-row tiles and 32-row tail tiles (on the second stream)."""
    E, H, I, k, T = 16, 512, 256, 4, 1024
    g = torch.Generator().manual_seed(seed)
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.05
    dn = torch.randn(E, H, I, generator=g) * 0.05
    mod = e4b.Experts4bit.from_float(gu.to(DEV), dn.to(DEV), compute_dtype=torch.bfloat16,
                                     compress_statistics=True).eval()
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    bias = -3.0 * torch.log1p(torch.arange(E, dtype=torch.float32))
    val, idx = torch.topk(torch.randn(T, E, generator=g) + bias, k, dim=-1)
    w = torch.softmax(val, -1).to(torch.bfloat16).to(DEV)
    idx = idx.to(DEV)
    counts = torch.bincount(idx.flatten().cpu(), minlength=E)
    assert int(((counts % 256 > 0) & (counts % 256 <= 32)).sum()) >= 2, counts  # tails exist
    return mod, x, idx, w


def _eager_and_graph_agree(mod, x, idx, w):
    """Repeated eager forwards are bit-identical, and a captured forward replays bit-identically
    to them, with eager forwards and synchronizations between the replays; returns the result."""
    first = mod(x, idx, w)
    for _ in range(3):
        assert torch.equal(mod(x, idx, w), first)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = mod(x, idx, w)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
        assert torch.equal(mod(x, idx, w), first)
        torch.cuda.synchronize()
    return first


def test_lora_prefill_side_stream_is_deterministic_and_graph_safe():
    """The grouped LoRA forward at prefill size also runs its 32-row tail tiles on a second
    stream (t = x . A^T before the fork, t2 after the join): eager repeats and graph replays are
    bit-identical, and the result meets the LoRA oracle bars on every expert's first and last
    token."""
    _announce("LoRA prefill side stream, graph replays")
    base, x, idx, w = _skewed_prefill_layer(seed=78)
    mod = e4b.ExpertsLoRA(base, r=16, alpha=32, dtype=torch.float32).to(DEV).eval()
    g = torch.Generator(device=DEV).manual_seed(79)
    with torch.no_grad():
        for p in (mod.gate_up_lora_B, mod.down_lora_B):
            p.copy_(torch.randn(p.shape, generator=g, device=DEV) * 0.05)
        assert e4b.enable_fast(mod) == 1
        first = _eager_and_graph_agree(mod, x, idx, w)
    assert torch.isfinite(first).all()
    flat = idx.reshape(-1).cpu().numpy()
    rows = sorted({int(t) for e in np.unique(flat) for t in (np.nonzero(flat == e)[0][[0, -1]] // idx.shape[1])})
    w1, w2 = oracle_weights(base)
    lo1 = tuple(t.detach().float().cpu().numpy() for t in (mod.gate_up_lora_A, mod.gate_up_lora_B))
    lo2 = tuple(t.detach().float().cpu().numpy() for t in (mod.down_lora_A, mod.down_lora_B))
    xs, ids, ws = x[rows].float().cpu().numpy(), idx[rows].cpu().numpy(), w[rows].float().cpu().numpy()
    want = moe.forward_lora_fp32(xs, ids, ws, w1, w2, lo1, lo2, mod.scaling)
    assert np.linalg.norm(want - moe.forward_fp32(xs, ids, ws, w1, w2)) / np.linalg.norm(want) > 0.05
    lt1 = tuple(t.detach().cpu() for t in (mod.gate_up_lora_A, mod.gate_up_lora_B))
    lt2 = tuple(t.detach().cpu() for t in (mod.down_lora_A, mod.down_lora_B))
    ref = moe.reference_lora_loop(x[rows].cpu(), idx[rows].cpu(), w[rows].cpu(),
                                  lambda e, dt: torch.from_numpy(w1[e]).to(dt),
                                  lambda e, dt: torch.from_numpy(w2[e]).to(dt), lt1, lt2, mod.scaling,
                                  num_experts=base.num_experts, compute_dtype=torch.bfloat16)
    _assert_fidelity(first[rows], ref, want, f"lora prefill side stream on {len(rows)} tokens")


def test_narrow_tiles_general_epilogues():
    """The narrow kernel's general epilogue paths (32-row tiles in fp16 mode, K = 512 and 256):
    a plain up projection (has_gate=False, the activation epilogue, bf16 rows) against the oracle,
    and DeepSeek-V4's clamped SwiGLU against the module's own forward with the clamp visibly
    active."""
    _announce("narrow tiles: act and clamp epilogues")
    mod, hs, top_i, top_w = _make(E=8, H=512, inter=256, k=4, tokens=48, seed=41, has_gate=False, scale=0.05)
    with torch.no_grad():
        ref = mod(hs, top_i, top_w)
        assert e4b.enable_fast(mod) == 1
        fast = mod(hs, top_i, top_w)
        w1, w2 = F._qweights(mod)
        assert w1.shift is not None  # the fp16 mode ran, so the narrow kernel
    _assert_fidelity(fast, ref, _oracle(mod, hs, top_i, top_w), "narrow act epilogue")

    from experts4bit_qlora_amd.arch.deepseek_v4 import _DeepseekV4ForwardMixin

    TOL = 1.5e-2
    E, H, INTER, K, T = 8, 512, 256, 3, 48

    def v4(limit):
        g = torch.Generator().manual_seed(42)
        m = _DeepseekV4ForwardMixin.from_deepseek_v4(torch.randn(E, 2 * INTER, H, generator=g) * 0.2,
                                                     torch.randn(E, H, INTER, generator=g) * 0.2, limit=limit,
                                                     compute_dtype=torch.bfloat16).to(DEV).eval()
        x = (torch.randn(T, H, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
        val, idx = torch.topk(torch.randn(T, E, generator=g), K, dim=-1)
        return m, x, idx.to(DEV), torch.softmax(val, dim=-1).to(torch.bfloat16).to(DEV)

    mod, x, idx, w = v4(2.0)
    unclamped, *_ = v4(0.0)
    with torch.no_grad():
        ref = mod(x, idx, w)
        ref_noclamp = unclamped(x, idx, w)
        assert _b_rel(ref, ref_noclamp) > 10 * TOL
        assert e4b.enable_fast(mod) == 1
        got = mod(x, idx, w)
    assert _b_rel(got, ref) < TOL, _b_rel(got, ref)
    assert _b_rel(got, ref_noclamp) > 10 * TOL
