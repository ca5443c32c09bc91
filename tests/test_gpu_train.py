"""The training lane (``enable_fast_train``) under the reference's parity contract
(``tests/test_fused_train_parity.py:50-224``): forward values, dL/dx and dL/d(every LoRA
parameter) within the measured bf16 noise (forward < 1.5e-2, gradients < 1e-2 relative norm)
against the reference ``ExpertsLoRA.forward`` with a load-bearing adapter; the same assertions
REJECT a 1% LoRA-scaling mutant (the control), and forward parity alone would not.

Below the contract, each kernel of the backward against an independent computation: the grouped
dgrad against fp64 products over the oracle-decoded weights, the per-expert weight gradient
against numpy, the split LoRA passes against the fused one bit for bit.
"""
import numpy as np
import pytest
import torch

import experts4bit_qlora_amd as e4b
from experts4bit_qlora_amd import _native as N
from experts4bit_qlora_amd import fast as F
from experts4bit_qlora_amd import ops
from oracle_weights import oracle_weights

pytestmark = pytest.mark.gpu
DEV = "cuda"
E, HID, INTER, TOP_K = 8, 128, 192, 2
FWD_TOL = 1.5e-2
GRAD_TOL = 1.0e-2


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _rel(got, want):
    want = want.float()
    return ((got.float() - want).norm() / want.norm().clamp_min(1e-12)).item()


def _build(seed=0, scaling_bug=1.0, E_=E, hid=HID, inter=INTER, r=8, dq=False):
    """An ExpertsLoRA over a real NF4 base, B nonzero (test_fused_train_parity.py:76-95)."""
    torch.manual_seed(seed)
    gate_up = (torch.randn(E_, 2 * inter, hid) * 0.1).to(DEV)
    down = (torch.randn(E_, hid, inter) * 0.1).to(DEV)
    base = e4b.Experts4bit.from_float(gate_up, down, quant_type="nf4", compute_dtype=torch.bfloat16,
                                      compress_statistics=dq)
    mod = e4b.ExpertsLoRA(base, r=r, alpha=2 * r, dtype=torch.float32).to(DEV)
    with torch.no_grad():
        for p in (mod.gate_up_lora_B, mod.down_lora_B):
            p.normal_(0, 0.02)
    mod.scaling *= scaling_bug
    return mod.train()


def _inputs(n_tok=64, seed=1, E_=E, hid=HID, top_k=TOP_K):
    torch.manual_seed(seed)
    hs = torch.randn(n_tok, hid, dtype=torch.bfloat16, device=DEV)
    idx = torch.randint(0, E_, (n_tok, top_k), device=DEV)
    wts = torch.rand(n_tok, top_k, dtype=torch.bfloat16, device=DEV)
    torch.manual_seed(seed + 100)
    loss_w = torch.randn(n_tok, hid, device=DEV)
    return hs, idx, wts, loss_w


def _forward_backward(mod, hs, idx, wts, loss_w):
    hs = hs.clone().requires_grad_(True)
    for p in mod.parameters():
        p.grad = None
    out = mod(hs, idx, wts)
    assert out.requires_grad, "a training path that returns a detached tensor trains nothing"
    (out.float() * loss_w).sum().backward()
    grads = {n: p.grad.detach().clone() for n, p in mod.named_parameters() if p.grad is not None}
    assert grads, "no parameter received a gradient"
    return out.detach(), hs.grad.detach().clone(), grads


def assert_parity(candidate, reference, args=None, fwd_tol=FWD_TOL, grad_tol=GRAD_TOL):
    ref_p = dict(reference.named_parameters())
    for n, p in candidate.named_parameters():
        assert torch.equal(p.detach(), ref_p[n].detach()), f"fixtures differ at {n}"
    args = args or _inputs()
    ref_out, ref_dx, ref_grads = _forward_backward(reference, *args)
    got_out, got_dx, got_grads = _forward_backward(candidate, *args)
    measured = {"forward": _rel(got_out, ref_out), "dL/dx": _rel(got_dx, ref_dx)}
    assert measured["forward"] < fwd_tol, f"forward {measured['forward']:.3e}"
    assert measured["dL/dx"] < grad_tol, f"dL/dx {measured['dL/dx']:.3e}"
    assert set(got_grads) == set(ref_grads), sorted(set(got_grads) ^ set(ref_grads))
    for n in ref_grads:
        measured[f"dL/d{n}"] = _rel(got_grads[n], ref_grads[n])
        assert measured[f"dL/d{n}"] < grad_tol, f"dL/d{n} {measured[f'dL/d{n}']:.3e}"
    return measured


def test_training_path_matches_reference_forward_and_gradients():
    """test_fused_train_parity.py:180-189 for the enable_fast_train lane."""
    _announce("train parity contract")
    reference = _build(seed=0)
    candidate = _build(seed=0)
    assert e4b.enable_fast_train(candidate) == 1
    measured = assert_parity(candidate, reference)
    print("enable_fast_train: " + "  ".join(f"{k}={v:.2e}" for k, v in measured.items()), flush=True)


@pytest.mark.parametrize("n_tok,E_,hid,inter,r,dq", [(2048, 8, 256, 128, 16, False), (512, 16, 192, 256, 20, True),
                                                     (3, 8, 128, 192, 8, False)])
def test_training_path_contract_at_other_shapes(n_tok, E_, hid, inter, r, dq):
    """The contract with 128-row tiles (2048 tokens over 8 experts), double-quantized weights and
    an odd rank, and a 3-token batch."""
    _announce(f"train parity n_tok={n_tok} E={E_} hid={hid} inter={inter} r={r} dq={dq}")
    reference = _build(seed=5, E_=E_, hid=hid, inter=inter, r=r, dq=dq)
    candidate = _build(seed=5, E_=E_, hid=hid, inter=inter, r=r, dq=dq)
    assert e4b.enable_fast_train(candidate) == 1
    measured = assert_parity(candidate, reference, args=_inputs(n_tok, seed=6, E_=E_, hid=hid))
    print(f"n_tok={n_tok}: " + "  ".join(f"{k}={v:.2e}" for k, v in measured.items()), flush=True)


def test_contract_detects_a_wrong_gradient():
    """The control (test_fused_train_parity.py:192-205): a 1% LoRA-scaling error must fail."""
    _announce("train contract control")
    reference = _build(seed=0)
    mutant = _build(seed=0, scaling_bug=1.01)
    assert e4b.enable_fast_train(mutant) == 1
    with pytest.raises(AssertionError):
        assert_parity(mutant, reference)


def test_forward_parity_alone_would_miss_a_gradient_bug():
    """test_fused_train_parity.py:208-224, on the fused lane: the mutant's forward passes, its
    parameter gradients do not."""
    _announce("train forward-only control")
    reference = _build(seed=0)
    mutant = _build(seed=0, scaling_bug=1.01)
    assert e4b.enable_fast_train(mutant) == 1
    args = _inputs()
    ref_out, _, ref_grads = _forward_backward(reference, *args)
    got_out, _, got_grads = _forward_backward(mutant, *args)
    assert _rel(got_out, ref_out) < FWD_TOL
    worst = max(_rel(got_grads[n], ref_grads[n]) for n in ref_grads)
    assert worst > GRAD_TOL, worst


def test_enable_disable_markers_and_idempotence():
    _announce("train enable/disable")
    mod = _build(seed=0)
    ref_forward = mod.forward
    assert e4b.enable_fast_train(mod) == 1
    assert hasattr(mod, "_e4b_train_ref") and mod._e4b_dgrad is False
    assert e4b.enable_fast_train(mod) == 0  # already patched
    with pytest.warns(RuntimeWarning, match="dgrad"):
        assert e4b.enable_fast_train(mod, dgrad=True) == 0
    assert e4b.disable_fast_train(mod) == 1
    assert not hasattr(mod, "_e4b_train_ref") and not hasattr(mod, "_e4b_dgrad")
    assert mod.forward == ref_forward
    assert e4b.disable_fast_train(mod) == 0
    mod._e4b_batched_ref = mod.forward  # another lane's marker: skipped
    assert e4b.enable_fast_train(mod) == 0


# ------------------------------------------------------------------ the backward's kernels


def _nf4(E_, n, k, seed, dq=False):
    """A base whose gate_up weights are [E, n, k] (n output features, the dgrad's reduction)."""
    torch.manual_seed(seed)
    return e4b.Experts4bit.from_float((torch.randn(E_, n, k) * 0.05).to(DEV), (torch.randn(E_, k, n) * 0.05).to(DEV),
                                      compute_dtype=torch.bfloat16, has_gate=False, compress_statistics=dq)


@pytest.mark.parametrize("E_,n,k,T,top,tile,gdt,dq", [(8, 256, 320, 700, 2, 128, torch.bfloat16, False),
                                                       (8, 128, 192, 90, 2, 32, torch.bfloat16, True),
                                                       (4, 192, 512, 300, 3, 128, torch.float16, False),
                                                       (16, 64, 128, 33, 4, 32, torch.float16, True)])
def test_grouped_dgrad_matches_fp64(E_, n, k, T, top, tile, gdt, dq):
    """out[m] = g[m] . deq(W[e_m]) against fp64 products over the oracle-decoded weights, rounded
    to the gradient dtype as the kernel's operands are: tolerance 2^-16 of sum |g||w| per output
    (fp32 accumulation only: a wrong row, scale or nibble is off by O(1) of it); 128- and 32-row
    tiles, columns not a multiple of the tile."""
    _announce(f"grouped dgrad E={E_} n={n} k={k} T={T} top={top} tile={tile} g={gdt} dq={dq}")
    base = _nf4(E_, n, k, seed=7, dq=dq)
    w1, _ = F._qweights(base)
    g_ = torch.Generator(device=DEV).manual_seed(8)
    idx = torch.rand(T, E_, generator=g_, device=DEV).argsort(dim=1)[:, :top]  # distinct experts per token
    rb = ops.route(idx, E_, tile_m=tile)
    M = T * top
    g = torch.randn(M, n, generator=g_, device=DEV).to(gdt)
    got = ops.grouped_dgrad(g, w1, rb, M).double().cpu().numpy()
    W = oracle_weights(base)[0]
    Wr = {e: torch.from_numpy(W[e]).to(gdt).double().numpy() for e in range(E_)}  # the kernel's operand values
    offs = rb.offsets.cpu().numpy()
    gd = g.double().cpu().numpy()
    for e in range(E_):
        s, t = int(offs[e]), int(offs[e + 1])
        if s == t:
            continue
        want = gd[s:t] @ Wr[e]
        bound = np.abs(gd[s:t]) @ np.abs(Wr[e])
        assert np.all(np.abs(got[s:t] - want) <= bound * 2.0 ** -16 + 1e-30), e


@pytest.mark.parametrize("r,adt,gather", [(8, torch.float32, True), (20, torch.bfloat16, False), (64, torch.float32, True)])
def test_lora_wgrad_matches_numpy(r, adt, gather):
    """out[e] = scale * u_e^T a_e per expert over its sorted rows (gathered token rows or sorted
    rows), zeros for an expert without rows."""
    _announce(f"lora wgrad r={r} gather={gather}")
    E_, T, top, cols = 12, 150, 2, 320
    g_ = torch.Generator(device=DEV).manual_seed(9)
    idx = torch.randint(0, E_ - 2, (T, top), generator=g_, device=DEV)  # the last two experts get no rows
    rb = ops.route(idx, E_)
    M = T * top
    u = torch.randn(M, r, generator=g_, device=DEV)
    a = torch.randn(T if gather else M, cols, generator=g_, device=DEV).to(torch.bfloat16)
    got = ops.lora_wgrad(u, a, rb, M, E_, 1.5, gather_k=top if gather else 0).double().cpu().numpy()
    offs = rb.offsets.cpu().numpy()
    sf = rb.sorted_flat.cpu().numpy()[:M]
    ud, ad = u.double().cpu().numpy(), a.double().cpu().numpy()
    for e in range(E_):
        s, t = int(offs[e]), int(offs[e + 1])
        rows = ad[sf[s:t] // top] if gather else ad[s:t]
        want = 1.5 * ud[s:t].T @ rows if t > s else np.zeros((r, cols))
        bound = 1.5 * np.abs(ud[s:t]).T @ np.abs(rows) if t > s else np.zeros((r, cols))
        assert np.all(np.abs(got[e] - want) <= bound * 2.0 ** -16 + 1e-30), e


def test_split_lora_passes_equal_the_fused_delta():
    """e4b_lora_t then e4b_lora_t_add == e4b_lora_delta, bit for bit (the same kernels)."""
    _announce("lora split passes")
    E_, T, top, k_in, n_out, r = 8, 200, 2, 256, 384, 16
    g_ = torch.Generator(device=DEV).manual_seed(10)
    idx = torch.randint(0, E_, (T, top), generator=g_, device=DEV)
    rb = ops.route(idx, E_)
    M = T * top
    x = torch.randn(T, k_in, generator=g_, device=DEV).to(torch.bfloat16)
    A = torch.randn(E_, r, k_in, generator=g_, device=DEV) / r
    B = torch.randn(E_, n_out, r, generator=g_, device=DEV) * 0.02
    base = torch.randn(M, n_out, generator=g_, device=DEV)
    fused = ops.lora_delta(x, rb, M, E_, A, B, 2.0, base.clone(), gather_k=top, delta_dtype=torch.float32)
    t = ops.lora_t(x, rb, M, E_, A, gather_k=top)
    split = ops.lora_t_add(t, rb, M, E_, B, 2.0, base.clone())
    assert torch.equal(fused, split)


@pytest.mark.parametrize("n_tok,E_,top", [(64, 8, 2), (1024, 8, 4)])
def test_training_lane_is_bit_identical_across_runs(n_tok, E_, top):
    """ref tests/test_deterministic_scatter.py:62-80: the training forward and every gradient are
    bit-identical over repeated runs (no float atomics anywhere in the lane). 1,024 tokens x 4
    slots over 8 experts runs the 128-row tiles; 64 x 2 the 32-row ones."""
    _announce(f"train determinism n_tok={n_tok} E={E_} top={top}")
    mod = _build(seed=3, E_=E_)
    assert e4b.enable_fast_train(mod) == 1
    args = _inputs(n_tok=n_tok, seed=4, E_=E_, top_k=top)
    out0, dx0, g0 = _forward_backward(mod, *args)
    assert set(g0) == {"gate_up_lora_A", "gate_up_lora_B", "down_lora_A", "down_lora_B"}, sorted(g0)
    for run in range(1, 8):
        out, dx, grads = _forward_backward(mod, *args)
        assert torch.equal(out, out0), f"run {run}: forward differs"
        assert torch.equal(dx, dx0), f"run {run}: dL/dx differs"
        for n in g0:
            assert torch.equal(grads[n], g0[n]), f"run {run}: dL/d{n} differs"
