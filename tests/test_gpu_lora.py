"""The one-call LoRA forward, ``e4b_moe_lora_forward``: the ExpertsLoRA forward that
``enable_fast`` binds (reference ``engines/fast.py:163-257``; the module math of
``lora.py:251-256, 329-407``).

Small batches add the low-rank deltas inside the decode GEMVs (each lane of a column group takes
a share of the rank, so the delta rides the group's reduction); larger ones run the grouped
GEMMs with the group deltas on the device. Checked here:

* against the fp64 LoRA oracle (``oracle/moe.py: forward_lora_fp32``) over the oracle-decoded
  weights, at the layer bars (rel-Frobenius <= 1e-2, max-abs <= 2e-2 on row-RMS-normalised
  outputs), on geometries that reach every decode kernel shape (4-, 8-, 16- and 32-lane column
  groups, the single-token, multi-token and items kernels), every adapter dtype and ranks 1..64,
  with the adapter moving the output well past those bars;
* with zero adapters, bit for bit against the bare decode forward (the delta adds exactly zero,
  so any change to the kernels' base arithmetic shows);
* the down delta alone (gate_up adapter zero, fp32 output) against its fp64 value from the bare
  h, to 2^-18 of the magnitude bound -- a wrong rank index, B layout or slot weight fails it;
* the decode and grouped paths against each other, dropped ids, graph replays and no syncs.
"""
import numpy as np
import pytest
import torch

import experts4bit_qlora_amd as e4b
from experts4bit_qlora_amd import _native as N
from experts4bit_qlora_amd import fast as F
from experts4bit_qlora_amd import ops
from oracle import moe
from oracle_weights import oracle_weights

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPI = {"swiglu": N.EPI_SWIGLU, "act": N.EPI_ACT, "clamp_swiglu": N.EPI_CLAMP_SWIGLU}


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _base(E, H, I, seed, dq=False, has_gate=True, cdt=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    n1 = 2 * I if has_gate else I
    return e4b.Experts4bit.from_float(torch.randn(E, n1, H, generator=g, device=DEV) * 0.02,
                                      torch.randn(E, H, I, generator=g, device=DEV) * 0.02, compute_dtype=cdt,
                                      has_gate=has_gate, compress_statistics=dq).eval()


def _adapters(base, r, adt, seed, zero1=False, zero2=False):
    """(A1, B1), (A2, B2): A ~ N(0, 1/r^2) as ExpertsLoRA initialises it (lora.py:177-178), B ~
    N(0, 0.02^2) (a trained adapter: the delta is of the order of the base projection)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    E = base.num_experts
    n1, H = base._gate_up_shape
    _, I = base._down_shape
    a1 = torch.randn(E, r, H, generator=g, device=DEV) / r
    b1 = torch.randn(E, n1, r, generator=g, device=DEV) * 0.02
    a2 = torch.randn(E, r, I, generator=g, device=DEV) / r
    b2 = torch.randn(E, H, r, generator=g, device=DEV) * 0.02
    if zero1:
        b1.zero_()
    if zero2:
        b2.zero_()
    return (a1.to(adt), b1.to(adt)), (a2.to(adt), b2.to(adt))


def _inputs(T, E, H, k, seed, xdt=torch.bfloat16, drop=False):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, H, generator=g, device=DEV).to(xdt)
    w, idx = torch.topk(torch.softmax(torch.randn(T, E, generator=g, device=DEV), -1), k, dim=-1)
    if drop:  # ids outside [0, E): their slots are dropped
        idx[0, 0] = -1
        if T > 1:
            idx[T - 1, k - 1] = E
    return x, idx, w.to(xdt)


def _oracle(base, x, idx, w, lora1, lora2, scaling, epi):
    """fp64 LoRA oracle; dropped slots enter with weight 0 (and any valid id)."""
    E = base.num_experts
    ids = idx.cpu().numpy().copy()
    ws = w.float().cpu().numpy().copy()
    bad = (ids < 0) | (ids >= E)
    ids[bad] = 0
    ws[bad] = 0.0
    w1, w2 = oracle_weights(base)
    lo1 = tuple(t.float().cpu().numpy() for t in lora1)
    lo2 = tuple(t.float().cpu().numpy() for t in lora2)
    return moe.forward_lora_fp32(x.float().cpu().numpy(), ids, ws, w1, w2, lo1, lo2, scaling, epilogue=epi)


def _call(base, x, idx, w, lora1, lora2, scaling, epi, path, out_dtype=None, limit=0.0):
    w1, w2 = F._qweights(base)
    return ops.moe_lora_forward(x, idx, w, w1, w2, lora1, lora2, scaling, EPI[epi if isinstance(epi, str) else epi[0]],
                                out_dtype or x.dtype, limit=limit, path=path)


def _bars(got, want, label):
    fro, maxabs, _ = moe.rel_errors(got.float().cpu().numpy(), want)
    print(f"[fidelity] {label}: rel-fro {fro:.2e} max-abs/row-rms {maxabs:.2e}", flush=True)
    assert np.isfinite(fro) and fro <= 1e-2 and maxabs <= 2e-2, (label, fro, maxabs)


# (E, H, I): the decode kernel shapes they reach -- gate_up k = H, down k = I
GEOMS = {
    "g4c2": (8, 256, 128),      # up 4-lane groups x 2 chunks; down 32 lanes, 4 of 32 chunks
    "g4c4": (16, 512, 384),     # up 4 x 4; down 32 lanes, 12 chunks
    "g8": (8, 1024, 512),       # up 8 x 4; down 32 x 1
    "olmoe": (64, 2048, 1024),  # up 16 x 4 (the bench layer); down 32 x 1
    "g16c6": (8, 3072, 768),    # up 16 x 6; down 32 x 1, 24 of 32 chunks
    "g32": (8, 1024, 4096),     # up 8 x 4; down 32 x 4
}


@pytest.mark.parametrize("geom,T,k,r,adt,xdt,dq,epi", [
    ("olmoe", 1, 8, 16, torch.float32, torch.bfloat16, False, "swiglu"),
    ("olmoe", 1, 8, 64, torch.bfloat16, torch.bfloat16, False, "swiglu"),
    ("olmoe", 8, 8, 16, torch.float32, torch.bfloat16, False, "swiglu"),
    ("olmoe", 5, 8, 20, torch.float16, torch.float16, True, "swiglu"),
    ("olmoe", 8, 8, 64, torch.float32, torch.bfloat16, True, "swiglu"),
    ("g4c2", 1, 2, 1, torch.float32, torch.bfloat16, False, "swiglu"),
    ("g4c2", 7, 2, 16, torch.bfloat16, torch.bfloat16, False, "act"),
    ("g4c4", 3, 4, 33, torch.float16, torch.bfloat16, True, "swiglu"),
    ("g4c4", 1, 4, 64, torch.float32, torch.float16, False, ("clamp_swiglu", 1.0)),
    ("g8", 2, 4, 8, torch.bfloat16, torch.bfloat16, False, "swiglu"),
    ("g8", 1, 6, 48, torch.float32, torch.bfloat16, True, "act"),
    ("g16c6", 1, 4, 16, torch.float32, torch.bfloat16, False, "swiglu"),
    ("g16c6", 8, 4, 12, torch.bfloat16, torch.bfloat16, False, "swiglu"),  # 8 x 3072 > the items stage
    ("g32", 4, 2, 16, torch.float32, torch.bfloat16, False, "swiglu"),
    ("g32", 1, 2, 64, torch.float16, torch.float16, True, "swiglu"),
])
def test_decode_lora_matches_the_lora_oracle(geom, T, k, r, adt, xdt, dq, epi):
    E, H, I = GEOMS[geom]
    _announce(f"decode LoRA geom={geom} T={T} k={k} r={r} adapters={adt} x={xdt} dq={dq} epi={epi}")
    gated = epi != "act"
    base = _base(E, H, I, seed=100 + T + r, dq=dq, has_gate=gated, cdt=xdt)
    lora1, lora2 = _adapters(base, r, adt, seed=200 + r)
    scaling = 2.0
    x, idx, w = _inputs(T, E, H, k, seed=300 + T, xdt=xdt)
    limit = epi[1] if isinstance(epi, tuple) else 0.0
    got = _call(base, x, idx, w, lora1, lora2, scaling, epi, N.PATH_GEMV, limit=limit)
    want = _oracle(base, x, idx, w, lora1, lora2, scaling, epi)
    w1, w2 = oracle_weights(base)
    ids, ws = idx.cpu().numpy(), w.float().cpu().numpy()
    bare = moe.forward_fp32(x.float().cpu().numpy(), ids, ws, w1, w2, epi)
    moved = np.linalg.norm(want - bare) / np.linalg.norm(want)
    assert moved > 0.05, moved  # the adapter moves the output well past the bars
    _bars(got, want, f"decode {geom} T={T} r={r}")


@pytest.mark.parametrize("T", [1, 4, 8])
def test_decode_and_grouped_paths_agree_with_the_oracle(T):
    """The same call through the decode GEMVs (E4B_PATH_GEMV) and the grouped GEMMs
    (E4B_PATH_MFMA), with dropped ids: both within the bars of the oracle."""
    E, H, I = GEOMS["olmoe"]
    _announce(f"decode vs grouped LoRA T={T}")
    base = _base(E, H, I, seed=11)
    lora1, lora2 = _adapters(base, 16, torch.float32, seed=12)
    x, idx, w = _inputs(T, E, H, 8, seed=13 + T, drop=True)
    want = _oracle(base, x, idx, w, lora1, lora2, 2.0, "swiglu")
    dec = _call(base, x, idx, w, lora1, lora2, 2.0, "swiglu", N.PATH_GEMV)
    grp = _call(base, x, idx, w, lora1, lora2, 2.0, "swiglu", N.PATH_MFMA)
    _bars(dec, want, f"decode T={T}")
    _bars(grp, want, f"grouped T={T}")


@pytest.mark.parametrize("geom,T,out_dtype", [("olmoe", 1, torch.bfloat16), ("olmoe", 6, torch.float32),
                                              ("g4c2", 3, torch.float32), ("g16c6", 8, torch.bfloat16),
                                              ("g32", 2, torch.float32)])
def test_zero_adapters_are_bit_identical_to_the_bare_decode(geom, T, out_dtype):
    E, H, I = GEOMS[geom]
    _announce(f"zero-adapter decode geom={geom} T={T} out={out_dtype}")
    base = _base(E, H, I, seed=21)
    k = 4
    x, idx, w = _inputs(T, E, H, k, seed=22)
    w1, w2 = F._qweights(base)
    bare = ops.moe_forward(x, idx, w, w1, w2, N.EPI_SWIGLU, out_dtype, path=N.PATH_GEMV)
    for r, adt in ((16, torch.float32), (40, torch.bfloat16)):
        lora1, lora2 = _adapters(base, r, adt, seed=23, zero1=True, zero2=True)
        got = _call(base, x, idx, w, lora1, lora2, 2.0, "swiglu", N.PATH_GEMV, out_dtype=out_dtype)
        assert torch.equal(got, bare), (r, adt)


@pytest.mark.parametrize("geom,T,r,adt", [("olmoe", 1, 16, torch.float32), ("olmoe", 8, 64, torch.bfloat16),
                                          ("g4c4", 3, 5, torch.float16), ("g32", 2, 16, torch.float32)])
def test_down_delta_matches_its_fp64_value(geom, T, r, adt):
    """gate_up adapter zero, fp32 output: out_lora - out_bare == sum_s w_s * scaling *
    (h_s . A2[e]^T) . B2[e]^T, h the bare decode's own h, to 2^-18 of the magnitude bound."""
    E, H, I = GEOMS[geom]
    _announce(f"down delta geom={geom} T={T} r={r} adapters={adt}")
    base = _base(E, H, I, seed=31)
    k = 4
    x, idx, w = _inputs(T, E, H, k, seed=32)
    lora1, lora2 = _adapters(base, r, adt, seed=33, zero1=True)
    scaling = 1.5
    w1, w2 = F._qweights(base)
    bare = ops.moe_forward(x, idx, w, w1, w2, N.EPI_SWIGLU, torch.float32, path=N.PATH_GEMV)
    got = _call(base, x, idx, w, lora1, lora2, scaling, "swiglu", N.PATH_GEMV, out_dtype=torch.float32)
    h = ops.decode_gate_up(x, idx, w1, N.EPI_SWIGLU).double().cpu().numpy()  # [T*k, I] flat order
    A2, B2 = (t.double().cpu().numpy() for t in lora2)
    W2 = oracle_weights(base)[1]
    ids, ws = idx.cpu().numpy(), w.double().cpu().numpy()
    want = np.zeros((T, H))
    bound = np.zeros((T, H))
    for t in range(T):
        for s in range(k):
            e, f = ids[t, s], t * k + s
            hv = h[f]
            want[t] += ws[t, s] * scaling * ((A2[e] @ hv) @ B2[e].T)
            bound[t] += abs(ws[t, s]) * (np.abs(W2[e]) @ np.abs(hv) +
                                         scaling * (np.abs(A2[e]) @ np.abs(hv)) @ np.abs(B2[e]).T)
    diff = (got.double() - bare.double()).cpu().numpy()
    err = np.abs(diff - want)
    assert np.all(err <= bound * 2.0 ** -18 + 1e-9), float((err - bound * 2.0 ** -18).max())
    assert np.linalg.norm(want) > 1e-2 * np.linalg.norm(bare.double().cpu().numpy())  # a real delta


def test_graph_replays_match_eager_and_the_forward_never_syncs():
    """The decode LoRA forward of a 4-layer step captured in a HIP graph: replays with new
    inputs copied in equal the eager call bit for bit, and neither syncs."""
    E, H, I = GEOMS["olmoe"]
    _announce("LoRA decode graph replay")
    layers = []
    for l in range(4):
        base = _base(E, H, I, seed=40 + l)
        lora1, lora2 = _adapters(base, 16, torch.float32, seed=50 + l)
        layers.append((base, F._qweights(base), lora1, lora2))
    static = [_inputs(1, E, H, 8, seed=60 + l) for l in range(4)]

    def step(inputs):
        return [ops.moe_lora_forward(x, idx, w, w1, w2, lo1, lo2, 2.0, N.EPI_SWIGLU, x.dtype)
                for (base, (w1, w2), lo1, lo2), (x, idx, w) in zip(layers, inputs)]

    step(static)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(static)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step(static)
    for rep in range(3):
        fresh = [_inputs(1, E, H, 8, seed=70 + 10 * rep + l) for l in range(4)]
        for (x, idx, w), (x2, idx2, w2) in zip(static, fresh):
            x.copy_(x2)
            idx.copy_(idx2)
            w.copy_(w2)
        torch.cuda.set_sync_debug_mode("error")
        try:
            graph.replay()
            eager = step(fresh)
        finally:
            torch.cuda.set_sync_debug_mode("default")
        torch.cuda.synchronize()
        for l, (o, e_) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e_), (rep, l)


@pytest.mark.parametrize("T", [1, 8])
def test_expertslora_module_takes_the_one_call_path(T):
    """An ExpertsLoRA under enable_fast at decode batch sizes: the same result as the direct
    one-call forward, and within the bars of the oracle."""
    E, H, I = GEOMS["olmoe"]
    _announce(f"ExpertsLoRA module one-call T={T}")
    base = _base(E, H, I, seed=81)
    mod = e4b.ExpertsLoRA(base, r=16, alpha=32, dtype=torch.float32).to(DEV).eval()
    with torch.no_grad():
        for p in (mod.gate_up_lora_B, mod.down_lora_B):
            p.copy_(torch.randn(p.shape, generator=torch.Generator(device=DEV).manual_seed(82), device=DEV) * 0.02)
    x, idx, w = _inputs(T, E, H, 8, seed=83)
    assert e4b.enable_fast(mod) == 1
    with torch.no_grad():
        got = mod(x, idx, w)
        direct = _call(base, x, idx, w, (mod.gate_up_lora_A, mod.gate_up_lora_B), (mod.down_lora_A, mod.down_lora_B),
                       mod.scaling, "swiglu", N.PATH_AUTO)
    assert torch.equal(got, direct)
    want = _oracle(base, x, idx, w, (mod.gate_up_lora_A.detach(), mod.gate_up_lora_B.detach()),
                   (mod.down_lora_A.detach(), mod.down_lora_B.detach()), mod.scaling, "swiglu")
    _bars(got, want, f"module T={T}")
