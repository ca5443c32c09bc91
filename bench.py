"""Benchmark of the frozen-expert MoE forward on one MI355X.

Workload: OLMoE-1B-7B geometry, all 16 MoE layers stacked, decode.
E=64 experts, hidden 2048, moe_intermediate 1024, top-8 softmax routing (not renormalised),
SwiGLU; weights N(0, 0.02) from per-layer seeds, NF4 / blocksize 64 / fp32 absmax; bf16 N(0,1)
activations. One "step" = one decode pass through the 16 layers at batch 1 (route, gate_up +
SwiGLU, down, combine per layer), replayed from a HIP graph (the fused path never syncs). Inputs
and weights are resident in HBM when the timed region starts.

``value`` = routed-expert HBM bytes per step / step time (GB/s): each distinct routed expert's
3,538,944 bytes (packed NF4 + fp32 absmax, both projections) counted once per layer. The line
also carries us/layer and tok/s at batches 1, 8 and 64, the Qwen3-30B-A3B-geometry 4096-token
Zipf prefill in TFLOP/s, the Qwen3-geometry double-quant decode at batches 1, 32
and 256, the gpt-oss MXFP4 layer at 1 and 2048 tokens, the
ExpertsLoRA decode step and training step (forward + backward, grouped dgrad TFLOP/s), the
dominant kernel's roofline measured with HIP events on the launch stream, and the reference
per-expert loop timed on the host CPU.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-prefill] [--no-extra]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer µs + achieved HBM GB/s at bs=1; MFMA TFLOP/s at 4096-token prefill"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

OLMOE = dict(E=64, H=2048, I=1024, k=8, layers=16, renorm=False)
QWEN3 = dict(E=128, H=2048, I=768, k=8, renorm=True)
GPTOSS = dict(E=32, H=2880, I=2880, k=4)


# HBM bytes per launch, from the two counter runs summarised in profiles/ (FETCH_SIZE and
# WRITE_SIZE, scaled by what a 256 MiB device copy reads for each in the same runs). Keyed by
# the kernel it was measured on, so a changed kernel reports null until it is measured again.
MEASURED_TRAFFIC = {
    "decode_up_kernel<bf16, nf4, G=16, CPL=4, full, gated>": 19_074_000,
    "decode_down_kernel<bf16, nf4, G=32, CPL=1, JOBS=1, full>": 9_711_000,
    # prefill: keyed by the kernel and the projection ("<kernel> gate_up_256row"); measured
    # again for each kernel change (profiles/prefill_qwen3_4096_zipf.txt)
    "gemm_wide8_kernel<bf16, nf4_dq, fp16 mode> gate_up_256row": 421_200_000,
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def nf4_expert_bytes(H, I):
    """Packed NF4 + fp32 absmax bytes of one expert, both projections."""
    gu = 2 * I * H // 2 + 2 * I * H // 64 * 4
    dn = H * I // 2 + H * I // 64 * 4
    return gu, dn


def dq_expert_bytes(H, I):
    """Packed NF4 + u8 absmax codes + fp32 absmax2 + fp32 offset, both projections."""
    tot = 0
    for n, k in ((2 * I, H), (H, I)):
        nb = n * k // 64
        tot += n * k // 2 + nb + math.ceil(nb / 256) * 4 + 4
    return tot


def make_layer(cfg, seed, dq=False):
    import torch

    import experts4bit_qlora_amd as e4b

    g = torch.Generator(device="cuda").manual_seed(seed)
    E, H, I = cfg["E"], cfg["H"], cfg["I"]
    gu = torch.randn(E, 2 * I, H, generator=g, device="cuda") * 0.02
    dn = torch.randn(E, H, I, generator=g, device="cuda") * 0.02
    mod = e4b.Experts4bit.from_float(gu, dn, compute_dtype=torch.bfloat16, compress_statistics=dq).eval()
    del gu, dn
    return mod


def make_inputs(cfg, T, seed, zipf=None):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(T, cfg["H"], generator=g, device="cuda").to(torch.bfloat16)
    logits = torch.randn(T, cfg["E"], generator=g, device="cuda")
    if zipf is not None:
        rank = torch.randperm(cfg["E"], generator=torch.Generator().manual_seed(seed + 1)).cuda() + 1
        logits = logits - zipf * torch.log(rank.float())
    w, idx = torch.topk(torch.softmax(logits, -1), cfg["k"], dim=-1)
    if cfg.get("renorm"):
        w = w / w.sum(-1, keepdim=True)
    return x, idx, w.to(torch.bfloat16)


def graph_of(fn):
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def time_graph(g, steps, warmup):
    import torch

    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per replay


def decode_bench(mods, cfg, T, steps, warmup, seed0):
    """Time the 16-layer decode step at batch T; returns a dict of figures."""
    import torch

    inputs = [make_inputs(cfg, T, seed0 + 10 * l) for l in range(len(mods))]
    distinct = [int(torch.unique(idx).numel()) for _, idx, _ in inputs]
    gu_b, dn_b = nf4_expert_bytes(cfg["H"], cfg["I"])
    step_bytes = sum(distinct) * (gu_b + dn_b)

    def step():
        with torch.no_grad():
            return [m(x, idx, w) for m, (x, idx, w) in zip(mods, inputs)]

    eager = step()
    g, outs = graph_of(step)
    g.replay()
    torch.cuda.synchronize()
    for a, b in zip(eager, outs):  # the graph replays the exact eager computation
        assert torch.equal(a, b), "graph replay differs from the eager forward"
    # eager wall time (Python + launches, back-to-back steps), for reference
    n_eager = max(10, steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_eager):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / n_eager
    ms = time_graph(g, steps, warmup)
    L = len(mods)
    return {
        "batch": T,
        "ms_per_step": ms,
        "us_per_layer": ms * 1e3 / L,
        "tok_per_s": T / (ms / 1e3),
        "routed_bytes_per_step": step_bytes,
        "working_set_bytes": step_bytes,  # distinct weights one replay reads (each read once)
        "distinct_experts_per_layer": round(sum(distinct) / L, 2),
        "hbm_gbs": step_bytes / (ms / 1e3) / 1e9,
        "hbm_frac": step_bytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS,
        "eager_ms_per_step": eager_ms,
        "eager_vs_graph": round(eager_ms / ms, 3),
    }


def rotating_ids(L, E, k, seed):
    """Expert-id sets for cache-honest bs=1 legs: layer l's experts split into R = E // k disjoint
    sets of k (bank [R, L, 1, k]) and the buffer a captured graph reads (ids [L, 1, k])."""
    import torch

    R = E // k
    g = torch.Generator().manual_seed(seed)
    bank = torch.stack([torch.randperm(E, generator=g)[: R * k].view(R, 1, k) for _ in range(L)], 1).cuda()
    return bank, bank[0].clone()


def time_rotating(gr, bank, ids, steps, warmup):
    """ms per replay of a graph reading `ids`, with set r % R copied into it before replay r (so a
    layer's experts come back only after R - 1 replays of other experts); the copies are timed
    alone and subtracted. Returns (ms, copy_ms)."""
    import torch

    R = bank.shape[0]

    def run(n, replay):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for r in range(n):
            ids.copy_(bank[r % R])
            if replay:
                gr.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / n

    run(warmup * R, True)
    n = max(steps, 4 * R)
    ms = run(n, True)
    copy_ms = run(n, False)
    return ms - copy_ms, copy_ms


def rotating_decode_bench(mods, cfg, steps, warmup, seed0):
    """The bs=1 decode step with the routed experts rotated between replays, to show the graph
    replays are not served from the 256 MB Infinity Cache: each layer's experts are split into
    E / k disjoint sets of k, and replay r routes every layer's token to set r mod (E / k), so an
    expert's weights are read again only after E / k - 1 replays of other experts (3.2 GB at
    OLMoE geometry). One device copy before each replay installs the set; the same copies are
    timed alone and subtracted."""
    import torch

    L, E, k = len(mods), cfg["E"], cfg["k"]
    bank, ids = rotating_ids(L, E, k, seed0)  # the graph reads layer l's ids from ids[l]
    inputs = [make_inputs(cfg, 1, seed0 + 10 * l) for l in range(L)]

    def step():
        with torch.no_grad():
            return [m(x, ids[l], w) for l, (m, (x, _, w)) in enumerate(zip(mods, inputs))]

    gr, _ = graph_of(step)
    ms, copy_ms = time_rotating(gr, bank, ids, steps, warmup)
    gu_b, dn_b = nf4_expert_bytes(cfg["H"], cfg["I"])
    return {"us_per_layer": round(ms * 1e3 / L, 3), "id_sets": bank.shape[0],
            "copy_us_per_step": round(copy_ms * 1e3, 2),
            "working_set_bytes": L * E * (gu_b + dn_b)}


def lora_bench(mods, cfg, steps, warmup, seed0, bare, rank=16):
    """The 16-layer decode step through ExpertsLoRA wrappers (the module load_moe_4bit_streaming
    builds) over the same bases: rank-16 fp32 adapters with nonzero B (a trained adapter, so the
    LoRA path runs), graph-replayed like the bare step; us per layer and the ratio to the bare
    layer at the same batch."""
    import torch

    import experts4bit_qlora_amd as e4b

    wrappers = []
    for l, m in enumerate(mods):
        w = e4b.ExpertsLoRA(m, r=rank, alpha=2 * rank, dtype=torch.float32).to("cuda").eval()
        g = torch.Generator(device="cuda").manual_seed(seed0 + 50 + l)
        with torch.no_grad():
            for p in (w.gate_up_lora_B, w.down_lora_B):
                p.copy_(torch.randn(p.shape, generator=g, device="cuda") * 0.02)
        assert e4b.enable_fast(w) == 1
        wrappers.append(w)
    out = {}
    for T in (1, 8):
        inputs = [make_inputs(cfg, T, seed0 + 10 * l) for l in range(len(mods))]

        def step():
            with torch.no_grad():
                return [m(x, idx, w) for m, (x, idx, w) in zip(wrappers, inputs)]

        g, _ = graph_of(step)
        ms = time_graph(g, steps, warmup)
        us = ms * 1e3 / len(mods)
        out[f"bs{T}"] = {"us_per_layer": round(us, 3), "vs_bare_layer": round(us / bare[T]["us_per_layer"], 3),
                         "rank": rank}
    out["prefill4096"] = lora_prefill_bench(mods[0], cfg, steps, warmup, seed0, rank, torch.float32, wrappers[0])
    out["prefill4096_r64_bf16"] = lora_prefill_bench(mods[0], cfg, steps, warmup, seed0, 64, torch.bfloat16)
    for w, m in zip(wrappers, mods):
        e4b.disable_fast(w)  # restores the wrapped bases too: patch them again
        assert e4b.enable_fast(m) == 1
    return out


def lora_prefill_bench(base, cfg, steps, warmup, seed0, rank, dtype, wrapper=None):
    """One layer at 4,096 tokens, bare and through an ExpertsLoRA wrapper (rank, adapter dtype,
    nonzero B), each graph-replayed on its own: the grouped LoRA form (t = x . A^T on the matrix
    cores, fp16-mode GEMMs whose accumulators start as the tile's delta)."""
    import torch

    import experts4bit_qlora_amd as e4b

    made = wrapper is None
    if made:
        wrapper = e4b.ExpertsLoRA(base, r=rank, alpha=2 * rank, dtype=dtype).to("cuda").eval()
        g = torch.Generator(device="cuda").manual_seed(seed0 + 90 + rank)
        with torch.no_grad():
            for p in (wrapper.gate_up_lora_B, wrapper.down_lora_B):
                p.copy_((torch.randn(p.shape, generator=g, device="cuda") * 0.02).to(p.dtype))
        assert e4b.enable_fast(wrapper) == 1
    T = 4096
    x, idx, w = make_inputs(cfg, T, seed0 + 7)

    def layer_ms(mod):
        def step():
            with torch.no_grad():
                return mod(x, idx, w)

        g, _ = graph_of(step)
        return time_graph(g, steps, warmup)

    bare_ms, lora_ms = layer_ms(base), layer_ms(wrapper)
    # (no disable_fast on the wrapper: it would also restore the wrapped base's own forward)
    return {"ms_lora": round(lora_ms, 4), "ms_bare": round(bare_ms, 4), "vs_bare_layer": round(lora_ms / bare_ms, 3),
            "rank": rank, "adapter_dtype": str(dtype).replace("torch.", ""), "tokens": T}


def dominant_kernel_roofline(mods, cfg, steps, warmup, seed0):
    """The decode gate_up kernel (routing + gate_up GEMV + SwiGLU) at bs=1 alone, 16 layers per
    graph replay, timed with HIP events on the launch stream: achieved = routed gate_up bytes
    per launch / average launch duration. The second decode kernel (down GEMV + k-slot combine)
    is timed the same way, on the h the first one wrote; it is reported beside the roofline.
    Both replay with rotating expert sets (time_rotating): one replay reads 302 MB (up) or 151 MB
    (down) of weights, within the 256 MB Infinity Cache's reach, so each replay routes every layer
    to the next of 8 disjoint expert sets and a set's weights return only after 7 other replays
    (2.4 GB / 1.2 GB cycled)."""
    import torch

    from experts4bit_qlora_amd import _native as N
    from experts4bit_qlora_amd import fast as F
    from experts4bit_qlora_amd import ops

    L = len(mods)
    inputs = [make_inputs(cfg, 1, seed0 + 10 * l) for l in range(L)]
    qws = [F._qweights(m) for m in mods]
    bank, ids = rotating_ids(L, cfg["E"], cfg["k"], seed0 + 5)
    torch.cuda.synchronize()

    def launches():
        return [ops.decode_gate_up(x, ids[l], qw[0], N.EPI_SWIGLU) for l, ((x, _, _), qw) in enumerate(zip(inputs, qws))]

    g, hs = graph_of(launches)
    ms, _ = time_rotating(g, bank, ids, steps * 4, warmup)
    per_launch_us = ms * 1e3 / L
    gu_b, dn_b = nf4_expert_bytes(cfg["H"], cfg["I"])
    bytes_per_launch = cfg["k"] * gu_b  # 8 distinct routed experts at bs=1
    achieved = bytes_per_launch / (per_launch_us * 1e-6) / 1e9
    kernel = "decode_up_kernel<bf16, nf4, G=16, CPL=4, full, gated>"

    def down_launches():
        return [ops.decode_down_combine(h, ids[l], w, qw[1], x.dtype)
                for l, (h, (x, _, w), qw) in enumerate(zip(hs, inputs, qws))]

    g2, _ = graph_of(down_launches)
    ms2, _ = time_rotating(g2, bank, ids, steps * 4, warmup)
    down_us = ms2 * 1e3 / L
    down_bytes = cfg["k"] * dn_b
    return {
        "bound": "hbm",
        "kernel": kernel + " (routing + gate_up + SwiGLU, bs=1)",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": MEASURED_TRAFFIC.get(kernel),
        "bytes_per_launch": bytes_per_launch,
        "avg_launch_us": round(per_launch_us, 3),
        "timer": "HIP events on the launch stream, 16 launches per graph replay, expert sets rotated",
        "working_set_bytes": L * cfg["E"] * gu_b,  # gate_up weights cycled by the rotation
        "second_kernel": {
            "kernel": "decode_down_kernel<bf16, nf4, G=32, CPL=1, JOBS=1, full> (down + k-slot combine, bs=1)",
            "avg_launch_us": round(down_us, 3),
            "bytes_per_launch": down_bytes,
            "achieved": round(down_bytes / (down_us * 1e-6) / 1e9, 1),
            "frac": round(down_bytes / (down_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": MEASURED_TRAFFIC.get("decode_down_kernel<bf16, nf4, G=32, CPL=1, JOBS=1, full>"),
            "working_set_bytes": L * cfg["E"] * dn_b,
        },
    }


def prefill_gemm_roofline(mod, x, idx, w, cfg, reps=20):
    """The prefill's four GEMM launches (fp16 matrix-core mode), each timed with HIP events that
    the library records on the launch's own stream right before and after it (e4b_set_probe),
    over `reps` forwards: algorithmic FLOP of each launch (the rows its tiles hold, both gate_up
    halves) / its average duration, against the dense bf16/fp16 peak. The 256-row tiles
    (gemm_wide8_kernel) carry every expert's rows except a last tile of at most 32 rows, which the
    32-row launch (gemm_narrow_kernel, on the library's second stream beside the 256-row launch)
    takes. Each forward is queued behind a short device-side wait, so the host has issued the
    whole forward before the device reaches the first recorded event. The 32-row launches stream a
    whole expert's weights per tile for a few rows: their entries also carry the weight bytes of
    those tiles and the HBM rate."""
    import torch

    from experts4bit_qlora_amd import _native as N

    L = N.lib()
    H, I = cfg["H"], cfg["I"]
    counts = torch.bincount(idx.reshape(-1), minlength=cfg["E"]).cpu().tolist()
    tail = [c % 256 if 0 < c % 256 <= 32 else 0 for c in counts]
    rows = {256: sum(counts) - sum(tail), 32: sum(tail)}
    flop = {(bm, "gate_up"): 2 * r * 2 * I * H for bm, r in rows.items()}
    flop.update({(bm, "down"): 2 * r * H * I for bm, r in rows.items()})
    # weight bytes per expert and projection (the prefill layer is double-quantized NF4)
    n_tail = sum(1 for t in tail if t)

    def proj_bytes(n, k):
        nb = n * k // 64
        return n * k // 2 + nb + math.ceil(nb / 256) * 4 + 4
    tail_bytes = {"gate_up": n_tail * proj_bytes(2 * I, H), "down": n_tail * proj_bytes(H, I)}
    kernels = {256: "gemm_wide8_kernel<bf16, nf4_dq, fp16 mode>", 32: "gemm_narrow_kernel<nf4_dq>"}
    sites = {("gate_up", 256): N.PROBE_GATE_UP_BIG, ("gate_up", 32): N.PROBE_GATE_UP_TAIL,
             ("down", 256): N.PROBE_DOWN_BIG, ("down", 32): N.PROBE_DOWN_TAIL}
    before, after = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    before.record()
    after.record()  # the events exist (torch creates them at their first record)
    torch.cuda.synchronize()
    out = {}
    with torch.no_grad():
        mod(x, idx, w)
        for (proj, bm), site in sites.items():
            durs = []
            for _ in range(reps):
                torch.cuda._sleep(100_000)
                N.check("e4b_set_probe", L.e4b_set_probe(site, before.cuda_event, after.cuda_event))
                try:
                    mod(x, idx, w)
                finally:
                    N.check("e4b_set_probe", L.e4b_set_probe(N.PROBE_OFF, None, None))
                torch.cuda.synchronize()
                durs.append(before.elapsed_time(after) * 1e3)
            us = sum(durs) / len(durs)
            tf = flop[(bm, proj)] / (us * 1e-6) / 1e12
            key = f"{proj}_{bm}row"
            out[key] = {"kernel": kernels[bm], "avg_launch_us": round(us, 2), "median_launch_us":
                        round(statistics.median(durs), 2), "calls": len(durs), "flop_per_launch": flop[(bm, proj)],
                        "achieved": round(tf, 1), "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
            if bm == 32:  # whole experts' weights for a few rows each: the HBM view
                gbs = tail_bytes[proj] / (us * 1e-6) / 1e9
                out[key].update({"tiles": n_tail, "weight_bytes": tail_bytes[proj],
                                 "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
    dom_key = max(out, key=lambda key: out[key]["avg_launch_us"])
    dom = out[dom_key]
    return {"bound": "mfma", "kernel": f"{dom['kernel']} ({dom_key.rsplit('_', 1)[0]}, dominant prefill GEMM)",
            "achieved": dom["achieved"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": dom["frac"],
            "traffic": MEASURED_TRAFFIC.get(f"{dom['kernel']} {dom_key}"),
            "flop_per_launch": dom["flop_per_launch"], "avg_launch_us": dom["avg_launch_us"],
            "timer": f"HIP events recorded by the library on the launch's stream (e4b_set_probe), {reps} forwards "
                     "per launch", "launches": out}


def pmc_pass(mods, cfg, seed0):
    """One eager decode layer (gate_up kernel, then down + combine kernel) per layer at batch 1
    (no graph, so a counter run sees each dispatch), then one 256 MiB device-to-device copy:
    its FETCH_SIZE / WRITE_SIZE per dispatch against the 268,435,456 bytes it must move give
    the counters' bytes-per-KiB scale."""
    import torch

    from experts4bit_qlora_amd import _native as N
    from experts4bit_qlora_amd import fast as F
    from experts4bit_qlora_amd import ops

    inputs = [make_inputs(cfg, 1, seed0 + 10 * l) for l in range(len(mods))]
    torch.cuda.synchronize()
    for (x, idx, w), m in zip(inputs, mods):
        w1, w2 = F._qweights(m)
        h = ops.decode_gate_up(x, idx, w1, N.EPI_SWIGLU)
        ops.decode_down_combine(h, idx, w, w2, x.dtype)
    torch.cuda.synchronize()
    copy_bytes = calibration_copy()
    gu_b, _ = nf4_expert_bytes(cfg["H"], cfg["I"])
    print(json.dumps({"pmc_pass": {"kernel_bytes_per_launch": cfg["k"] * gu_b, "launches": len(mods),
                                   "copy_bytes": copy_bytes}}), flush=True)


def calibration_copy():
    """One 256 MiB device-to-device copy: a counter run reads its FETCH_SIZE / WRITE_SIZE against
    the 268,435,456 bytes it must move, which gives the counters' bytes-per-KiB scale."""
    import torch

    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    return src.numel()


def prefill_bench(steps, warmup):
    """Qwen3-30B-A3B geometry, one layer, 4096 tokens, Zipf(1.1) routing, double-quant."""
    import torch

    cfg = QWEN3
    mod = make_layer(cfg, seed=1000 + 300, dq=True)
    import experts4bit_qlora_amd as e4b

    e4b.enable_fast(mod)
    x, idx, w = make_inputs(cfg, 4096, seed=1000 + 301, zipf=1.1)
    counts = torch.bincount(idx.reshape(-1), minlength=cfg["E"])

    def step():
        with torch.no_grad():
            return mod(x, idx, w)

    g, _ = graph_of(step)
    ms = time_graph(g, max(steps, 10), warmup)
    flops = 2 * cfg["k"] * 4096 * (2 * cfg["I"] * cfg["H"] + cfg["H"] * cfg["I"])
    tflops = flops / (ms / 1e3) / 1e12
    roof = prefill_gemm_roofline(mod, x, idx, w, cfg)
    return {
        "roofline": roof,
        "workload": "Qwen3-30B-A3B geometry, 1 layer, 4096-token prefill, Zipf(1.1), NF4 double-quant",
        "ms": ms,
        "tflops": tflops,
        "mfma_frac": tflops / BF16_PEAK_TFLOPS,
        "flop": flops,
        "max_rows_per_expert": int(counts.max().item()),
        "min_rows_per_expert": int(counts.min().item()),
    }


def qwen3_decode_benches(steps, warmup, layers=8, batches=(1, 32, 256)):
    """configs[2], Qwen3 decode with double-quant weights: a stack of layers per graph replay;
    batch 1 runs the decode kernels, 32 and 256 the 32-row MFMA tiles (gemm_narrow_kernel)."""
    import torch

    import experts4bit_qlora_amd as e4b

    out = {}
    cfg = QWEN3
    mods = [make_layer(cfg, seed=1000 + 200 + l, dq=True) for l in range(layers)]
    for m in mods:
        e4b.enable_fast(m)
    per_expert = dq_expert_bytes(cfg["H"], cfg["I"])
    for T in batches:
        inputs = [make_inputs(cfg, T, seed=1000 + 210 + T + 7 * l) for l in range(layers)]
        if T == 1:
            # 8 layers x 8 experts = 156 MB per replay, within the Infinity Cache's reach: rotate
            # 16 disjoint expert sets per layer (a set returns after 15 other replays, 2.5 GB)
            bank, ids = rotating_ids(layers, cfg["E"], cfg["k"], 1000 + 215)

            def step():
                with torch.no_grad():
                    return [m(x, ids[l], w) for l, (m, (x, _, w)) in enumerate(zip(mods, inputs))]

            g, _ = graph_of(step)
            ms = time_rotating(g, bank, ids, steps * 2, warmup)[0] / layers
            nbytes = cfg["k"] * per_expert
            ws = layers * cfg["E"] * per_expert
        else:
            def step():
                with torch.no_grad():
                    return [m(x, idx, w) for m, (x, idx, w) in zip(mods, inputs)]

            g, _ = graph_of(step)
            ms = time_graph(g, steps * 2, warmup) / layers
            nbytes = sum(int(torch.unique(idx).numel()) for _, idx, _ in inputs) / layers * per_expert
            ws = nbytes * layers  # 8 layers of 112-128 distinct experts: 2.2-2.5 GB per replay
        out[f"qwen3_dq_bs{T}"] = {"us": ms * 1e3, "hbm_gbs": nbytes / (ms / 1e3) / 1e9, "layers": layers,
                                  "working_set_bytes": int(ws), "expert_sets_rotated": T == 1}
    return out


def extra_benches(steps, warmup, qwen_layers=8, gptoss_layers=4):
    """configs[2] (Qwen3 decode, double-quant) and configs[4] (gpt-oss MXFP4 + biases): a stack of
    layers (independent weights and inputs) per graph replay, as for the OLMoE decode step, so the
    per-layer time does not carry a whole graph launch; us = replay time / layers."""
    import torch

    import experts4bit_qlora_amd as e4b

    out = qwen3_decode_benches(steps, warmup, qwen_layers)
    torch.cuda.empty_cache()
    out.update(gptoss_benches(steps, warmup, gptoss_layers))
    return out


def gptoss_benches(steps, warmup, gptoss_layers=4):
    """gpt-oss MXFP4 layers with biases, batch 1 (decode kernels, expert sets rotated)
    and 2,048 tokens (256-row tiles on the eight-wave wide kernel, 32-row tails)."""
    import torch

    import experts4bit_qlora_amd as e4b

    out = {}
    cfg = GPTOSS
    E, H, I = cfg["E"], cfg["H"], cfg["I"]
    mods = []
    for l in range(gptoss_layers):
        g0 = torch.Generator(device="cuda").manual_seed(1400 + l)
        gu = torch.randn(E, 2 * I, H, generator=g0, device="cuda") * 0.02
        dn = torch.randn(E, H, I, generator=g0, device="cuda") * 0.02
        b1 = torch.randn(E, 2 * I, generator=g0, device="cuda") * 0.02
        b2 = torch.randn(E, H, generator=g0, device="cuda") * 0.02
        mod = e4b.GptOssExpertsMxfp4.from_float(gu, b1, dn, b2).eval()
        del gu, dn
        e4b.enable_fast(mod)
        mods.append(mod)
    per_expert = (2 * I * H + H * I) // 2 + (2 * I * H + H * I) // 32 + (2 * I + H) * 2
    for T in (1, 2048):
        inputs = []
        for l in range(gptoss_layers):
            gi = torch.Generator(device="cuda").manual_seed(1410 + T + 13 * l)
            x = torch.randn(T, H, generator=gi, device="cuda").to(torch.bfloat16)
            val, idx = torch.topk(torch.randn(T, E, generator=gi, device="cuda"), cfg["k"], dim=-1)
            inputs.append((x, idx, torch.softmax(val, -1).to(torch.bfloat16)))
        if T == 1:
            # 4 layers x 4 experts = 212 MB per replay, within the Infinity Cache's reach: rotate 8
            # disjoint expert sets per layer (a set returns after 7 other replays, 1.7 GB)
            bank, ids = rotating_ids(gptoss_layers, E, cfg["k"], 1415)

            def step():
                with torch.no_grad():
                    return [m(x, ids[l], w) for l, (m, (x, _, w)) in enumerate(zip(mods, inputs))]

            g, _ = graph_of(step)
            ms = time_rotating(g, bank, ids, steps, warmup)[0] / gptoss_layers
            nbytes = cfg["k"] * per_expert
            ws = gptoss_layers * E * per_expert
        else:
            def step():
                with torch.no_grad():
                    return [m(x, idx, w) for m, (x, idx, w) in zip(mods, inputs)]

            g, _ = graph_of(step)
            ms = time_graph(g, steps, warmup) / gptoss_layers
            nbytes = sum(int(torch.unique(idx).numel()) for _, idx, _ in inputs) / gptoss_layers * per_expert
            ws = nbytes * gptoss_layers
        flops = 2 * cfg["k"] * T * (2 * I * H + H * I)
        out[f"gptoss_mxfp4_bs{T}"] = {"us": ms * 1e3, "hbm_gbs": nbytes / (ms / 1e3) / 1e9,
                                      "tflops": flops / (ms / 1e3) / 1e12, "layers": gptoss_layers,
                                      "working_set_bytes": int(ws), "expert_sets_rotated": T == 1}
    return out


def train_bench(steps, warmup, tokens=2048, rank=16, ref_steps=3):
    """The training lane on one OLMoE-geometry layer (E=64, H=2048, I=1024, top-8): ExpertsLoRA
    with rank-16 fp32 adapters (B nonzero), a 2048-token micro-batch, loss = sum(out * fixed
    weights). Times the fused forward + backward (enable_fast_train) and the module's reference
    per-expert loop (same GPU, same module) with events, and the grouped dgrad of each projection
    alone: algorithmic FLOP 2 * M * n * k per launch / its average time, against the dense bf16
    peak."""
    import torch

    import experts4bit_qlora_amd as e4b
    from experts4bit_qlora_amd import fast as F
    from experts4bit_qlora_amd import ops

    cfg = OLMOE
    base = make_layer(cfg, seed=4242)
    mod = e4b.ExpertsLoRA(base, r=rank, alpha=2 * rank, dtype=torch.float32).to("cuda").train()
    g = torch.Generator(device="cuda").manual_seed(4243)
    with torch.no_grad():
        for p in (mod.gate_up_lora_B, mod.down_lora_B):
            p.copy_(torch.randn(p.shape, generator=g, device="cuda") * 0.02)
    x, idx, w = make_inputs(cfg, tokens, seed=4244)
    loss_w = torch.randn(tokens, cfg["H"], generator=g, device="cuda")

    def step():
        xs = x.detach().requires_grad_(True)
        for p in mod.parameters():
            p.grad = None
        (mod(xs, idx, w).float() * loss_w).sum().backward()

    def timed(n_steps, n_warm):
        for _ in range(n_warm):
            step()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(n_steps):
            step()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / n_steps

    ref_ms = timed(ref_steps, 1)
    assert e4b.enable_fast_train(mod) == 1
    fused_ms = timed(steps, warmup)

    # the dgrad launches alone, on the routing the lane builds
    E, H, I, k = cfg["E"], cfg["H"], cfg["I"], cfg["k"]
    M = tokens * k
    w1, w2 = F._qweights(base)
    rb = ops.route(idx, E, tile_m=128 if M >= 64 * min(E, M) else 32)
    dg = {}
    for name, qw, n_, k_ in (("gate_up", w1, 2 * I, H), ("down", w2, H, I)):
        gr = torch.randn(M, n_, generator=g, device="cuda").to(torch.bfloat16)
        for _ in range(warmup):
            ops.grouped_dgrad(gr, qw, rb, M)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            ops.grouped_dgrad(gr, qw, rb, M)
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1e3 / steps
        flop = 2 * M * n_ * k_
        tf = flop / (us * 1e-6) / 1e12
        dg[name] = {"avg_launch_us": round(us, 1), "flop_per_launch": flop, "achieved": round(tf, 1),
                    "unit": "TFLOP/s", "peak": BF16_PEAK_TFLOPS, "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
    e4b.disable_fast_train(mod)
    return {"workload": f"1 OLMoE-geometry layer, {tokens} tokens x top-{k}, ExpertsLoRA r={rank} fp32 adapters, "
                        "forward + backward (dL/dx and every adapter gradient)",
            "fused_ms": round(fused_ms, 3), "reference_loop_ms": round(ref_ms, 3),
            "speedup_vs_reference_loop": round(ref_ms / fused_ms, 2),
            "reference": "the module's reference forward (per-expert dequantize + linear loop, torch autograd) on "
                         f"the same GPU, {ref_steps} steps",
            "dgrad": dg}


def cpu_baseline(mod, cfg, budget_s=20.0):
    """The reference per-expert loop (the oracle's torch-CPU restatement of ExpertsNbit.forward)
    on the host cores, one OLMoE layer at batch 1, same weights and inputs."""
    import torch

    from oracle import moe as omoe

    # the box's CPU share (OMP_NUM_THREADS), not os.cpu_count() of the whole host
    threads = torch.get_num_threads()
    packed1, absmax1 = mod.gate_up_proj.cpu(), mod.gate_up_absmax.cpu()
    packed2, absmax2 = mod.down_proj.cpu(), mod.down_absmax.cpu()
    code = mod.code.cpu()
    n1, k1 = mod._gate_up_shape
    n2, k2 = mod._down_shape
    x, idx, w = make_inputs(cfg, 1, seed=1000 + 100 + 0)
    x, idx, w = x.cpu(), idx.cpu(), w.cpu()

    def w1(e, dt):
        return omoe.dequant_torch_expert(packed1[e], absmax1[e], code, n1, k1, dt)

    def w2(e, dt):
        return omoe.dequant_torch_expert(packed2[e], absmax2[e], code, n2, k2, dt)

    def run():
        return omoe.reference_loop(x, idx, w, w1, w2, cfg["E"], compute_dtype=torch.bfloat16)

    for _ in range(3):
        run()
    times = []
    t_begin = time.perf_counter()
    while len(times) < 10 or (time.perf_counter() - t_begin < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_begin > budget_s and len(times) >= 3:
            break
    med = statistics.median(times)
    gu_b, dn_b = nf4_expert_bytes(cfg["H"], cfg["I"])
    nbytes = cfg["k"] * (gu_b + dn_b)
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "us_per_layer": round(med * 1e6, 1),
        "sample": f"1 OLMoE layer (E=64, H=2048, I=1024, top-8), batch 1, {len(times)} timed reps after 3 "
                  "warm-ups, median; torch-CPU restatement of ExpertsNbit.forward with the pure-torch NF4 "
                  "dequant (bitsandbytes' CPU dequant is not installed)",
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip configs[2] (Qwen3 double-quant decode) and "
                    "configs[4] (gpt-oss MXFP4)")
    ap.add_argument("--kernel-only", action="store_true", help="only the dominant-kernel loop (for profiling)")
    ap.add_argument("--prefill-only", action="store_true", help="only the configs[3] prefill (for profiling)")
    ap.add_argument("--train-only", action="store_true", help="only the training-lane leg (for profiling)")
    ap.add_argument("--lora-prefill-only", action="store_true",
                    help="only the 4096-token ExpertsLoRA layer legs, rank 16 fp32 and rank 64 bf16 (for profiling)")
    ap.add_argument("--gptoss-only", action="store_true",
                    help="only the configs[4] gpt-oss MXFP4 legs, batches 1 and 2048 (for profiling)")
    ap.add_argument("--qwen-decode-only", action="store_true",
                    help="only the configs[2] Qwen3 double-quant decode legs, batches 1, 32, 256 (for profiling)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="for counter runs: the dominant kernel eagerly once per layer, then a 256 MiB "
                         "device copy whose counter reading calibrates bytes per counted KiB")
    ap.add_argument("--pmc-copy", action="store_true",
                    help="with --prefill-only: the 256 MiB calibration copy after the prefill (counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import experts4bit_qlora_amd as e4b
    from experts4bit_qlora_amd import _native as N

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    N.lib()  # fail loudly if the kernel library is missing
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_bench(args.steps, args.warmup)}), flush=True)
        if args.pmc_copy:
            calibration_copy()
        return
    if args.lora_prefill_only:
        cfg = OLMOE
        base = make_layer(cfg, seed=1000 + 100)
        assert e4b.enable_fast(base) == 1
        res = {f"r{r}_{str(dt).replace('torch.', '')}": lora_prefill_bench(base, cfg, args.steps, args.warmup, 1000 + 100,
                                                                          r, dt)
               for r, dt in ((16, torch.float32), (64, torch.bfloat16))}
        print(json.dumps({"lora_prefill": res}), flush=True)
        return
    if args.train_only:
        print(json.dumps({"train": train_bench(args.steps, args.warmup)}), flush=True)
        return
    if args.gptoss_only:
        print(json.dumps({"gptoss": gptoss_benches(args.steps, args.warmup)}), flush=True)
        return
    if args.qwen_decode_only:
        print(json.dumps({"qwen3_decode": qwen3_decode_benches(args.steps, args.warmup)}), flush=True)
        return
    cfg = OLMOE
    log("building 16 OLMoE-geometry NF4 layers")
    mods = [make_layer(cfg, seed=1000 + 100 + l) for l in range(cfg["layers"])]
    for m in mods:
        assert e4b.enable_fast(m) == 1
    torch.cuda.synchronize()

    if args.pmc_pass:
        pmc_pass(mods, cfg, seed0=1000 + 100)
        return

    log("dominant kernel roofline (gate_up GEMV, bs=1)")
    roof = dominant_kernel_roofline(mods, cfg, args.steps, args.warmup, seed0=1000 + 100)
    if args.kernel_only:
        print(json.dumps({"roofline": roof}))
        return

    decode = {}
    for T in (1, 8, 64):
        log(f"decode step, batch {T}")
        decode[T] = decode_bench(mods, cfg, T, args.steps, args.warmup, seed0=1000 + 100)
    main_line = decode[1]
    log("decode step, batch 1, experts rotated between replays")
    decode[1]["rotating_experts"] = rotating_decode_bench(mods, cfg, args.steps, args.warmup, seed0=1000 + 100)
    log("ExpertsLoRA decode step, batches 1 and 8; one layer at 4096 tokens")
    lora = lora_bench(mods, cfg, args.steps, args.warmup, 1000 + 100, decode)

    prefill = None
    if not args.no_prefill:
        log("Qwen3 4096-token Zipf prefill")
        prefill = prefill_bench(args.steps, args.warmup)

    extra = None
    train = None
    if not args.no_extra:
        log("configs[2] Qwen3 double-quant decode and configs[4] gpt-oss MXFP4")
        extra = extra_benches(args.steps, args.warmup)
        log("training lane: ExpertsLoRA forward + backward, 2048 tokens")
        train = train_bench(args.steps, args.warmup)

    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (reference per-expert loop on the host)")
        cpu = cpu_baseline(mods[0], cfg)

    line = {
        "metric": METRIC,
        "value": round(main_line["hbm_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_line["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "OLMoE-1B-7B geometry, 16 stacked MoE layers, decode batch 1 (configs[1])",
            "experts": cfg["E"], "hidden": cfg["H"], "moe_intermediate": cfg["I"], "top_k": cfg["k"],
            "layers": cfg["layers"], "quant": "NF4, blocksize 64, fp32 absmax", "global_batch": 1,
            "parallelism": "single GPU",
        },
        "us_per_layer": round(main_line["us_per_layer"], 3),
        "tok_per_s": round(main_line["tok_per_s"], 1),
        "hbm_frac": round(main_line["hbm_frac"], 4),
        "decode": {f"bs{T}": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}
                   for T, d in decode.items()},
        "roofline": roof,
        "cpu_baseline": cpu,
        "lora_decode": lora,
    }
    if prefill is not None:
        line["prefill"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in prefill.items()}
    if extra is not None:
        line["extra"] = extra
    if train is not None:
        line["train"] = train
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
